// MoE block prologue: residual add, post-attention RMSNorm and router logits.
//
// Replaces, for one chunk of tokens:
//   MoeAll2AllBlock.all2all_chunk_routing_compute (generation/blocks/moe/moe_all2all.py:329-336):
//     residual = _add_to_residual(residual, hidden_states)   (generation/utils/compute_utils.py:14)
//     normed   = post_attention_layernorm(residual)
//   _rmsnorm (generation/modules/rmsnorm/base_rmsnorm.py:6-12):
//     t = r.float(); t = t * rsqrt(mean(t^2) + eps); normed = weight * t.to(bf16)
//   the router gate, F.linear(normed, gate_w) (generation/modules/linear/base_linear.py:28-36; in bf16 for
//   the Qwen3 / Mixtral gates, whose logits are therefore rounded to bf16) or
//   F.linear(normed.float(), gate_w.float()) (DeepseekV3MoEGate, models/deepseek_v3/
//   modeling_deepseek_v3.py:155-157; fp32 logits).
//
// One wave per token row: the row lives in the wave's registers (16-byte vectors, at most 16
// per lane: H <= 8192), the mean of squares is a wave reduction, and the residual and normed
// rows are written once.  Small routers (E <= 32, gate <= 128 KiB) are dotted in the same
// pass against the gate weights staged in LDS once per workgroup (a persistent grid of
// workgroups, each wave taking every n-th row); larger routers (E a multiple of 64) take the
// normed rows through the grouped MFMA GEMM as one dense segment.
#include "common.h"
#include "kernels.h"

namespace eimoe {

namespace {

constexpr int kProWaves = 4;
constexpr int kProThreads = 64 * kProWaves;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

__device__ __forceinline__ bf16x2_t as_bf16x2(uint32_t w) { return __builtin_bit_cast(bf16x2_t, w); }

__device__ __forceinline__ float lo_f32(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_f32(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Sums each of the EP values over the wave, halving the set at each exchange: EP/2 + EP/4 +
// ... + 1 exchanges until a lane holds one value, then plain butterflies (EP + 5 - log2 EP
// exchanges in all, against 6 EP for one wave sum per value).  Lane l returns the total of
// d[l / (64 / EP)].
template <int EP>
__device__ __forceinline__ float wave_sum_scatter(float (&d)[EP], int lane) {
  int n = EP;
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    if (n > 1) {
      const bool up = (lane & m) != 0;
      const int h = n / 2;
#pragma unroll
      for (int i = 0; i < h; ++i) {
        const float send = up ? d[i] : d[h + i];
        const float keep = up ? d[h + i] : d[i];
        d[i] = keep + __shfl_xor(send, m, 64);
      }
      n = h;
    } else {
      d[0] += __shfl_xor(d[0], m, 64);
    }
  }
  return d[0];
}

// VPL: 16-byte vectors (8 bf16) per lane.  EP > 0 fuses the router dots (gate staged in LDS)
// for up to EP experts (a power of two); EP == 0 leaves the router to the GEMM.
// PF: the next row's loads are issued before the current row is processed.
// seg_off (the router GEMM's one segment, [0, T]) is written by the first thread when given.
template <int VPL, int EP, bool PF>
__global__ __launch_bounds__(kProThreads) void prologue_kernel(
    const uint16_t* __restrict__ hidden, const uint16_t* __restrict__ residual, const uint16_t* __restrict__ norm_w,
    float eps, const uint16_t* __restrict__ gate_w, int T, int H, int E, int logits_bf16,
    uint16_t* __restrict__ res_out, uint16_t* __restrict__ normed, float* __restrict__ logits,
    int32_t* __restrict__ seg_off) {
  constexpr bool EF = EP > 0;
  extern __shared__ uint4 s_gate[];   // [E][H/8] when EF
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int nvec = H / 8;
  if (seg_off != nullptr && blockIdx.x == 0 && threadIdx.x == 0) {
    seg_off[0] = 0;
    seg_off[1] = T;
  }
  if constexpr (EF) {
    const uint4* g = reinterpret_cast<const uint4*>(gate_w);
    for (int i = threadIdx.x; i < E * nvec; i += kProThreads) s_gate[i] = g[i];
    __syncthreads();
  }
  const uint4* wr = reinterpret_cast<const uint4*>(norm_w);
  uint4 wv8[EF ? VPL : 1];   // RMSNorm weight, kept across rows when the grid is persistent
  if constexpr (EF) {
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      const int v = j * 64 + lane;
      wv8[j] = v < nvec ? wr[v] : make_uint4(0u, 0u, 0u, 0u);
    }
  }
  const int stride = gridDim.x * kProWaves;
  auto load_row = [&](int t, uint4 (&a)[VPL], uint4 (&b)[VPL]) {
    const uint4* hr = reinterpret_cast<const uint4*>(hidden + static_cast<long long>(t) * H);
    const uint4* rr = reinterpret_cast<const uint4*>(residual + static_cast<long long>(t) * H);
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      const int v = j * 64 + lane;
      a[j] = v < nvec ? hr[v] : make_uint4(0u, 0u, 0u, 0u);
      b[j] = v < nvec ? rr[v] : make_uint4(0u, 0u, 0u, 0u);
    }
  };
  uint4 ha[VPL], rb[VPL], hn[PF ? VPL : 1], rn[PF ? VPL : 1];
  int t = blockIdx.x * kProWaves + wv;
  if constexpr (PF) {
    if (t < T) load_row(t, ha, rb);
  }
  for (; t < T; t += stride) {
    if constexpr (PF) {
      if (t + stride < T) load_row(t + stride, hn, rn);
    } else {
      load_row(t, ha, rb);
    }
    // r = bf16(residual + hidden), held in ha from here on
    uint4* ro = reinterpret_cast<uint4*>(res_out + static_cast<long long>(t) * H);
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      const int v = j * 64 + lane;
      uint32_t aw[4] = {ha[j].x, ha[j].y, ha[j].z, ha[j].w};
      const uint32_t bw[4] = {rb[j].x, rb[j].y, rb[j].z, rb[j].w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        aw[q] = pack_bf16x2(lo_f32(bw[q]) + lo_f32(aw[q]), hi_f32(bw[q]) + hi_f32(aw[q]));
        const float rl = lo_f32(aw[q]), rh = hi_f32(aw[q]);
        ss += rl * rl + rh * rh;
      }
      ha[j] = make_uint4(aw[0], aw[1], aw[2], aw[3]);
      if (v < nvec) ro[v] = ha[j];
    }
    const float rs = 1.0f / sqrtf(wave_sum(ss) / static_cast<float>(H) + eps);
    // normed = bf16(weight * bf16(r * rs)), held in ha from here on
    uint4* no = reinterpret_cast<uint4*>(normed + static_cast<long long>(t) * H);
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      const int v = j * 64 + lane;
      uint4 w8;
      if constexpr (EF) w8 = wv8[j];
      else w8 = v < nvec ? wr[v] : make_uint4(0u, 0u, 0u, 0u);
      uint32_t rw[4] = {ha[j].x, ha[j].y, ha[j].z, ha[j].w};
      const uint32_t ww[4] = {w8.x, w8.y, w8.z, w8.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t tq = pack_bf16x2(lo_f32(rw[q]) * rs, hi_f32(rw[q]) * rs);
        rw[q] = pack_bf16x2(lo_f32(ww[q]) * lo_f32(tq), hi_f32(ww[q]) * hi_f32(tq));
      }
      ha[j] = make_uint4(rw[0], rw[1], rw[2], rw[3]);
      if (v < nvec) no[v] = ha[j];
    }
    if constexpr (EF) {
      // router dots against the staged gate rows, two bf16 products per v_dot2 (fp32 sums)
      float d[EP];
#pragma unroll
      for (int e = 0; e < EP; ++e) {
        d[e] = 0.f;
        if (e < E) {
#pragma unroll
          for (int j = 0; j < VPL; ++j) {
            const int v = j * 64 + lane;
            if (v < nvec) {
              const uint4 gq = s_gate[e * nvec + v];
              d[e] = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(ha[j].x), as_bf16x2(gq.x), d[e], false);
              d[e] = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(ha[j].y), as_bf16x2(gq.y), d[e], false);
              d[e] = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(ha[j].z), as_bf16x2(gq.z), d[e], false);
              d[e] = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(ha[j].w), as_bf16x2(gq.w), d[e], false);
            }
          }
        }
      }
      const float tot = wave_sum_scatter<EP>(d, lane);
      constexpr int kSpan = 64 / EP;   // lanes holding each expert's total
      const int e = lane / kSpan;
      if (lane % kSpan == 0 && e < E)
        logits[static_cast<long long>(t) * E + e] = logits_bf16 ? bf16_to_f32(f32_to_bf16(tot)) : tot;
    }
    if constexpr (PF) {
#pragma unroll
      for (int j = 0; j < VPL; ++j) {
        ha[j] = hn[j];
        rb[j] = rn[j];
      }
    }
  }
}

// logits = sum of the K-split planes in order (and rounded to bf16 values when asked)
// (in place when n_split == 1 and planes == out)
__global__ void sum_planes_kernel(const float* planes, int n_split, long long n, int round, float* out) {
  for (long long i = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x; i < n;
       i += static_cast<long long>(gridDim.x) * 256) {
    float v = planes[i];
    for (int s = 1; s < n_split; ++s) v += planes[static_cast<long long>(s) * n + i];
    out[i] = round ? bf16_to_f32(f32_to_bf16(v)) : v;
  }
}

template <int VPL, int EP, bool PF>
hipError_t launch_prologue_v(const void* hidden, const void* residual, const void* norm_w, float eps,
                             const void* gate_w, int T, int H, int E, int logits_bf16, void* res_out, void* normed,
                             float* logits, int32_t* seg_off, hipStream_t s) {
  const size_t lds = EP ? static_cast<size_t>(E) * H * 2 : 0;
  if (lds > 64 * 1024) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(prologue_kernel<VPL, EP, PF>),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    if (e != hipSuccess) return e;
  }
  // fused: a persistent grid amortises staging the gate (2 workgroups per CU); else a wave per row
  long long grid = (T + kProWaves - 1) / kProWaves;
  if (EP && grid > 2ll * kNumCu) grid = 2ll * kNumCu;
  if (grid < 1) grid = 1;
  hipLaunchKernelGGL((prologue_kernel<VPL, EP, PF>), dim3(static_cast<unsigned>(grid)), dim3(kProThreads), lds, s,
                     static_cast<const uint16_t*>(hidden), static_cast<const uint16_t*>(residual),
                     static_cast<const uint16_t*>(norm_w), eps, static_cast<const uint16_t*>(gate_w), T, H, E,
                     logits_bf16, static_cast<uint16_t*>(res_out), static_cast<uint16_t*>(normed), logits, seg_off);
  return hipGetLastError();
}

// The fused kernel loops over rows and prefetches the next one where the registers allow it.
template <int EP>
hipError_t launch_prologue_e(int vpl, const void* hidden, const void* residual, const void* norm_w, float eps,
                             const void* gate_w, int T, int H, int E, int logits_bf16, void* res_out, void* normed,
                             float* logits, int32_t* seg_off, hipStream_t s) {
#define EIMOE_PRO(V, PF) \
  return launch_prologue_v<V, EP, PF>(hidden, residual, norm_w, eps, gate_w, T, H, E, logits_bf16, res_out, normed, \
                                      logits, seg_off, s)
  if (vpl <= 1) EIMOE_PRO(1, (EP > 0));
  if (vpl <= 2) EIMOE_PRO(2, (EP > 0));
  if (vpl <= 4) EIMOE_PRO(4, (EP > 0));
  if (vpl <= 8) EIMOE_PRO(8, (EP > 0 && EP <= 16));
  EIMOE_PRO(16, false);
#undef EIMOE_PRO
}

hipError_t launch_prologue_fused(int vpl, const void* hidden, const void* residual, const void* norm_w, float eps,
                                 const void* gate_w, int T, int H, int E, int logits_bf16, void* res_out,
                                 void* normed, float* logits, hipStream_t s) {
#define EIMOE_PRO_E(P)                                                                                              \
  return launch_prologue_e<P>(vpl, hidden, residual, norm_w, eps, gate_w, T, H, E, logits_bf16, res_out, normed, \
                              logits, nullptr, s)
  if (E <= 1) EIMOE_PRO_E(1);
  if (E <= 2) EIMOE_PRO_E(2);
  if (E <= 4) EIMOE_PRO_E(4);
  if (E <= 8) EIMOE_PRO_E(8);
  if (E <= 16) EIMOE_PRO_E(16);
  EIMOE_PRO_E(32);
#undef EIMOE_PRO_E
}

}  // namespace

bool prologue_fused_router(int H, int E) { return E <= kPrologueFusedMaxE && 2ll * E * H <= kPrologueFusedMaxGate; }

// Router GEMM shape for the non-fused path: 128x128 tiles from 512 rows on when E allows (else
// 16x64), and the K dimension (H) split into fp32 planes, each at least 512 deep, until there
// are two tiles per CU (4096 x 256 x 7168: 64 tiles, 8 planes: 24 us against 28 us with 4 and
// 73 us unsplit, measured on MI355X).
PrologueGemm prologue_router_gemm(int T, int H, int E) {
  PrologueGemm g{};
  const bool m_tile = E % 128 == 0 && T >= 512;
  g.tile = m_tile ? kTileM : kTileXS;
  const long long tiles = ((T + (m_tile ? 127 : 15)) / (m_tile ? 128 : 16)) * static_cast<long long>(E / (m_tile ? 128 : 64));
  g.k_split = 1;
  while (g.k_split < kPrologueMaxSplit && tiles * g.k_split < 2ll * kNumCu && H % (128 * g.k_split) == 0 &&
         H / (2 * g.k_split) >= 512)
    g.k_split *= 2;
  return g;
}

size_t prologue_workspace_bytes(int T, int H, int E) {
  if (T < 0 || H < 1 || E < 1 || prologue_fused_router(H, E)) return 0;
  const PrologueGemm g = prologue_router_gemm(T, H, E);
  return 256 + (g.k_split > 1 ? static_cast<size_t>(g.k_split) * T * E * sizeof(float) : 0);
}

hipError_t launch_moe_prologue(const void* hidden, const void* residual, const void* norm_w, float eps,
                               const void* gate_w, int T, int H, int E, int logits_bf16, void* res_out, void* normed,
                               float* logits, void* workspace, hipStream_t s) {
  const int vpl = (H / 8 + 63) / 64;
  if (prologue_fused_router(H, E))
    return launch_prologue_fused(vpl, hidden, residual, norm_w, eps, gate_w, T, H, E, logits_bf16, res_out, normed,
                                 logits, s);
  // router GEMM: the T normed rows as one segment against the [E, H] gate, fp32 out
  int32_t* seg_off = static_cast<int32_t*>(workspace);
  hipError_t e = launch_prologue_e<0>(vpl, hidden, residual, norm_w, eps, gate_w, T, H, E, logits_bf16, res_out,
                                          normed, logits, seg_off, s);
  if (e != hipSuccess) return e;
  const PrologueGemm g = prologue_router_gemm(T, H, E);
  float* planes = g.k_split > 1 ? reinterpret_cast<float*>(static_cast<char*>(workspace) + 256) : logits;
  GemmArgs p{};
  p.a = normed;
  p.lda = H;
  p.b = gate_w;
  p.b_estride = static_cast<long long>(E) * H;
  p.ldb = H;
  p.nb_rows = E;
  p.N = E;
  p.K = H / g.k_split;
  p.seg_off = seg_off;
  p.S = 1;
  p.e_mod = 1;
  p.c = planes;
  p.ldc = E;
  p.c_split_stride = static_cast<long long>(T) * E;
  p.k_split = g.k_split;
  p.max_rows = T;
  p.a_rows_cap = T;
  if ((e = launch_grouped_gemm(p, kEpiStoreF32, false, false, T, g.tile, s)) != hipSuccess) return e;
  if (g.k_split > 1 || logits_bf16) {
    const long long n = static_cast<long long>(T) * E;
    long long blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(sum_planes_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, planes, g.k_split, n,
                       logits_bf16, logits);
    e = hipGetLastError();
  }
  return e;
}

}  // namespace eimoe
