// MoE block prologue: residual add, post-attention RMSNorm and router logits.
//
// Replaces, for one chunk of tokens:
//   MoeAll2AllBlock.all2all_chunk_routing_compute (generation/blocks/moe/moe_all2all.py:329-336):
//     residual = _add_to_residual(residual, hidden_states)   (generation/utils/compute_utils.py:14)
//     normed   = post_attention_layernorm(residual)
//   _rmsnorm (generation/modules/norms/base_rmsnorm.py:6-12):
//     t = r.float(); t = t * rsqrt(mean(t^2) + eps); normed = weight * t.to(bf16)
//   the router gate, F.linear(normed, gate_w) (modules/linears/base_linear.py:28-36; in bf16 for
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

// VPL: 16-byte vectors (8 bf16) per lane; EF: fuse the router dots (gate staged in LDS).
template <int VPL, bool EF>
__global__ __launch_bounds__(kProThreads) void prologue_kernel(
    const uint16_t* __restrict__ hidden, const uint16_t* __restrict__ residual, const uint16_t* __restrict__ norm_w,
    float eps, const uint16_t* __restrict__ gate_w, int T, int H, int E, int logits_bf16,
    uint16_t* __restrict__ res_out, uint16_t* __restrict__ normed, float* __restrict__ logits) {
  extern __shared__ uint4 s_gate[];   // [E][H/8] when EF
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int nvec = H / 8;
  if constexpr (EF) {
    const uint4* g = reinterpret_cast<const uint4*>(gate_w);
    for (int i = threadIdx.x; i < E * nvec; i += kProThreads) s_gate[i] = g[i];
    __syncthreads();
  }
  uint4 wv8[VPL];   // RMSNorm weight, the same for every row
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int v = j * 64 + lane;
    wv8[j] = v < nvec ? reinterpret_cast<const uint4*>(norm_w)[v] : make_uint4(0u, 0u, 0u, 0u);
  }
  for (int t = blockIdx.x * kProWaves + wv; t < T; t += gridDim.x * kProWaves) {
    const uint4* hr = reinterpret_cast<const uint4*>(hidden + static_cast<long long>(t) * H);
    const uint4* rr = reinterpret_cast<const uint4*>(residual + static_cast<long long>(t) * H);
    uint4* ro = reinterpret_cast<uint4*>(res_out + static_cast<long long>(t) * H);
    uint4 r8[VPL];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      const int v = j * 64 + lane;
      r8[j] = make_uint4(0u, 0u, 0u, 0u);
      if (v < nvec) {
        const uint4 a = hr[v], b = rr[v];
        const uint32_t aw[4] = {a.x, a.y, a.z, a.w}, bw[4] = {b.x, b.y, b.z, b.w};
        uint32_t o[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float lo = bf16_to_f32(static_cast<uint16_t>(bw[q])) + bf16_to_f32(static_cast<uint16_t>(aw[q]));
          const float hi = bf16_to_f32(static_cast<uint16_t>(bw[q] >> 16)) + bf16_to_f32(static_cast<uint16_t>(aw[q] >> 16));
          o[q] = pack_bf16x2(lo, hi);
          const float rl = bf16_to_f32(static_cast<uint16_t>(o[q])), rh = bf16_to_f32(static_cast<uint16_t>(o[q] >> 16));
          ss += rl * rl + rh * rh;
        }
        r8[j] = make_uint4(o[0], o[1], o[2], o[3]);
        ro[v] = r8[j];
      }
    }
    const float rs = 1.0f / sqrtf(wave_sum(ss) / static_cast<float>(H) + eps);
    uint4* no = reinterpret_cast<uint4*>(normed + static_cast<long long>(t) * H);
    // normed = bf16(weight * bf16(r * rs)); router dots against the staged gate rows
    uint4 n8[VPL];
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      const int v = j * 64 + lane;
      const uint32_t rw[4] = {r8[j].x, r8[j].y, r8[j].z, r8[j].w};
      const uint32_t ww[4] = {wv8[j].x, wv8[j].y, wv8[j].z, wv8[j].w};
      uint32_t o[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float tl = bf16_to_f32(f32_to_bf16(bf16_to_f32(static_cast<uint16_t>(rw[q])) * rs));
        const float th = bf16_to_f32(f32_to_bf16(bf16_to_f32(static_cast<uint16_t>(rw[q] >> 16)) * rs));
        o[q] = pack_bf16x2(bf16_to_f32(static_cast<uint16_t>(ww[q])) * tl,
                           bf16_to_f32(static_cast<uint16_t>(ww[q] >> 16)) * th);
      }
      n8[j] = make_uint4(o[0], o[1], o[2], o[3]);
      if (v < nvec) no[v] = n8[j];
    }
    if constexpr (EF) {
      float mine = 0.f;
#pragma unroll 1
      for (int e = 0; e < E; ++e) {
        float d = 0.f;
#pragma unroll
        for (int j = 0; j < VPL; ++j) {
          const int v = j * 64 + lane;
          if (v < nvec) {
            const uint4 gq = s_gate[e * nvec + v];
            const uint32_t gw[4] = {gq.x, gq.y, gq.z, gq.w};
            const uint32_t nw[4] = {n8[j].x, n8[j].y, n8[j].z, n8[j].w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              d += bf16_to_f32(static_cast<uint16_t>(nw[q])) * bf16_to_f32(static_cast<uint16_t>(gw[q]));
              d += bf16_to_f32(static_cast<uint16_t>(nw[q] >> 16)) * bf16_to_f32(static_cast<uint16_t>(gw[q] >> 16));
            }
          }
        }
        d = wave_sum(d);
        if (lane == e) mine = d;
      }
      if (lane < E)
        logits[static_cast<long long>(t) * E + lane] = logits_bf16 ? bf16_to_f32(f32_to_bf16(mine)) : mine;
    }
  }
}

__global__ void round_bf16_kernel(float* __restrict__ x, long long n) {
  for (long long i = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x; i < n;
       i += static_cast<long long>(gridDim.x) * 256)
    x[i] = bf16_to_f32(f32_to_bf16(x[i]));
}

__global__ void one_segment_kernel(int32_t* off, int T) {
  if (threadIdx.x == 0) {
    off[0] = 0;
    off[1] = T;
  }
}

template <int VPL, bool EF>
hipError_t launch_prologue_v(const void* hidden, const void* residual, const void* norm_w, float eps,
                             const void* gate_w, int T, int H, int E, int logits_bf16, void* res_out, void* normed,
                             float* logits, hipStream_t s) {
  const size_t lds = EF ? static_cast<size_t>(E) * H * 2 : 0;
  if (lds > 64 * 1024) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(prologue_kernel<VPL, EF>),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    if (e != hipSuccess) return e;
  }
  // fused: a persistent grid amortises staging the gate (2 workgroups per CU); else a wave per row
  long long grid = (T + kProWaves - 1) / kProWaves;
  if (EF && grid > 2ll * kNumCu) grid = 2ll * kNumCu;
  if (grid < 1) grid = 1;
  hipLaunchKernelGGL((prologue_kernel<VPL, EF>), dim3(static_cast<unsigned>(grid)), dim3(kProThreads), lds, s,
                     static_cast<const uint16_t*>(hidden), static_cast<const uint16_t*>(residual),
                     static_cast<const uint16_t*>(norm_w), eps, static_cast<const uint16_t*>(gate_w), T, H, E,
                     logits_bf16, static_cast<uint16_t*>(res_out), static_cast<uint16_t*>(normed), logits);
  return hipGetLastError();
}

template <bool EF>
hipError_t launch_prologue_e(int vpl, const void* hidden, const void* residual, const void* norm_w, float eps,
                             const void* gate_w, int T, int H, int E, int logits_bf16, void* res_out, void* normed,
                             float* logits, hipStream_t s) {
#define EIMOE_PRO(V) \
  return launch_prologue_v<V, EF>(hidden, residual, norm_w, eps, gate_w, T, H, E, logits_bf16, res_out, normed, \
                                  logits, s)
  if (vpl <= 1) EIMOE_PRO(1);
  if (vpl <= 2) EIMOE_PRO(2);
  if (vpl <= 4) EIMOE_PRO(4);
  if (vpl <= 8) EIMOE_PRO(8);
  EIMOE_PRO(16);
#undef EIMOE_PRO
}

}  // namespace

bool prologue_fused_router(int H, int E) { return E <= kPrologueFusedMaxE && 2ll * E * H <= kPrologueFusedMaxGate; }

hipError_t launch_moe_prologue(const void* hidden, const void* residual, const void* norm_w, float eps,
                               const void* gate_w, int T, int H, int E, int logits_bf16, void* res_out, void* normed,
                               float* logits, int32_t* seg_off, hipStream_t s) {
  const int vpl = (H / 8 + 63) / 64;
  if (prologue_fused_router(H, E))
    return launch_prologue_e<true>(vpl, hidden, residual, norm_w, eps, gate_w, T, H, E, logits_bf16, res_out, normed,
                                   logits, s);
  hipError_t e = launch_prologue_e<false>(vpl, hidden, residual, norm_w, eps, gate_w, T, H, E, logits_bf16, res_out,
                                          normed, logits, s);
  if (e != hipSuccess) return e;
  // router GEMM: the T normed rows as one segment against the [E, H] gate, fp32 out
  hipLaunchKernelGGL(one_segment_kernel, dim3(1), dim3(64), 0, s, seg_off, T);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  GemmArgs p{};
  p.a = normed;
  p.lda = H;
  p.b = gate_w;
  p.b_estride = static_cast<long long>(E) * H;
  p.ldb = H;
  p.nb_rows = E;
  p.N = E;
  p.K = H;
  p.seg_off = seg_off;
  p.S = 1;
  p.e_mod = 1;
  p.c = logits;
  p.ldc = E;
  p.k_split = 1;
  p.max_rows = T;
  p.a_rows_cap = T;
  if ((e = launch_grouped_gemm(p, kEpiStoreF32, false, false, T, kTileAuto, s)) != hipSuccess) return e;
  if (logits_bf16) {
    const long long n = static_cast<long long>(T) * E;
    long long blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(round_bf16_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, logits, n);
    e = hipGetLastError();
  }
  return e;
}

}  // namespace eimoe
