// Router: softmax -> top-k -> optional renormalisation, one token per lane group.
//
// Replaces Qwen3MoeSparseMoeBlock._routing (easyinfra/models/qwen3_moe/
// modeling_qwen3_moe.py:255-266): softmax(logits, fp32), topk(k), w /= sum(w).
// Selection is by logit (softmax is monotonic), ties to the lower expert id, so
// the ids do not depend on exp rounding and are bit-exact against the CPU oracle.
// Weights: exp(l - max) / sum over the k picks (renormalise) or over all experts.
//
// Layout: a wave holds 64/LPT tokens; lane group of LPT lanes owns one token row,
// each lane VPL logits (experts li, li+LPT, ...).  Argmax rounds are all-reduces inside
// the lane group (DPP lane permutes up to 16 lanes).
#include "kernels.h"
#include "routing.h"

namespace eimoe {

template <int LPT, int VPL, int KMAX>
__global__ __launch_bounds__(256) void router_topk_kernel(const float* __restrict__ logits, int T, int E, int k,
                                                          int renorm, int32_t* __restrict__ ids,
                                                          float* __restrict__ wts) {
  route_rows<LPT, VPL, KMAX, kLdsNone>(logits, T, E, k, renorm, ids, wts, nullptr,
                                       (blockIdx.x * blockDim.x + threadIdx.x) >> 6, (gridDim.x * blockDim.x) >> 6);
}

// The router fused with the many-workgroup align's first pass: workgroup b routes tokens
// [b*TB, (b+1)*TB) (TB = WPB waves x 64/LPT tokens, one routing step per wave), which are the
// flat ids [b*TB*k, (b+1)*TB*k): align chunk b, whose per-expert counts it writes to
// hist_g[b][n_loc] (LDS integer atomics: the counts do not depend on their order).
template <int LPT, int VPL, int KMAX, int WPB>
__global__ __launch_bounds__(64 * WPB) void router_hist_kernel(const float* __restrict__ logits, int T, int E, int k,
                                                               int renorm, int32_t* __restrict__ ids,
                                                               float* __restrict__ wts, int e_lo, int n_loc,
                                                               int32_t* __restrict__ hist_g) {
  extern __shared__ int s_hist[];   // [n_loc]
  for (int i = threadIdx.x; i < n_loc; i += 64 * WPB) s_hist[i] = 0;
  __syncthreads();
  route_rows<LPT, VPL, KMAX, kLdsHist>(logits, T, E, k, renorm, ids, wts, s_hist,
                                       blockIdx.x * WPB + (threadIdx.x >> 6), gridDim.x * WPB, e_lo, n_loc);
  __syncthreads();
  for (int e = threadIdx.x; e < n_loc; e += 64 * WPB)
    hist_g[static_cast<long long>(blockIdx.x) * n_loc + e] = s_hist[e];
}

template <int LPT, int VPL>
static hipError_t launch_router_lv(const float* logits, int T, int E, int k, int renorm, int32_t* ids, float* w,
                                   hipStream_t s) {
  constexpr int TPW = 64 / LPT;
  const int waves = (T + TPW - 1) / TPW;
  int blocks = (waves + 3) / 4;
  if (blocks > 4096) blocks = 4096;
  if (blocks < 1) blocks = 1;
  if (k <= 8)
    hipLaunchKernelGGL((router_topk_kernel<LPT, VPL, 8>), dim3(blocks), dim3(256), 0, s, logits, T, E, k, renorm, ids, w);
  else
    hipLaunchKernelGGL((router_topk_kernel<LPT, VPL, 32>), dim3(blocks), dim3(256), 0, s, logits, T, E, k, renorm, ids, w);
  return hipGetLastError();
}

template <int LPT, int VPL>
static hipError_t launch_router_hist_lv(const float* logits, int T, int E, int k, int renorm, int32_t* ids, float* w,
                                        int e_lo, int n_loc, int blocks, int wpb, int32_t* hist, hipStream_t s) {
  const size_t lds = static_cast<size_t>(n_loc) * sizeof(int);
  if (wpb == 8) {
    if (k <= 8)
      hipLaunchKernelGGL((router_hist_kernel<LPT, VPL, 8, 8>), dim3(blocks), dim3(512), lds, s, logits, T, E, k,
                         renorm, ids, w, e_lo, n_loc, hist);
    else
      hipLaunchKernelGGL((router_hist_kernel<LPT, VPL, 32, 8>), dim3(blocks), dim3(512), lds, s, logits, T, E, k,
                         renorm, ids, w, e_lo, n_loc, hist);
  } else if (k <= 8) {
    hipLaunchKernelGGL((router_hist_kernel<LPT, VPL, 8, 4>), dim3(blocks), dim3(256), lds, s, logits, T, E, k, renorm,
                       ids, w, e_lo, n_loc, hist);
  } else {
    hipLaunchKernelGGL((router_hist_kernel<LPT, VPL, 32, 4>), dim3(blocks), dim3(256), lds, s, logits, T, E, k, renorm,
                       ids, w, e_lo, n_loc, hist);
  }
  return hipGetLastError();
}

// Lane group of the router for E experts (as launch_router_topk picks it).
static int topk_lanes(int E) { return E <= 8 ? 8 : E <= 128 ? 16 : E <= 256 ? 32 : 64; }

struct RouteHistPlan {
  int blocks;   // 0: not used
  int chunk;    // flat ids per workgroup
  int wpb;      // waves per workgroup (4 or 8)
};

// Each placing workgroup sums the whole chunk-count matrix, so the matrix is kept small:
// measured against the router + two-pass align (one box, cache-cold layers): Qwen3-30B-A3B
// 32-expert share at 256 and 600 tokens (512 and 1216 cells) 89.0 -> 86.7 and 105.9 -> 101.7
// us, at 2048 tokens (4096 cells) equal, DeepSeek-V2-Lite 4096 tokens (16384 cells) 611 -> 620 us.
constexpr long long kRouteHistMaxCells = 2048;

// Workgroups of 4 waves, or of 8 where that keeps the matrix within bounds (the Qwen3-30B-A3B
// share at 1536 / 2048 tokens: 1536 / 2048 cells of 8-wave workgroups instead of the router, the
// histogram launch and the place launch; layers 125.7 / 133.0 -> 122.8 / 130.3 us cold, one box).
static RouteHistPlan route_hist_plan(int T, int E, int k, int n_loc) {
  RouteHistPlan r{0, 0, 0};
  for (int wpb = 4; wpb <= 8; wpb *= 2) {
    const int tb = wpb * (64 / topk_lanes(E));   // tokens per workgroup: one routing step per wave
    const long long blocks = (static_cast<long long>(T) + tb - 1) / tb;
    if (blocks < 2) return r;
    if (blocks * n_loc > kRouteHistMaxCells) continue;
    r.blocks = static_cast<int>(blocks);
    r.chunk = tb * k;
    r.wpb = wpb;
    return r;
  }
  return r;
}

static hipError_t launch_router_hist(const float* logits, int T, int E, int k, int renorm, int32_t* ids, float* w,
                                     int e_lo, int n_loc, int blocks, int wpb, int32_t* hist, hipStream_t s) {
#define EIMOE_RH(L, V) \
  return launch_router_hist_lv<L, V>(logits, T, E, k, renorm, ids, w, e_lo, n_loc, blocks, wpb, hist, s)
  if (E <= 8) EIMOE_RH(8, 1);
  if (E <= 16) EIMOE_RH(16, 1);
  if (E <= 32) EIMOE_RH(16, 2);
  if (E <= 64) EIMOE_RH(16, 4);
  if (E <= 128) EIMOE_RH(16, 8);
  if (E <= 256) EIMOE_RH(32, 8);
  EIMOE_RH(64, 8);
#undef EIMOE_RH
}

// Lane groups of 16 up to 128 experts: each selection round is a 4-step butterfly shared
// by 4 tokens of the wave (a 64-lane group would spend 6 steps on one token).
hipError_t launch_router_topk(const float* logits, int T, int E, int k, int renorm, int32_t* ids, float* w,
                              hipStream_t s) {
  if (E <= 8) return launch_router_lv<8, 1>(logits, T, E, k, renorm, ids, w, s);
  if (E <= 16) return launch_router_lv<16, 1>(logits, T, E, k, renorm, ids, w, s);
  if (E <= 32) return launch_router_lv<16, 2>(logits, T, E, k, renorm, ids, w, s);
  if (E <= 64) return launch_router_lv<16, 4>(logits, T, E, k, renorm, ids, w, s);
  if (E <= 128) return launch_router_lv<16, 8>(logits, T, E, k, renorm, ids, w, s);
  if (E <= 256) return launch_router_lv<32, 8>(logits, T, E, k, renorm, ids, w, s);
  return launch_router_lv<64, 8>(logits, T, E, k, renorm, ids, w, s);
}

// ---------------------------------------------------------------------------- grouped
// DeepSeek-V3 gate, "noaux_tc" (DeepseekV3MoEGate.forward, models/deepseek_v3/
// modeling_deepseek_v3.py:151-203), on precomputed fp32 logits:
//   s = sigmoid(logits); c = s + bias;
//   group score = sum of the top 2 of c inside each of n_group equal expert groups;
//   keep the topk_group best groups, c := 0 outside them (masked_fill 0.0, not -inf);
//   ids = top-k of c; w = s[ids]; w /= sum(w) + 1e-20 when renormalising (k > 1);
//   w *= scaling.
// Selection depends on how s rounds (the bias breaks the monotonicity that lets the
// softmax router compare logits), so s is computed in double and rounded once to fp32:
// the correctly rounded sigmoid, which the oracle computes the same way.  Ties go to the
// lower group / expert id; the picks come out in descending order of c.
// One wave per token (kGroupedWaves per workgroup); lane l holds experts l*VPL..+VPL-1.
// Group scores and group selection go through LDS, so any n_group dividing E works.
constexpr int kGroupedWaves = 4;
constexpr int kGroupedMaxE = 512;

__device__ __forceinline__ float sigmoid_rn(float x) {
  return static_cast<float>(1.0 / (1.0 + exp(-static_cast<double>(x))));
}

__device__ __forceinline__ void top2_insert(float v, float& a1, float& a2) {
  if (v > a1) {
    a2 = a1;
    a1 = v;
  } else if (v > a2) {
    a2 = v;
  }
}

template <int VPL>
__global__ __launch_bounds__(64 * kGroupedWaves) void router_grouped_kernel(
    const float* __restrict__ logits, int T, int E, int k, int n_group, int topk_group, const float* __restrict__ bias,
    int renorm, float scaling, int32_t* __restrict__ ids, float* __restrict__ wts) {
  __shared__ float s_gs[kGroupedWaves][kGroupedMaxE / 2];   // group scores (groups hold >= 2 experts)
  __shared__ int s_sel[kGroupedWaves][kGroupedMaxE / 2];
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int t = blockIdx.x * kGroupedWaves + wv;
  if (t >= T) return;   // wave-uniform; no barrier below
  const float NEG_INF = -__builtin_inff();
  const int gsize = E / n_group;

  float sg[VPL], c[VPL];
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int e = lane * VPL + j;
    if (e < E) {
      sg[j] = sigmoid_rn(logits[static_cast<long long>(t) * E + e]);
      c[j] = sg[j] + (bias ? bias[e] : 0.f);
    } else {
      sg[j] = 0.f;
      c[j] = NEG_INF;
    }
  }
  // group scores: top-2 sum per group, one wave-wide reduction per group
#pragma unroll 1
  for (int g = 0; g < n_group; ++g) {
    float a1 = NEG_INF, a2 = NEG_INF;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      const int e = lane * VPL + j;
      if (e < E && e / gsize == g) top2_insert(c[j], a1, a2);
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
      const float b1 = __shfl_xor(a1, m, 64);
      const float b2 = __shfl_xor(a2, m, 64);
      const float hi = fmaxf(a1, b1);
      a2 = fmaxf(fminf(a1, b1), fmaxf(a2, b2));
      a1 = hi;
    }
    if (lane == 0) s_gs[wv][g] = a1 + a2;
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  // keep the topk_group best groups (ties to the lower group index)
  for (int g = lane; g < n_group; g += 64) {
    const float v = s_gs[wv][g];
    int rank = 0;
    for (int h = 0; h < n_group; ++h) {
      const float u = s_gs[wv][h];
      rank += (u > v || (u == v && h < g)) ? 1 : 0;
    }
    s_sel[wv][g] = rank < topk_group;
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  uint32_t avail = 0;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int e = lane * VPL + j;
    if (e < E) {
      if (!s_sel[wv][e / gsize]) c[j] = 0.f;
      avail |= 1u << j;
    }
  }
  // top-k of the masked scores; pick r is kept by lane r (k <= 32)
  int my_id = -1;
#pragma unroll 1
  for (int r = 0; r < k; ++r) {
    float bv = NEG_INF;
    int bi = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      const int e = lane * VPL + j;
      if (((avail >> j) & 1u) && (c[j] > bv || (c[j] == bv && e < bi))) {
        bv = c[j];
        bi = e;
      }
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
      const float ov = __shfl_xor(bv, m, 64);
      const int oi = __shfl_xor(bi, m, 64);
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
    }
    if (lane == r) my_id = bi;
    if (bi / VPL == lane) avail &= ~(1u << (bi % VPL));
  }
  // weight = unbiased sigmoid of the pick, fetched from its owner lane
  float w = 0.f;
  const int src = my_id >= 0 ? my_id / VPL : 0;
  const int jj = my_id >= 0 ? my_id % VPL : 0;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const float v = __shfl(sg[j], src, 64);
    if (j == jj) w = v;
  }
  if (lane >= k) w = 0.f;
  if (renorm && k > 1) {
    float sum = w;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) sum += __shfl_xor(sum, m, 64);
    w = w / (sum + 1e-20f);
  }
  w = w * scaling;
  if (lane < k) {
    ids[static_cast<long long>(t) * k + lane] = my_id;
    wts[static_cast<long long>(t) * k + lane] = w;
  }
}

hipError_t launch_router_grouped(const float* logits, int T, int E, int k, int n_group, int topk_group,
                                 const float* bias, int renorm, float scaling, int32_t* ids, float* w,
                                 hipStream_t s) {
  const unsigned blocks = static_cast<unsigned>((T + kGroupedWaves - 1) / kGroupedWaves);
  const dim3 g(blocks > 0 ? blocks : 1), b(64 * kGroupedWaves);
  const int vpl = (E + 63) / 64;
#define EIMOE_RG(V) \
  hipLaunchKernelGGL((router_grouped_kernel<V>), g, b, 0, s, logits, T, E, k, n_group, topk_group, bias, renorm, \
                     scaling, ids, w)
  if (vpl <= 1) EIMOE_RG(1);
  else if (vpl <= 2) EIMOE_RG(2);
  else if (vpl <= 4) EIMOE_RG(4);
  else EIMOE_RG(8);
#undef EIMOE_RG
  return hipGetLastError();
}

// ---------------------------------------------------------------------------- EPLB
// Logical -> physical expert ids (eplb_map_to_physical_and_record, generation/blocks/moe/
// base.py:40-64): slot i of the flattened [T,k] ids takes replica i mod count[id] of its
// logical expert, so repeated picks of one expert spread over its replicas
// deterministically.  Ids outside [0, n_logical) (or a count outside [1, max_rep]) map to -1.
__global__ __launch_bounds__(256) void eplb_map_kernel(const int32_t* __restrict__ ids, int n,
                                                       const int32_t* __restrict__ log2phy, int n_logical,
                                                       int max_rep, const int32_t* __restrict__ replica_count,
                                                       int32_t* __restrict__ phys) {
  for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) {
    const int l = ids[i];
    int out = -1;
    if (l >= 0 && l < n_logical) {
      const int c = replica_count[l];
      if (c >= 1 && c <= max_rep) out = log2phy[static_cast<long long>(l) * max_rep + i % c];
    }
    phys[i] = out;
  }
}

hipError_t launch_eplb_map(const int32_t* ids, int n, const int32_t* log2phy, int n_logical, int max_rep,
                           const int32_t* replica_count, int32_t* phys, hipStream_t s) {
  int blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(eplb_map_kernel, dim3(blocks), dim3(256), 0, s, ids, n, log2phy, n_logical, max_rep,
                     replica_count, phys);
  return hipGetLastError();
}

// Router and align in one workgroup, for batches its 16 waves route in a few steps: the
// ids stay in LDS between the two phases, and one launch (a few microseconds of dispatch
// and cold-cache latency at decode sizes) replaces two.  Same outputs as the two kernels.
template <int LPT, int VPL, int KMAX>
__global__ __launch_bounds__(kAlignThreads) void route_align_kernel(
    const float* __restrict__ logits, int T, int E, int k, int renorm, int e_lo, int n_loc, int32_t* __restrict__ ids,
    float* __restrict__ wts, int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
    int32_t* __restrict__ sorted_flat, int32_t* __restrict__ sorted_tok, int32_t* __restrict__ pos, int rank) {
  extern __shared__ int lds[];
  int* s_ids = lds + align_lds_ints(n_loc);   // [T*k] after the align's histogram
  if (rank) {   // then [T*E] logits and [T*k] picked values
    float* s_lg = reinterpret_cast<float*>(s_ids + T * k);
    route_rank(logits, T, E, k, renorm, ids, wts, s_ids, s_lg, s_lg + T * E);
  } else {
    route_rows<LPT, VPL, KMAX, kLdsIds>(logits, T, E, k, renorm, ids, wts, s_ids, threadIdx.x >> 6, kAlignWaves);
  }
  __syncthreads();
  if (T * k <= 64) {   // a decode step's few ids: one wave sorts them without further barriers
    if (threadIdx.x < 64) align_tiny(s_ids, T * k, k, e_lo, n_loc, counts, offsets, sorted_flat, sorted_tok, pos, lds);
    return;
  }
  align_rows<true>(s_ids, T * k, k, e_lo, n_loc, counts, offsets, sorted_flat, sorted_tok, pos, lds);
}

namespace {

constexpr int kRouteAlignMaxSteps = 2;          // routing steps of the 16 waves
constexpr size_t kRouteAlignMaxLds = 64 * 1024;

int router_lanes(int E) { return E <= 8 ? 8 : E <= 128 ? 16 : 32; }

// A token or two over wider routers take the rank selection (route_rank): the k argmax rounds
// of route_rows are a chain of dependent lane-group reductions (~0.44 us each at 128 experts),
// while ranking costs T*E*E compares on the one workgroup's VALU.  Measured (one box, cache-cold
// Qwen3-30B-A3B 32-expert share): 1 token 23.2 -> 21.5 us; with the rank path up to T*E = 4096,
// 8 tokens 49.4 -> 55.9 us and 32 tokens 66.6 -> 97.5 us.
bool route_by_rank(int T, int E) { return E >= 16 && static_cast<long long>(T) * E <= 256; }

size_t route_align_lds_bytes(int T, int E, int k, int n_loc) {
  const size_t extra = route_by_rank(T, E) ? static_cast<size_t>(T) * E + static_cast<size_t>(T) * k : 0;
  return (static_cast<size_t>(align_lds_ints(n_loc)) + static_cast<size_t>(T) * k + extra) * sizeof(int);
}

template <int LPT, int VPL>
hipError_t launch_route_align_lv(const float* logits, int T, int E, int k, int renorm, int e_lo, int n_loc,
                                 int32_t* ids, float* w, int32_t* counts, int32_t* offsets, int32_t* sorted_flat,
                                 int32_t* sorted_tok, int32_t* pos, hipStream_t s) {
  const size_t lds = route_align_lds_bytes(T, E, k, n_loc);
  const int rank = route_by_rank(T, E) ? 1 : 0;
  if (k <= 8)
    hipLaunchKernelGGL((route_align_kernel<LPT, VPL, 8>), dim3(1), dim3(kAlignThreads), lds, s, logits, T, E, k,
                       renorm, e_lo, n_loc, ids, w, counts, offsets, sorted_flat, sorted_tok, pos, rank);
  else
    hipLaunchKernelGGL((route_align_kernel<LPT, VPL, 32>), dim3(1), dim3(kAlignThreads), lds, s, logits, T, E, k,
                       renorm, e_lo, n_loc, ids, w, counts, offsets, sorted_flat, sorted_tok, pos, rank);
  return hipGetLastError();
}

}  // namespace

size_t route_hist_ints(int T, int E, int k, int n_loc) {
  if (route_align_fused(T, E, k, n_loc)) return 0;
  return static_cast<size_t>(route_hist_plan(T, E, k, n_loc).blocks) * n_loc;
}

bool route_align_fused(int T, int E, int k, int n_loc) {
  const long long per_step = static_cast<long long>(kAlignWaves) * (64 / router_lanes(E));
  return T >= 1 && E <= 256 && (T + per_step - 1) / per_step <= kRouteAlignMaxSteps &&
         route_align_lds_bytes(T, E, k, n_loc) <= kRouteAlignMaxLds;
}

hipError_t launch_route_align(const float* logits, int T, int E, int k, int renorm, int e_lo, int n_loc,
                              int32_t* ids, float* w, int32_t* counts, int32_t* offsets, int32_t* sorted_flat,
                              int32_t* sorted_tok, int32_t* pos, int32_t* hist, hipStream_t s) {
  if (!route_align_fused(T, E, k, n_loc)) {
    const RouteHistPlan rp = route_hist_plan(T, E, k, n_loc);
    if (hist != nullptr && rp.blocks > 0) {
      hipError_t e = launch_router_hist(logits, T, E, k, renorm, ids, w, e_lo, n_loc, rp.blocks, rp.wpb, hist, s);
      if (e != hipSuccess) return e;
      return launch_align_place(ids, T, k, e_lo, n_loc, rp.blocks, rp.chunk, hist, counts, offsets, sorted_flat,
                                sorted_tok, pos, s);
    }
    hipError_t e = launch_router_topk(logits, T, E, k, renorm, ids, w, s);
    if (e != hipSuccess) return e;
    return launch_align(ids, T, k, e_lo, n_loc, counts, offsets, sorted_flat, sorted_tok, pos, hist, s);
  }
#define EIMOE_RA(L, V) \
  return launch_route_align_lv<L, V>(logits, T, E, k, renorm, e_lo, n_loc, ids, w, counts, offsets, sorted_flat, \
                                     sorted_tok, pos, s)
  if (E <= 8) EIMOE_RA(8, 1);
  if (E <= 16) EIMOE_RA(16, 1);
  if (E <= 32) EIMOE_RA(16, 2);
  if (E <= 64) EIMOE_RA(16, 4);
  if (E <= 128) EIMOE_RA(16, 8);
  EIMOE_RA(32, 8);   // E <= 256 here (wider rows hold k <= 32 picks in too many registers)
#undef EIMOE_RA
}

}  // namespace eimoe
