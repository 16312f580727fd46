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
  route_rows<LPT, VPL, KMAX, false>(logits, T, E, k, renorm, ids, wts, nullptr,
                                    (blockIdx.x * blockDim.x + threadIdx.x) >> 6, (gridDim.x * blockDim.x) >> 6);
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

// Router and align in one workgroup, for batches its 16 waves route in a few steps: the
// ids stay in LDS between the two phases, and one launch (a few microseconds of dispatch
// and cold-cache latency at decode sizes) replaces two.  Same outputs as the two kernels.
template <int LPT, int VPL, int KMAX>
__global__ __launch_bounds__(kAlignThreads) void route_align_kernel(
    const float* __restrict__ logits, int T, int E, int k, int renorm, int e_lo, int n_loc, int32_t* __restrict__ ids,
    float* __restrict__ wts, int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
    int32_t* __restrict__ sorted_flat, int32_t* __restrict__ sorted_tok, int32_t* __restrict__ pos) {
  extern __shared__ int lds[];
  int* s_ids = lds + align_lds_ints(n_loc);   // [T*k] after the align's histogram
  route_rows<LPT, VPL, KMAX, true>(logits, T, E, k, renorm, ids, wts, s_ids, threadIdx.x >> 6, kAlignWaves);
  __syncthreads();
  align_rows<true>(s_ids, T * k, k, e_lo, n_loc, counts, offsets, sorted_flat, sorted_tok, pos, lds);
}

namespace {

constexpr int kRouteAlignMaxSteps = 2;          // routing steps of the 16 waves
constexpr size_t kRouteAlignMaxLds = 64 * 1024;

int router_lanes(int E) { return E <= 8 ? 8 : E <= 128 ? 16 : 32; }

size_t route_align_lds_bytes(int T, int k, int n_loc) {
  return (static_cast<size_t>(align_lds_ints(n_loc)) + static_cast<size_t>(T) * k) * sizeof(int);
}

template <int LPT, int VPL>
hipError_t launch_route_align_lv(const float* logits, int T, int E, int k, int renorm, int e_lo, int n_loc,
                                 int32_t* ids, float* w, int32_t* counts, int32_t* offsets, int32_t* sorted_flat,
                                 int32_t* sorted_tok, int32_t* pos, hipStream_t s) {
  const size_t lds = route_align_lds_bytes(T, k, n_loc);
  if (k <= 8)
    hipLaunchKernelGGL((route_align_kernel<LPT, VPL, 8>), dim3(1), dim3(kAlignThreads), lds, s, logits, T, E, k,
                       renorm, e_lo, n_loc, ids, w, counts, offsets, sorted_flat, sorted_tok, pos);
  else
    hipLaunchKernelGGL((route_align_kernel<LPT, VPL, 32>), dim3(1), dim3(kAlignThreads), lds, s, logits, T, E, k,
                       renorm, e_lo, n_loc, ids, w, counts, offsets, sorted_flat, sorted_tok, pos);
  return hipGetLastError();
}

}  // namespace

bool route_align_fused(int T, int E, int k, int n_loc) {
  const long long per_step = static_cast<long long>(kAlignWaves) * (64 / router_lanes(E));
  return T >= 1 && E <= 256 && (T + per_step - 1) / per_step <= kRouteAlignMaxSteps &&
         route_align_lds_bytes(T, k, n_loc) <= kRouteAlignMaxLds;
}

hipError_t launch_route_align(const float* logits, int T, int E, int k, int renorm, int e_lo, int n_loc,
                              int32_t* ids, float* w, int32_t* counts, int32_t* offsets, int32_t* sorted_flat,
                              int32_t* sorted_tok, int32_t* pos, hipStream_t s) {
  if (!route_align_fused(T, E, k, n_loc)) {
    hipError_t e = launch_router_topk(logits, T, E, k, renorm, ids, w, s);
    if (e != hipSuccess) return e;
    return launch_align(ids, T, k, e_lo, n_loc, counts, offsets, sorted_flat, sorted_tok, pos, s);
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
