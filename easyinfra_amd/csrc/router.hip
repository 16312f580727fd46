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
#include "common.h"
#include "kernels.h"

namespace eimoe {

// All-reduce inside a lane group of LPT lanes.  Groups of up to 16 lanes stay inside one
// DPP row, so the steps are VALU lane permutes (quad xor-1, quad xor-2, half-row mirror, row
// mirror) instead of LDS-routed shuffles; wider groups finish with shuffles.  Both reductions
// (max by value then lowest index; sum) combine every lane of the group whatever the pairing.
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(v, v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(dpp_i<CTRL>(__float_as_int(v)));
}

__device__ __forceinline__ void take_better(float& bv, int& bi, float ov, int oi) {
  if (ov > bv || (ov == bv && oi < bi)) {
    bv = ov;
    bi = oi;
  }
}

template <int LPT>
__device__ __forceinline__ void group_argmax(float& bv, int& bi) {
  if constexpr (LPT >= 2) take_better(bv, bi, dpp_f<0xB1>(bv), dpp_i<0xB1>(bi));     // quad_perm [1,0,3,2]
  if constexpr (LPT >= 4) take_better(bv, bi, dpp_f<0x4E>(bv), dpp_i<0x4E>(bi));     // quad_perm [2,3,0,1]
  if constexpr (LPT >= 8) take_better(bv, bi, dpp_f<0x141>(bv), dpp_i<0x141>(bi));   // row_half_mirror
  if constexpr (LPT >= 16) take_better(bv, bi, dpp_f<0x140>(bv), dpp_i<0x140>(bi));  // row_mirror
#pragma unroll
  for (int m = 16; m < LPT; m <<= 1) take_better(bv, bi, __shfl_xor(bv, m, LPT), __shfl_xor(bi, m, LPT));
}

template <int LPT>
__device__ __forceinline__ float group_sum(float x) {
  if constexpr (LPT >= 2) x += dpp_f<0xB1>(x);
  if constexpr (LPT >= 4) x += dpp_f<0x4E>(x);
  if constexpr (LPT >= 8) x += dpp_f<0x141>(x);
  if constexpr (LPT >= 16) x += dpp_f<0x140>(x);
#pragma unroll
  for (int m = 16; m < LPT; m <<= 1) x += __shfl_xor(x, m, LPT);
  return x;
}

template <int LPT, int VPL, int KMAX>
__global__ __launch_bounds__(256) void router_topk_kernel(const float* __restrict__ logits, int T, int E, int k,
                                                          int renorm, int32_t* __restrict__ ids,
                                                          float* __restrict__ wts) {
  constexpr int TPW = 64 / LPT;
  const int lane = threadIdx.x & 63;
  const int sub = lane / LPT;
  const int li = lane % LPT;
  const int wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int nwaves = (gridDim.x * blockDim.x) >> 6;
  const float NEG_INF = -__builtin_inff();

  for (int t0 = wave * TPW; t0 < T; t0 += nwaves * TPW) {
    const int t = t0 + sub;
    const bool tv = t < T;
    float v[VPL];
    uint32_t avail = 0;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      const int e = li + j * LPT;
      const bool ok = tv && e < E;
      v[j] = ok ? logits[static_cast<long long>(t) * E + e] : NEG_INF;
      if (ok) avail |= 1u << j;
    }
    float selv[KMAX];
    int seli[KMAX];
#pragma unroll
    for (int r = 0; r < KMAX; ++r) {
      if (r < k) {
        float bv = NEG_INF;
        int bi = 0x7fffffff;
#pragma unroll
        for (int j = 0; j < VPL; ++j) {
          const int e = li + j * LPT;
          if ((avail >> j) & 1u) {
            if (v[j] > bv || (v[j] == bv && e < bi)) {
              bv = v[j];
              bi = e;
            }
          }
        }
        group_argmax<LPT>(bv, bi);
        selv[r] = bv;
        seli[r] = bi;
        if (bi != 0x7fffffff && (bi % LPT) == li) avail &= ~(1u << (bi / LPT));
      }
    }
    const float mx = selv[0];
    float denom = 0.f;
    if (renorm) {
#pragma unroll
      for (int r = 0; r < KMAX; ++r)
        if (r < k) denom += expf(selv[r] - mx);
    } else {
      float part = 0.f;
#pragma unroll
      for (int j = 0; j < VPL; ++j) {
        const int e = li + j * LPT;
        if (tv && e < E) part += expf(v[j] - mx);
      }
      denom = group_sum<LPT>(part);
    }
    if (tv) {
#pragma unroll
      for (int r = 0; r < KMAX; ++r) {
        if (r < k && (r % LPT) == li) {
          ids[static_cast<long long>(t) * k + r] = seli[r];
          wts[static_cast<long long>(t) * k + r] = expf(selv[r] - mx) / denom;
        }
      }
    }
  }
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

}  // namespace eimoe
