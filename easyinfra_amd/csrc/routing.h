// Device bodies of the router (softmax -> top-k) and of the align (stable counting sort
// by expert), shared by their own kernels and by the single-workgroup kernel that runs
// both for small batches.  Reference citations are at the kernels (router.hip, align.hip).
#pragma once
#include "common.h"

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

// Route tokens wave, wave + nwaves, ... (TPW tokens per wave and step): softmax, top-k
// by logit (ties to the lower id), weights over the picks or over all experts.  LDS_OUT
// kLdsIds: the ids are also stored to lds[t*k + r] for an align in the same workgroup;
// kLdsHist: each pick of a local expert (ids e_lo + [0, n_loc)) adds 1 to lds[id - e_lo].
constexpr int kLdsNone = 0, kLdsIds = 1, kLdsHist = 2;
template <int LPT, int VPL, int KMAX, int LDS_OUT>
__device__ __forceinline__ void route_rows(const float* __restrict__ logits, int T, int E, int k, int renorm,
                                           int32_t* __restrict__ ids, float* __restrict__ wts, int* lds,
                                           int wave, int nwaves, int e_lo = 0, int n_loc = 0) {
  constexpr int TPW = 64 / LPT;
  constexpr int KPL = (KMAX + LPT - 1) / LPT;   // picks held per lane
  const int lane = threadIdx.x & 63;
  const int sub = lane / LPT;
  const int li = lane % LPT;
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
    // Pick r lives in lane r % LPT of the group (slot r / LPT), so the rounds form a rolled
    // loop: the kernel stays a few hundred instructions, which matters when it runs from a
    // cold instruction cache (a decode step's router is a few microseconds of latency).
    float myv[KPL];
    int myi[KPL];
#pragma unroll
    for (int j = 0; j < KPL; ++j) {
      myv[j] = NEG_INF;
      myi[j] = -1;
    }
    float mx = NEG_INF;
#pragma unroll 1
    for (int r = 0; r < k; ++r) {
      float bv = NEG_INF;
      int bi = 0x7fffffff;
      // Selects, no branches: written with && / || the compiler made each value a divergent
      // branch block (eight per round at 128 experts), ~0.65 us per pick (timestamped: top-8 of
      // 128 took 5.3 us of the Qwen3-shape route+align kernel).
#pragma unroll
      for (int j = 0; j < VPL; ++j) {
        const int e = li + j * LPT;
        const bool better = (((avail >> j) & 1u) != 0) & ((v[j] > bv) | ((v[j] == bv) & (e < bi)));
        bv = better ? v[j] : bv;
        bi = better ? e : bi;
      }
      group_argmax<LPT>(bv, bi);
      if (r == 0) mx = bv;
      if (r % LPT == li) {
#pragma unroll
        for (int j = 0; j < KPL; ++j)
          if (j == r / LPT) {
            myv[j] = bv;
            myi[j] = bi;
          }
      }
      if (bi != 0x7fffffff && (bi % LPT) == li) avail &= ~(1u << (bi / LPT));
    }
    float ex[KPL];
    float part = 0.f;
#pragma unroll
    for (int j = 0; j < KPL; ++j) {
      ex[j] = j * LPT + li < k ? expf(myv[j] - mx) : 0.f;
      part += ex[j];
    }
    if (!renorm) {
      part = 0.f;
#pragma unroll
      for (int j = 0; j < VPL; ++j) {
        const int e = li + j * LPT;
        if (tv && e < E) part += expf(v[j] - mx);
      }
    }
    const float denom = group_sum<LPT>(part);
    if (tv) {
#pragma unroll
      for (int j = 0; j < KPL; ++j) {
        const int r = j * LPT + li;
        if (r < k) {
          ids[static_cast<long long>(t) * k + r] = myi[j];
          if constexpr (LDS_OUT == kLdsIds) lds[t * k + r] = myi[j];
          if constexpr (LDS_OUT == kLdsHist) {
            const int g = myi[j] - e_lo;
            if (g >= 0 && g < n_loc) atomicAdd(&lds[g], 1);
          }
          wts[static_cast<long long>(t) * k + r] = ex[j] / denom;
        }
      }
    }
  }
}

// Top-k by rank for a few tokens, by the whole workgroup: value i of token t is pick r of
// the token when exactly r values of its row beat it (a larger logit, or an equal one at a
// lower id): the picks and their order of route_rows' k argmax rounds, with no dependent
// rounds.  NaN logits neither beat nor are picked; slots past a row's non-NaN values keep
// id 0x7fffffff and value -inf, as there.  The T*E logits are staged in s_lg, the picked
// values in s_pv[T*k], the ids in lds_ids[T*k]; ids and weights (pick r in lane r % 16 of
// its token's 16-lane group, as route_rows with 16-lane groups) are written out.
__device__ __forceinline__ void route_rank(const float* __restrict__ logits, int T, int E, int k, int renorm,
                                           int32_t* __restrict__ ids, float* __restrict__ wts, int* lds_ids,
                                           float* s_lg, float* s_pv) {
  const int tid = threadIdx.x;
  const int nthr = blockDim.x;
  const int V = T * E;
  const float NEG_INF = -__builtin_inff();
  for (int i = tid; i < V; i += nthr) s_lg[i] = logits[i];
  for (int i = tid; i < T * k; i += nthr) {
    lds_ids[i] = 0x7fffffff;
    s_pv[i] = NEG_INF;
  }
  __syncthreads();
  int G = 16;   // lanes per value (a power of two within a DPP row)
  while (G > 1 && V * G > nthr) G >>= 1;
  const int per_pass = nthr / G;
  for (int base = 0; base < V; base += per_pass) {
    const int v = base + tid / G;
    const int li = tid % G;
    int beats = 0;
    float x = 0.f;
    int t = 0, i = 0;
    if (v < V) {
      t = v / E;
      i = v - t * E;
      x = s_lg[v];
      const float* row = s_lg + t * E;
#pragma unroll 8   // LDS reads in flight together: the loop is otherwise a chain of read latencies
      for (int j = li; j < E; j += G) {
        const float y = row[j];
        beats += ((y > x) | ((y == x) & (j < i))) ? 1 : 0;
      }
    }
    if (G >= 2) beats += dpp_i<0xB1>(beats);
    if (G >= 4) beats += dpp_i<0x4E>(beats);
    if (G >= 8) beats += dpp_i<0x141>(beats);
    if (G >= 16) beats += dpp_i<0x140>(beats);
    if (v < V && li == 0 && x == x && beats < k) {
      lds_ids[t * k + beats] = i;
      s_pv[t * k + beats] = x;
    }
  }
  __syncthreads();
  for (int t0 = 0; t0 < T; t0 += nthr / 16) {
    const int t = t0 + tid / 16;
    const int li = tid % 16;
    const bool tv = t < T;
    const float mx = tv ? s_pv[t * k] : 0.f;
    const float ex0 = (tv && li < k) ? expf(s_pv[t * k + li] - mx) : 0.f;
    const float ex1 = (tv && li + 16 < k) ? expf(s_pv[t * k + li + 16] - mx) : 0.f;
    float part = ex0 + ex1;
    if (!renorm) {
      part = 0.f;
      if (tv)
        for (int e = li; e < E; e += 16) part += expf(s_lg[t * E + e] - mx);
    }
    const float denom = group_sum<16>(part);
    if (tv) {
      if (li < k) {
        ids[static_cast<long long>(t) * k + li] = lds_ids[t * k + li];
        wts[static_cast<long long>(t) * k + li] = ex0 / denom;
      }
      if (li + 16 < k) {
        ids[static_cast<long long>(t) * k + li + 16] = lds_ids[t * k + li + 16];
        wts[static_cast<long long>(t) * k + li + 16] = ex1 / denom;
      }
    }
  }
}

constexpr int kAlignWaves = 16;
constexpr int kAlignThreads = kAlignWaves * 64;
constexpr int kAlignBatch = 8;

// Local expert of flat ids i0 + 64r + lane (r < kAlignBatch), -1 outside [.., end) or the window.
__device__ __forceinline__ void load_batch(const int32_t* __restrict__ ids, int i0, int end, int lane, int e_lo,
                                           int n_loc, int (&e)[kAlignBatch]) {
  int raw[kAlignBatch];
#pragma unroll
  for (int r = 0; r < kAlignBatch; ++r) {
    const int i = i0 + r * 64 + lane;
    raw[r] = i < end ? ids[i] : INT32_MIN;
  }
#pragma unroll
  for (int r = 0; r < kAlignBatch; ++r) {
    const int g = raw[r] == INT32_MIN ? -1 : raw[r] - e_lo;
    e[r] = (g >= 0 && g < n_loc) ? g : -1;
  }
}

// e[r] for a wave-uniform r without indexing a register array (a select chain; the id
// loops stay rolled, so the kernel's code stays small).
__device__ __forceinline__ int pick(const int (&e)[kAlignBatch], int r) {
  int v = e[0];
#pragma unroll
  for (int j = 1; j < kAlignBatch; ++j) v = r == j ? e[j] : v;
  return v;
}

__device__ __forceinline__ uint64_t match_mask(int e, int nbits, uint64_t valid) {
  uint64_t m = valid;
  for (int b = 0; b < nbits; ++b) {
    const bool bit = (e >> b) & 1;
    const uint64_t bal = __ballot(bit);
    m &= bit ? bal : ~bal;
  }
  return m;
}

constexpr int align_lds_ints(int n_loc) { return kAlignWaves * n_loc + 2 * n_loc + 1; }

// Per-wave histogram of the local experts of flat ids [beg, end) into hist_w[n_loc]
// (one wave; the leader of each group of equal ids adds its group's size).  ROLLED walks a
// batch's rows in a loop (small code: measured faster for a few hundred ids, where the
// kernel is latency-bound), otherwise the rows are unrolled so their ballot chains overlap.
template <bool ROLLED>
__device__ __forceinline__ void count_slice(const int32_t* __restrict__ ids, int beg, int end, int e_lo, int n_loc,
                                            int nbits, int* hist_w) {
  const int lane = threadIdx.x & 63;
  auto count_row = [&](int e) {
    const uint64_t valid = __ballot(e >= 0);
    const uint64_t m = match_mask(e < 0 ? 0 : e, nbits, valid);
    if (e >= 0 && lane == __ffsll(static_cast<unsigned long long>(m)) - 1) hist_w[e] += __popcll(m);
  };
  for (int i0 = beg; i0 < end; i0 += 64 * kAlignBatch) {
    int eb[kAlignBatch];
    load_batch(ids, i0, end, lane, e_lo, n_loc, eb);
    if constexpr (ROLLED) {
#pragma unroll 1
      for (int r = 0; r < kAlignBatch && i0 + r * 64 < end; ++r) count_row(pick(eb, r));
    } else {
#pragma unroll
      for (int r = 0; r < kAlignBatch; ++r) count_row(eb[r]);
    }
  }
}

// Stable placement of flat ids [beg, end) (one wave): an id's slot is its expert's cursor
// cur_w[e] plus its rank among equal ids below it in the row; the group leader advances
// the cursor after every lane has read it (one wave's LDS operations run in program order).
template <bool ROLLED>
__device__ __forceinline__ void place_slice(const int32_t* __restrict__ ids, int beg, int end, int k, int e_lo,
                                            int n_loc, int nbits, int* cur_w, int32_t* __restrict__ sorted_flat,
                                            int32_t* __restrict__ sorted_tok, int32_t* __restrict__ pos) {
  const int lane = threadIdx.x & 63;
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  auto place_row = [&](int i, int e) {
    const uint64_t valid = __ballot(e >= 0);
    const uint64_t m = match_mask(e < 0 ? 0 : e, nbits, valid);
    int p = -1;
    if (e >= 0) p = cur_w[e] + __popcll(m & lt_mask);
    __builtin_amdgcn_wave_barrier();
    if (e >= 0 && lane == __ffsll(static_cast<unsigned long long>(m)) - 1) cur_w[e] += __popcll(m);
    if (i < end) {
      pos[i] = p;
      if (p >= 0) {
        sorted_flat[p] = i;
        sorted_tok[p] = i / k;
      }
    }
  };
  for (int i0 = beg; i0 < end; i0 += 64 * kAlignBatch) {
    int eb[kAlignBatch];
    load_batch(ids, i0, end, lane, e_lo, n_loc, eb);
    if constexpr (ROLLED) {
#pragma unroll 1
      for (int r = 0; r < kAlignBatch && i0 + r * 64 < end; ++r) place_row(i0 + r * 64 + lane, pick(eb, r));
    } else {
#pragma unroll
      for (int r = 0; r < kAlignBatch; ++r) place_row(i0 + r * 64 + lane, eb[r]);
    }
  }
}

// Exclusive scan of tot[0, n) into offs[0, n] by wave 0 (offs[n] = total).
__device__ __forceinline__ void scan_experts(const int* tot, int n, int* offs) {
  const int lane = threadIdx.x & 63;
  if ((threadIdx.x >> 6) == 0) {
    const int per = (n + 63) / 64;
    const int b0 = lane * per;
    int s = 0;
    for (int j = 0; j < per; ++j)
      if (b0 + j < n) s += tot[b0 + j];
    const int incl = wave_incl_scan(s);
    int run = incl - s;
    for (int j = 0; j < per; ++j) {
      if (b0 + j < n) {
        offs[b0 + j] = run;
        run += tot[b0 + j];
      }
    }
    if (lane == 63) offs[n] = incl;
  }
}

// The same sort for at most 64 flat ids, by one wave with no workgroup barrier: lane i
// holds id i, the match mask of its expert gives its group's size (written by the group's
// lowest lane) and its rank, and a wave scan over the experts gives the offsets.
// lds holds 2*n_loc + 1 ints.  Same outputs as align_rows.
__device__ __forceinline__ void align_tiny(const int32_t* __restrict__ ids, int N, int k, int e_lo, int n_loc,
                                           int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
                                           int32_t* __restrict__ sorted_flat, int32_t* __restrict__ sorted_tok,
                                           int32_t* __restrict__ pos, int* lds) {
  int* cnt = lds;            // [n_loc]
  int* offs = lds + n_loc;   // [n_loc + 1]
  const int lane = threadIdx.x & 63;
  const int nbits = n_loc > 1 ? 32 - __clz(n_loc - 1) : 0;
  for (int e = lane; e < n_loc; e += 64) cnt[e] = 0;
  __builtin_amdgcn_wave_barrier();
  int e = -1;
  if (lane < N) {
    const int g = ids[lane] - e_lo;
    e = (g >= 0 && g < n_loc) ? g : -1;
  }
  const uint64_t valid = __ballot(e >= 0);
  const uint64_t m = match_mask(e < 0 ? 0 : e, nbits, valid);
  if (e >= 0 && lane == __ffsll(static_cast<unsigned long long>(m)) - 1) cnt[e] = __popcll(m);
  __builtin_amdgcn_wave_barrier();
  scan_experts(cnt, n_loc, offs);
  __builtin_amdgcn_wave_barrier();
  for (int x = lane; x < n_loc; x += 64) counts[x] = cnt[x];
  for (int x = lane; x <= n_loc; x += 64) offsets[x] = offs[x];
  if (lane < N) {
    const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    const int p = e >= 0 ? offs[e] + __popcll(m & lt_mask) : -1;
    pos[lane] = p;
    if (p >= 0) {
      sorted_flat[p] = lane;
      sorted_tok[p] = lane / k;
    }
  }
}

// Counting sort of N = T*k flat ids by local expert, in one workgroup of kAlignThreads
// threads; lds holds align_lds_ints(n_loc) ints.  ids may point to global memory or LDS.
// Each wave takes a contiguous slice of the ids in batches of kAlignBatch rows of 64
// (ROLLED: see count_slice; unrolled measured faster from a few thousand ids: 24 vs 36 us
// at 16384).
template <bool ROLLED>
__device__ __forceinline__ void align_rows(const int32_t* __restrict__ ids, int N, int k, int e_lo, int n_loc,
                                           int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
                                           int32_t* __restrict__ sorted_flat, int32_t* __restrict__ sorted_tok,
                                           int32_t* __restrict__ pos, int* lds) {
  int* hist = lds;                              // [kAlignWaves][n_loc]
  int* tot = lds + kAlignWaves * n_loc;         // [n_loc]
  int* offs = tot + n_loc;                      // [n_loc + 1]
  const int tid = threadIdx.x;
  const int w = tid >> 6;

  int chunk = (N + kAlignWaves - 1) / kAlignWaves;
  chunk = (chunk + 63) & ~63;
  const int beg = w * chunk;
  const int end = min(N, beg + chunk);
  const int nbits = n_loc > 1 ? 32 - __clz(n_loc - 1) : 0;

  for (int i = tid; i < kAlignWaves * n_loc; i += kAlignThreads) hist[i] = 0;
  __syncthreads();
  count_slice<ROLLED>(ids, beg, end, e_lo, n_loc, nbits, hist + w * n_loc);   // pass 1: per-wave histogram
  __syncthreads();

  // per expert: exclusive prefix over waves and total count
  for (int e = tid; e < n_loc; e += kAlignThreads) {
    int run = 0;
    for (int ww = 0; ww < kAlignWaves; ++ww) {
      const int c = hist[ww * n_loc + e];
      hist[ww * n_loc + e] = run;
      run += c;
    }
    tot[e] = run;
    counts[e] = run;
  }
  __syncthreads();
  scan_experts(tot, n_loc, offs);
  __syncthreads();
  for (int i = tid; i <= n_loc; i += kAlignThreads) offsets[i] = offs[i];
  for (int i = tid; i < kAlignWaves * n_loc; i += kAlignThreads) hist[i] += offs[i % n_loc];
  __syncthreads();
  place_slice<ROLLED>(ids, beg, end, k, e_lo, n_loc, nbits, hist + w * n_loc, sorted_flat, sorted_tok, pos);   // pass 2
}

}  // namespace eimoe
