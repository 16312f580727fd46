// moe_align / permute: per-expert counts, offsets and a stable expert-major
// permutation of the routed (token, slot) pairs, in one workgroup.
//
// Replaces, at ep=1:
//   _MoeBlock._all_expert_count_compute (easyinfra/generation/blocks/moe/base.py:343-364)
//     counts = zeros(E).scatter_add_(0, ids, 1), restricted to the local window (base.py:187)
//   MoeAll2AllBlock.all2all_chunk_routing_compute (moe_all2all.py:346-348)
//     idx = ids.view(-1).sort().indices; token = idx // k; slot = idx % k
// and the M-block schedule of TritonExperts.forward_ep (fused_moe.py:413-439): the
// GEMMs derive their tiles from ``offsets`` on the device, so no host sync is needed.
//
// Order is pinned stable: (expert, flat index t*k+slot).  Integer-only and bit-exact.
//
// Algorithm (16 waves, LDS counting sort): wave w owns a contiguous slice of the
// flat ids.  Pass 1 builds a per-wave histogram with match masks (8-10 ballots per
// 64 ids, no atomics).  A prefix over waves and experts turns it into per-(wave,
// expert) write cursors.  Pass 2 re-reads the slice; each id's slot is its cursor
// plus its rank among equal ids below it in the wave, so the result is stable.
// Both passes fetch kAlignBatch rows of 64 ids per lane before using any of them: one
// workgroup does all the work, so a dependent load per 64 ids would put a memory
// latency on every step (tens of microseconds at 16-25k routed pairs).
#include "common.h"
#include "kernels.h"

namespace eimoe {

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

__device__ __forceinline__ uint64_t match_mask(int e, int nbits, uint64_t valid) {
  uint64_t m = valid;
  for (int b = 0; b < nbits; ++b) {
    const bool bit = (e >> b) & 1;
    const uint64_t bal = __ballot(bit);
    m &= bit ? bal : ~bal;
  }
  return m;
}

__global__ __launch_bounds__(kAlignThreads) void align_kernel(const int32_t* __restrict__ ids, int N, int k,
                                                              int e_lo, int n_loc, int32_t* __restrict__ counts,
                                                              int32_t* __restrict__ offsets,
                                                              int32_t* __restrict__ sorted_flat,
                                                              int32_t* __restrict__ sorted_tok,
                                                              int32_t* __restrict__ pos) {
  extern __shared__ int lds[];
  int* hist = lds;                              // [kAlignWaves][n_loc]
  int* tot = lds + kAlignWaves * n_loc;         // [n_loc]
  int* offs = tot + n_loc;                      // [n_loc + 1]
  const int tid = threadIdx.x;
  const int w = tid >> 6;
  const int lane = tid & 63;
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));

  int chunk = (N + kAlignWaves - 1) / kAlignWaves;
  chunk = (chunk + 63) & ~63;
  const int beg = w * chunk;
  const int end = min(N, beg + chunk);
  const int nbits = n_loc > 1 ? 32 - __clz(n_loc - 1) : 0;

  for (int i = tid; i < kAlignWaves * n_loc; i += kAlignThreads) hist[i] = 0;
  __syncthreads();

  // pass 1: per-wave histogram
  for (int i0 = beg; i0 < end; i0 += 64 * kAlignBatch) {
    int eb[kAlignBatch];
    load_batch(ids, i0, end, lane, e_lo, n_loc, eb);
#pragma unroll
    for (int r = 0; r < kAlignBatch; ++r) {
      const int e = eb[r];
      const uint64_t valid = __ballot(e >= 0);
      const uint64_t m = match_mask(e < 0 ? 0 : e, nbits, valid);
      if (e >= 0 && lane == __ffsll(static_cast<unsigned long long>(m)) - 1)
        hist[w * n_loc + e] += __popcll(m);
    }
  }
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

  // exclusive scan over experts (wave 0)
  if (w == 0) {
    const int per = (n_loc + 63) / 64;
    const int b0 = lane * per;
    int s = 0;
    for (int j = 0; j < per; ++j)
      if (b0 + j < n_loc) s += tot[b0 + j];
    const int incl = wave_incl_scan(s);
    int run = incl - s;
    for (int j = 0; j < per; ++j) {
      if (b0 + j < n_loc) {
        offs[b0 + j] = run;
        run += tot[b0 + j];
      }
    }
    if (lane == 63) offs[n_loc] = incl;
  }
  __syncthreads();
  for (int i = tid; i <= n_loc; i += kAlignThreads) offsets[i] = offs[i];
  for (int i = tid; i < kAlignWaves * n_loc; i += kAlignThreads) hist[i] += offs[i % n_loc];
  __syncthreads();

  // pass 2: stable placement.  All lanes read their cursor before the group leader
  // advances it; one wave's LDS operations execute in program order.
  for (int i0 = beg; i0 < end; i0 += 64 * kAlignBatch) {
    int eb[kAlignBatch];
    load_batch(ids, i0, end, lane, e_lo, n_loc, eb);
#pragma unroll
    for (int r = 0; r < kAlignBatch; ++r) {
      const int i = i0 + r * 64 + lane;
      const int e = eb[r];
      const uint64_t valid = __ballot(e >= 0);
      const uint64_t m = match_mask(e < 0 ? 0 : e, nbits, valid);
      int p = -1;
      if (e >= 0) p = hist[w * n_loc + e] + __popcll(m & lt_mask);
      __builtin_amdgcn_wave_barrier();
      if (e >= 0 && lane == __ffsll(static_cast<unsigned long long>(m)) - 1)
        hist[w * n_loc + e] += __popcll(m);
      if (i < end) {
        pos[i] = p;
        if (p >= 0) {
          sorted_flat[p] = i;
          sorted_tok[p] = i / k;
        }
      }
    }
  }
}

size_t align_lds_bytes(int n_loc) {
  return static_cast<size_t>(kAlignWaves * n_loc + 2 * n_loc + 1) * sizeof(int);
}

hipError_t launch_align(const int32_t* ids, int T, int k, int e_lo, int n_loc, int32_t* counts, int32_t* offsets,
                        int32_t* sorted_flat, int32_t* sorted_tok, int32_t* pos, hipStream_t s) {
  const size_t lds = align_lds_bytes(n_loc);
  hipLaunchKernelGGL(align_kernel, dim3(1), dim3(kAlignThreads), lds, s, ids, T * k, k, e_lo, n_loc, counts,
                     offsets, sorted_flat, sorted_tok, pos);
  return hipGetLastError();
}

// Segments from a counts vector (the forward_ep entry: rows already grouped by
// (src_rank, local_expert), fused_moe.py:395-439).  offsets = exclusive cumsum.
__global__ __launch_bounds__(64) void counts_to_offsets_kernel(const int32_t* __restrict__ counts, int S,
                                                               int32_t* __restrict__ offsets) {
  const int lane = threadIdx.x;
  const int per = (S + 63) / 64;
  const int b0 = lane * per;
  int s = 0;
  for (int j = 0; j < per; ++j)
    if (b0 + j < S) s += counts[b0 + j];
  const int incl = wave_incl_scan(s);
  int run = incl - s;
  for (int j = 0; j < per; ++j) {
    if (b0 + j < S) {
      offsets[b0 + j] = run;
      run += counts[b0 + j];
    }
  }
  if (lane == 63) offsets[S] = incl;
}

hipError_t launch_counts_to_offsets(const int32_t* counts, int S, int32_t* offsets, hipStream_t s) {
  hipLaunchKernelGGL(counts_to_offsets_kernel, dim3(1), dim3(64), 0, s, counts, S, offsets);
  return hipGetLastError();
}

}  // namespace eimoe
