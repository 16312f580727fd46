// moe_align / permute: per-expert counts, offsets and a stable expert-major
// permutation of the routed (token, slot) pairs, in one workgroup (or, for large batches
// with a workspace, in two launches over many workgroups).
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
#include "kernels.h"
#include "routing.h"

namespace eimoe {

__global__ __launch_bounds__(kAlignThreads) void align_kernel(const int32_t* __restrict__ ids, int N, int k,
                                                              int e_lo, int n_loc, int32_t* __restrict__ counts,
                                                              int32_t* __restrict__ offsets,
                                                              int32_t* __restrict__ sorted_flat,
                                                              int32_t* __restrict__ sorted_tok,
                                                              int32_t* __restrict__ pos) {
  extern __shared__ int lds[];
  align_rows<false>(ids, N, k, e_lo, n_loc, counts, offsets, sorted_flat, sorted_tok, pos, lds);
}

// ---------------------------------------------------------------------------- many workgroups
// Large batches: the same counting sort on B workgroups of kAlignMbWaves waves, workgroup
// b owning the contiguous chunk [b*chunk, (b+1)*chunk) of the flat ids (each wave a
// quarter of it).  align_hist_kernel writes every chunk's per-expert counts to
// hist[B][n_loc]; align_place_kernel has each workgroup sum that matrix (the totals, and
// per expert the counts of the chunks before its own: its chunk's base), recount its
// chunk per wave and place its ids.  Chunks precede each other in flat order, so the
// order is the same stable (expert, flat index) order; workgroup 0 writes counts and
// offsets.
constexpr int kAlignMbWaves = 4;
constexpr int kAlignMbThreads = 64 * kAlignMbWaves;

__global__ __launch_bounds__(kAlignMbThreads) void align_hist_kernel(const int32_t* __restrict__ ids, int N, int e_lo,
                                                                     int n_loc, int chunk,
                                                                     int32_t* __restrict__ hist_g) {
  extern __shared__ int lds[];   // [kAlignMbWaves][n_loc]
  const int tid = threadIdx.x;
  const int w = tid >> 6;
  const int nbits = n_loc > 1 ? 32 - __clz(n_loc - 1) : 0;
  for (int i = tid; i < kAlignMbWaves * n_loc; i += kAlignMbThreads) lds[i] = 0;
  __syncthreads();
  const int sub = chunk / kAlignMbWaves;
  const long long beg = static_cast<long long>(blockIdx.x) * chunk + static_cast<long long>(w) * sub;
  if (beg < N) count_slice<false>(ids, static_cast<int>(beg), static_cast<int>(min<long long>(N, beg + sub)), e_lo, n_loc,
                                  nbits, lds + w * n_loc);
  __syncthreads();
  for (int e = tid; e < n_loc; e += kAlignMbThreads) {
    int c = 0;
#pragma unroll
    for (int ww = 0; ww < kAlignMbWaves; ++ww) c += lds[ww * n_loc + e];
    hist_g[static_cast<long long>(blockIdx.x) * n_loc + e] = c;
  }
}

__global__ __launch_bounds__(kAlignMbThreads) void align_place_kernel(
    const int32_t* __restrict__ ids, int N, int k, int e_lo, int n_loc, int chunk, const int32_t* __restrict__ hist_g,
    int32_t* __restrict__ counts, int32_t* __restrict__ offsets, int32_t* __restrict__ sorted_flat,
    int32_t* __restrict__ sorted_tok, int32_t* __restrict__ pos) {
  extern __shared__ int lds[];
  int* hist = lds;                                // [kAlignMbWaves][n_loc]
  int* tot = hist + kAlignMbWaves * n_loc;        // [n_loc]
  int* base = tot + n_loc;                        // [n_loc]
  int* offs = base + n_loc;                       // [n_loc + 1]
  const int tid = threadIdx.x;
  const int w = tid >> 6;
  const int nbits = n_loc > 1 ? 32 - __clz(n_loc - 1) : 0;
  for (int i = tid; i < kAlignMbWaves * n_loc; i += kAlignMbThreads) hist[i] = 0;
  for (int e = tid; e < n_loc; e += kAlignMbThreads) tot[e] = base[e] = 0;
  __syncthreads();
  // Column sums of the chunk-count matrix (at most kAlignMbMaxCells cells, coalesced;
  // integer LDS atomics, so the order does not matter): totals, and the chunks before this
  // one.  The first few cells per thread are loaded before the recount below, so their
  // latency overlaps it.
  const int cells = static_cast<int>(gridDim.x) * n_loc;
  const int own = static_cast<int>(blockIdx.x) * n_loc;
  constexpr int kEarly = 4;
  int early[kEarly];
#pragma unroll
  for (int j = 0; j < kEarly; ++j) {
    const int i = tid + j * kAlignMbThreads;
    early[j] = i < cells ? hist_g[i] : 0;
  }
  const int sub = chunk / kAlignMbWaves;
  const long long beg = static_cast<long long>(blockIdx.x) * chunk + static_cast<long long>(w) * sub;
  const int b0 = static_cast<int>(min<long long>(beg, N));
  const int b1 = static_cast<int>(min<long long>(beg + sub, N));
  count_slice<false>(ids, b0, b1, e_lo, n_loc, nbits, hist + w * n_loc);
  auto add_cell = [&](int i, int c) {
    if (c != 0) {
      atomicAdd(&tot[i % n_loc], c);
      if (i < own) atomicAdd(&base[i % n_loc], c);
    }
  };
#pragma unroll
  for (int j = 0; j < kEarly; ++j) add_cell(tid + j * kAlignMbThreads, early[j]);
#pragma unroll 4
  for (int i = tid + kEarly * kAlignMbThreads; i < cells; i += kAlignMbThreads) add_cell(i, hist_g[i]);
  __syncthreads();
  scan_experts(tot, n_loc, offs);
  __syncthreads();
  if (blockIdx.x == 0) {
    for (int e = tid; e < n_loc; e += kAlignMbThreads) counts[e] = tot[e];
    for (int i = tid; i <= n_loc; i += kAlignMbThreads) offsets[i] = offs[i];
  }
  // per-(wave, expert) cursors: expert start + chunks before this one + waves before this one
  for (int e = tid; e < n_loc; e += kAlignMbThreads) {
    int c = offs[e] + base[e];
#pragma unroll
    for (int ww = 0; ww < kAlignMbWaves; ++ww) {
      const int n = hist[ww * n_loc + e];
      hist[ww * n_loc + e] = c;
      c += n;
    }
  }
  __syncthreads();
  place_slice<false>(ids, b0, b1, k, e_lo, n_loc, nbits, hist + w * n_loc, sorted_flat, sorted_tok, pos);
}

size_t align_lds_bytes(int n_loc) { return static_cast<size_t>(align_lds_ints(n_loc)) * sizeof(int); }

hipError_t launch_align_place(const int32_t* ids, int T, int k, int e_lo, int n_loc, int blocks, int chunk,
                              const int32_t* hist, int32_t* counts, int32_t* offsets, int32_t* sorted_flat,
                              int32_t* sorted_tok, int32_t* pos, hipStream_t s) {
  if (blocks < 1 || chunk % kAlignMbWaves != 0 || static_cast<long long>(blocks) * n_loc > kAlignMbMaxCells)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(align_place_kernel, dim3(blocks), dim3(kAlignMbThreads),
                     static_cast<size_t>(kAlignMbWaves + 3) * n_loc * sizeof(int) + sizeof(int), s, ids, T * k, k, e_lo,
                     n_loc, chunk, hist, counts, offsets, sorted_flat, sorted_tok, pos);
  return hipGetLastError();
}

AlignPlan align_plan(int N, int n_loc) {
  AlignPlan pl{};
  if (N < kAlignMbMinIds) return pl;
  const int per = kAlignMbIdsPerBlock;
  int blocks = (N + per - 1) / per;
  if (blocks > kAlignMbMaxBlocks) blocks = kAlignMbMaxBlocks;
  if (blocks > kAlignMbMaxCells / n_loc) blocks = kAlignMbMaxCells / n_loc;   // each workgroup reads the matrix
  if (blocks < 1) blocks = 1;
  int chunk = (N + blocks - 1) / blocks;
  chunk = (chunk + 64 * kAlignMbWaves - 1) / (64 * kAlignMbWaves) * (64 * kAlignMbWaves);
  pl.blocks = (N + chunk - 1) / chunk;
  pl.chunk = chunk;
  pl.hist_ints = static_cast<size_t>(pl.blocks) * n_loc;
  return pl;
}

hipError_t launch_align(const int32_t* ids, int T, int k, int e_lo, int n_loc, int32_t* counts, int32_t* offsets,
                        int32_t* sorted_flat, int32_t* sorted_tok, int32_t* pos, int32_t* hist, hipStream_t s) {
  const int N = T * k;
  const AlignPlan pl = align_plan(N, n_loc);
  if (hist != nullptr && pl.blocks > 0) {
    hipLaunchKernelGGL(align_hist_kernel, dim3(pl.blocks), dim3(kAlignMbThreads),
                       static_cast<size_t>(kAlignMbWaves) * n_loc * sizeof(int), s, ids, N, e_lo, n_loc, pl.chunk, hist);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_align_place(ids, T, k, e_lo, n_loc, pl.blocks, pl.chunk, hist, counts, offsets, sorted_flat,
                              sorted_tok, pos, s);
  }
  const size_t lds = align_lds_bytes(n_loc);
  hipLaunchKernelGGL(align_kernel, dim3(1), dim3(kAlignThreads), lds, s, ids, N, k, e_lo, n_loc, counts,
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
