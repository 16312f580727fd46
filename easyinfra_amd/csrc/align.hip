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

size_t align_lds_bytes(int n_loc) { return static_cast<size_t>(align_lds_ints(n_loc)) * sizeof(int); }
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
