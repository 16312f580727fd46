// Weight-streaming grouped GEMM for segments with few rows (decode batches, cold
// experts), on the same bf16 MFMA and the same GemmArgs contract as gemm.hip.
//
// Replaces, for small per-expert row counts, fused_moe_kernel
// (easyinfra/generation/modules/moe/fused_moe.py:213-296) as launched at
// fused_moe.py:445-459 (gate/up + silu(g)*u) and :463-476 (down).
//
// At a handful of rows per expert the layer reads each weight once and does ~2*rows
// FLOP per weight byte, far below the MFMA ridge: the roofline is HBM bandwidth, and
// what limits it is the number of bytes in flight and how evenly the work spreads over
// the resident waves.  So:
//   * a task is (segment, 16*NFRAG-column group, 16*MBLK-row chunk) and one workgroup of W
//     waves runs it, each wave over 1/W of K: it streams the 16 weight rows of each B
//     fragment (gate and matching up rows for the SiLU GEMM) straight from HBM into MFMA
//     operand registers, U k-steps of 64 ahead (U * NFRAG * 2 KiB of weights in flight per
//     wave), with no LDS traffic and no barrier until the end, where the W partial sums are
//     added in wave order through LDS (deterministic) and wave 0 writes the tile.  The K
//     split multiplies the task count by W, so the grid is many short workgroups and the
//     last round of the launch is small;
//   * the segment's activation rows (gathered through a_rows) come through L2 the same
//     way; rows past the segment end are clamped to its last row and never stored;
//   * the row chunks of one column group are adjacent tasks (a hot expert's weights are
//     re-read from L2, not HBM).
// MFMA v_mfma_f32_16x16x32_bf16 operand layout: lane l holds row/column l%16 and k
// 8*(l/16)..+7 of a 32-wide k step; D lane l holds rows 4*(l/16)+r of column l%16.
// Operand modes (OPS): kOpsBF16 (bf16 x bf16); kOpsW8A8 (e4m3 activations and weights,
// v_mfma_scale_f32_16x16x128_f8f6f4 with unit block scales): one 128-wide k step per 128 bytes
// of a row, the same byte addresses per lane as the bf16 64-wide step; lane l feeds bytes
// 16q..+15 and 64+16q..+15 (q = l/16) of both operands, so the k sum is exact whatever order the
// instruction adds; the per-row activation scale and per-output-channel weight scale are applied
// in the epilogue.  kOpsW8A16 (e4m3 weights, bf16 activations, the bf16 MFMA): the weights load as
// in W8A8, 128 k per step; lane l's 16 weight bytes of each 64-byte half are widened to bf16
// exactly and feed two 32-wide MFMA steps, and the activations load four 16-byte vectors per step
// in the same k order (step j covers k (j/2)*64 + 16q + (j%2)*8 + 0..7: every k once); the weight
// scale is applied in the epilogue.
#include <algorithm>

#include "common.h"
#include "kernels.h"

namespace eimoe {

namespace {

struct StreamTask {
  int seg, row0, row_end, col0, split;
};

// Task -> (segment, column group, row chunk), computed by each wave on its own: segments
// in order, then column groups, then row chunks.  Returns false (wave-uniform) past the end.
__device__ __forceinline__ bool stream_task(const GemmArgs& p, int bm, int n_groups, int cols_per_group, int task,
                                            StreamTask& t) {
  const int lane = threadIdx.x & 63;
  // total row chunks, to peel the split index off first
  int total = 0;
  for (int base = 0; base < p.S; base += 64) {
    const int s = base + lane;
    int mt = 0;
    if (s < p.S) {
      const int r0 = min(max(p.seg_off[s], 0), p.max_rows);
      const int r1 = min(max(p.seg_off[s + 1], r0), p.max_rows);
      mt = (r1 - r0 + bm - 1) / bm;
    }
    total += __shfl(wave_incl_scan(mt), 63, 64);
  }
  const int per_split = total * n_groups;
  if (task >= per_split * p.k_split) return false;
  t.split = task / per_split;
  int rest = task - t.split * per_split;
  int run = 0;
  for (int base = 0; base < p.S; base += 64) {
    const int s = base + lane;
    int mt = 0, r0 = 0, r1 = 0;
    if (s < p.S) {
      r0 = min(max(p.seg_off[s], 0), p.max_rows);
      r1 = min(max(p.seg_off[s + 1], r0), p.max_rows);
      mt = (r1 - r0 + bm - 1) / bm;
    }
    const int incl = wave_incl_scan(mt);
    const int chunk_total = __shfl(incl, 63, 64);
    if (rest < (run + chunk_total) * n_groups) {
      // first lane whose inclusive prefix passes the task
      const unsigned long long hit = __ballot((run + incl) * n_groups > rest);
      const int src = __ffsll(static_cast<long long>(hit)) - 1;
      const int mt_s = __shfl(mt, src, 64);
      const int excl = __shfl(incl - mt, src, 64);
      const int seg_r0 = __shfl(r0, src, 64);
      const int seg_r1 = __shfl(r1, src, 64);
      const int local = rest - (run + excl) * n_groups;
      const int grp = local / mt_s;
      const int chunk = local - grp * mt_s;
      t.seg = base + src;
      t.row0 = seg_r0 + chunk * bm;
      t.row_end = min(t.row0 + bm, seg_r1);
      t.col0 = grp * cols_per_group;
      return true;
    }
    run += chunk_total;
  }
  return false;
}

enum StreamOps : int { kOpsBF16 = 0, kOpsW8A8 = 1, kOpsW8A16 = 2 };
constexpr int ops_step_k(int ops) { return ops == kOpsBF16 ? 64 : 128; }   // k per step
constexpr int ops_a_vecs(int ops) { return ops == kOpsW8A16 ? 4 : 2; }     // 16-byte A vectors per step

template <int NFRAG, int MBLK, int OPS>
struct StreamStage {
  bf16x8_t b[NFRAG][2];
  bf16x8_t a[MBLK][ops_a_vecs(OPS)];
};

template <int NFRAG, int MBLK, int OPS>
__device__ __forceinline__ void stream_load(StreamStage<NFRAG, MBLK, OPS>& st, __amdgpu_buffer_rsrc_t ra,
                                            __amdgpu_buffer_rsrc_t rb, const uint32_t (&a_voff)[MBLK],
                                            const uint32_t (&b_voff)[NFRAG], int step) {
#if defined(__HIP_DEVICE_COMPILE__)
  const int soff = step * 128;   // 128 weight bytes of a row per k step
#pragma unroll
  for (int f = 0; f < NFRAG; ++f)
#pragma unroll
    for (int h = 0; h < 2; ++h)
      st.b[f][h] = __builtin_bit_cast(bf16x8_t, __builtin_amdgcn_raw_buffer_load_b128(rb, b_voff[f], soff + h * 64, 0));
  if constexpr (OPS == kOpsW8A16) {
    // 128 bf16 activations (256 bytes) per step: vector j at (j/2)*128 + (j%2)*16 past the lane's 32q
#pragma unroll
    for (int m = 0; m < MBLK; ++m)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        st.a[m][j] = __builtin_bit_cast(
            bf16x8_t, __builtin_amdgcn_raw_buffer_load_b128(ra, a_voff[m], 2 * soff + (j / 2) * 128 + (j % 2) * 16, 0));
  } else {
#pragma unroll
    for (int m = 0; m < MBLK; ++m)
#pragma unroll
      for (int h = 0; h < 2; ++h)
        st.a[m][h] =
            __builtin_bit_cast(bf16x8_t, __builtin_amdgcn_raw_buffer_load_b128(ra, a_voff[m], soff + h * 64, 0));
  }
#endif
}

// Eight e4m3 weights (the low or high half of a 16-byte vector) widened to bf16, exactly.
__device__ __forceinline__ bf16x8_t widen_fp8x8(const bf16x8_t& v, int half) {
  const u32x4_t u = __builtin_bit_cast(u32x4_t, v);
  const u32x2_t lo = fp8x4_to_bf16x4(u[2 * half]);
  const u32x2_t hi = fp8x4_to_bf16x4(u[2 * half + 1]);
  return __builtin_bit_cast(bf16x8_t, u32x4_t{lo[0], lo[1], hi[0], hi[1]});
}

__device__ __forceinline__ i32x8_t cat_fp8(const bf16x8_t& lo, const bf16x8_t& hi) {
  const u32x4_t a = __builtin_bit_cast(u32x4_t, lo);
  const u32x4_t b = __builtin_bit_cast(u32x4_t, hi);
  return i32x8_t{(int)a[0], (int)a[1], (int)a[2], (int)a[3], (int)b[0], (int)b[1], (int)b[2], (int)b[3]};
}

template <int NFRAG, int MBLK, int OPS>
__device__ __forceinline__ void stream_mma(f32x4_t (&acc)[MBLK][NFRAG], const StreamStage<NFRAG, MBLK, OPS>& st) {
  if constexpr (OPS == kOpsW8A16) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int f = 0; f < NFRAG; ++f) {
        const bf16x8_t b = widen_fp8x8(st.b[f][j / 2], j % 2);
#pragma unroll
        for (int m = 0; m < MBLK; ++m)
          acc[m][f] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(st.a[m][j], b, acc[m][f], 0, 0, 0);
      }
  } else if constexpr (OPS == kOpsW8A8) {
#pragma unroll
    for (int m = 0; m < MBLK; ++m)
#pragma unroll
      for (int f = 0; f < NFRAG; ++f)
        acc[m][f] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(cat_fp8(st.a[m][0], st.a[m][1]),
                                                                      cat_fp8(st.b[f][0], st.b[f][1]), acc[m][f],
                                                                      0, 0, 0, 127, 0, 127);
  } else {
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int m = 0; m < MBLK; ++m)
#pragma unroll
        for (int f = 0; f < NFRAG; ++f)
          acc[m][f] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(st.a[m][h], st.b[f][h], acc[m][f], 0, 0, 0);
  }
}

constexpr int kShortSteps = 4;   // k steps per wave held in flight whole by the short-stream mode

// EPI kEpiSiluBF16: fragments [0, NFRAG/2) are gate rows col0 + 16f + (0..15), fragments
// [NFRAG/2, NFRAG) the matching up rows; else NFRAG fragments of 16 consecutive output
// columns.  W waves split K (the k-step count is a multiple of W*U: the launcher picks W
// and U; U = 0 is the short-stream mode, at most kShortSteps steps per wave).  OPS: the operand
// mode (StreamOps).
template <int EPI, int NFRAG, int MBLK, int U, int W, int OPS>
__global__ void __launch_bounds__(64 * W) grouped_gemm_stream_kernel(GemmArgs p) {
  constexpr bool SILU = (EPI == kEpiSiluBF16);
  static_assert(!SILU || NFRAG % 2 == 0, "SiLU pairs gate and up fragments");
  constexpr int G = NFRAG / 2;
  constexpr int BM = 16 * MBLK;
  constexpr int COLS = SILU ? 16 * G : 16 * NFRAG;
  __shared__ f32x4_t s_part[W > 1 ? W - 1 : 1][MBLK][NFRAG][64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  StreamTask t;
  if (!stream_task(p, BM, p.N / COLS, COLS, blockIdx.x, t)) return;   // uniform over the workgroup
  const int seg = __builtin_amdgcn_readfirstlane(t.seg);
  const int row0 = __builtin_amdgcn_readfirstlane(t.row0);
  const int row_end = __builtin_amdgcn_readfirstlane(t.row_end);
  const int col0 = __builtin_amdgcn_readfirstlane(t.col0);
  const int split = __builtin_amdgcn_readfirstlane(t.split);
  const long long k0 = static_cast<long long>(split) * p.K;
  const int expert = seg % p.e_mod;

  const int lr = lane & 15;
  const uint32_t kq = static_cast<uint32_t>((lane >> 4) * 16);   // this lane's 16-byte weight chunk
  constexpr bool FP8 = OPS != kOpsBF16;                            // e4m3 weights (128-wide k steps)
  constexpr bool A8 = OPS == kOpsW8A8;                             // e4m3 activations
  constexpr int EB = FP8 ? 1 : 2;                                  // bytes per weight
  constexpr int EA = A8 ? 1 : 2;                                   // bytes per activation
  // the lane's activation bytes: the same 16-byte chunk as its weights, or, for bf16 activations
  // against e4m3 weights, the 32 bytes holding the same k
  const uint32_t kqa = OPS == kOpsW8A16 ? 2 * kq : kq;
  const __amdgpu_buffer_rsrc_t ra =
      make_rsrc(static_cast<const uint8_t*>(p.a) + k0 * EA, (p.a_rows_cap * p.lda - k0) * EA);
  const __amdgpu_buffer_rsrc_t rb =
      make_rsrc(expert_weights(p, expert, EB) + k0 * EB, (p.b_estride - k0) * EB);
  uint32_t a_voff[MBLK], b_voff[NFRAG];
#pragma unroll
  for (int m = 0; m < MBLK; ++m) {
    const int r = min(row0 + m * 16 + lr, row_end - 1);
    const long long src = p.a_rows ? static_cast<long long>(p.a_rows[r]) : static_cast<long long>(r);
    a_voff[m] = static_cast<uint32_t>(src * p.lda * EA) + kqa;
  }
  int wrow[NFRAG];
#pragma unroll
  for (int f = 0; f < NFRAG; ++f) {
    wrow[f] = SILU ? (f < G ? col0 + f * 16 + lr : p.up_off + col0 + (f - G) * 16 + lr) : col0 + f * 16 + lr;
    b_voff[f] = static_cast<uint32_t>(static_cast<long long>(wrow[f]) * p.ldb * EB) + kq;
  }

  f32x4_t acc[MBLK][NFRAG];
#pragma unroll
  for (int m = 0; m < MBLK; ++m)
#pragma unroll
    for (int f = 0; f < NFRAG; ++f) acc[m][f] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // Ring of U register stages: step s lives in stage s % U and is fetched U-1 steps ahead.
  // U divides the step count (the launcher picks it), so the loop body has no branch and
  // the compiler's vmcnt waits stay exact; fetch indices are clamped to the last step, so
  // the final iterations re-read it (L2 hits) instead of branching.
  const int KW = p.K / ops_step_k(OPS) / W;   // k steps (128 weight bytes of a row each) of this wave
  const int s0 = wave * KW;
  const int s_last = s0 + KW - 1;
  if constexpr (U == 0) {
    // Short stream (KW <= kShortSteps, small grids): every load of the wave is issued
    // before the first MFMA, so the wave waits for one memory round trip, not KW.
    StreamStage<NFRAG, MBLK, OPS> st[kShortSteps];
#pragma unroll
    for (int u = 0; u < kShortSteps; ++u)
      if (u < KW) stream_load<NFRAG, MBLK, OPS>(st[u], ra, rb, a_voff, b_voff, s0 + u);
#pragma unroll
    for (int u = 0; u < kShortSteps; ++u)
      if (u < KW) stream_mma<NFRAG, MBLK, OPS>(acc, st[u]);
  } else {
    StreamStage<NFRAG, MBLK, OPS> st[U];
#pragma unroll
    for (int u = 0; u < U - 1; ++u) {
      stream_load<NFRAG, MBLK, OPS>(st[u], ra, rb, a_voff, b_voff, min(s0 + u, s_last));
#if defined(__HIP_DEVICE_COMPILE__)
      __builtin_amdgcn_sched_barrier(0);   // stage order must match the loop's for exact vmcnt waits
#endif
    }
    for (int s = s0; s <= s_last; s += U) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        stream_load<NFRAG, MBLK, OPS>(st[(u + U - 1) % U], ra, rb, a_voff, b_voff, min(s + u + U - 1, s_last));
        stream_mma<NFRAG, MBLK, OPS>(acc, st[u]);
#if defined(__HIP_DEVICE_COMPILE__)
        __builtin_amdgcn_sched_barrier(0);   // keep the ring order: the scheduler would batch all loads
#endif
      }
    }
  }
  if constexpr (W > 1) {
    if (wave > 0) {
#pragma unroll
      for (int m = 0; m < MBLK; ++m)
#pragma unroll
        for (int f = 0; f < NFRAG; ++f) s_part[wave - 1][m][f][lane] = acc[m][f];
    }
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int w = 0; w < W - 1; ++w)
#pragma unroll
      for (int m = 0; m < MBLK; ++m)
#pragma unroll
        for (int f = 0; f < NFRAG; ++f) acc[m][f] += s_part[w][m][f][lane];
  }

  const int lq = lane >> 4;
  // The e4m3 scales are loaded before the first store: loads between stores that may alias
  // them would wait for each other, a chain of memory latencies per row.
  // bf16 operands carry no scales (the products fold away at compile time); e4m3 weights always
  // carry their channel scales, e4m3 activations their row scales (the entry points require them).
  float cs[NFRAG];   // per-output-channel weight scales of this lane's fragment columns
  float rsv[MBLK][4];   // per-row activation scales
#pragma unroll
  for (int f = 0; f < NFRAG; ++f)
    cs[f] = FP8 ? p.b_scale[static_cast<long long>(expert) * p.nb_rows + wrow[f]] : 1.f;
  // rows past the segment read the last row's scale (never stored): no per-row branch, so the
  // row-map loads issue back to back, then the scale loads (not one dependent pair per row)
  int src_row[MBLK][4];
#pragma unroll
  for (int m = 0; m < MBLK; ++m)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = min(row0 + m * 16 + lq * 4 + r, row_end - 1);
      src_row[m][r] = A8 ? (p.a_rows ? p.a_rows[row] : row) : 0;
    }
#pragma unroll
  for (int m = 0; m < MBLK; ++m)
#pragma unroll
    for (int r = 0; r < 4; ++r) rsv[m][r] = A8 ? p.a_scale[src_row[m][r]] : 1.f;
#pragma unroll
  for (int m = 0; m < MBLK; ++m) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = row0 + m * 16 + lq * 4 + r;
      if (row >= row_end) continue;
      const float rs = rsv[m][r];
      if constexpr (SILU) {
#pragma unroll
        for (int f = 0; f < G; ++f) {
          const float g = acc[m][f][r] * rs * cs[f];
          const float u = acc[m][G + f][r] * rs * cs[G + f];
          const float h = silu_f32(g) * u;
          const uint16_t hb = f32_to_bf16(h);
          const long long off = static_cast<long long>(row) * p.ldc + col0 + f * 16 + lr;
          static_cast<uint16_t*>(p.c)[off] = hb;
          if (p.c_lo) static_cast<uint16_t*>(p.c_lo)[off] = f32_to_bf16(h - bf16_to_f32(hb));
        }
      } else {
#pragma unroll
        for (int f = 0; f < NFRAG; ++f) {
          const int col = col0 + f * 16 + lr;
          const long long off =
              static_cast<long long>(split) * p.c_split_stride + static_cast<long long>(row) * p.ldc + col;
          const float v = acc[m][f][r] * rs * cs[f];
          if constexpr (EPI == kEpiStoreF32) static_cast<float*>(p.c)[off] = v;
          else static_cast<uint16_t*>(p.c)[off] = f32_to_bf16(v);
        }
      }
    }
  }
}

// Upper bound on tasks (the grid): a segment of n > 0 rows has ceil(n/BM) <= floor(n/BM) + 1
// row chunks, the rows sum to at most max_rows and at most min(S, max_rows) segments are
// non-empty.
long long stream_tasks_bound(const GemmArgs& p, int max_rows, int nfrag, int mblk, int epi) {
  const int bm = 16 * mblk;
  const int cols = (epi == kEpiSiluBF16 ? 8 : 16) * nfrag;
  const long long chunks = static_cast<long long>(max_rows) / bm + std::min(p.S, max_rows);
  return chunks * (p.N / cols) * p.k_split;
}

template <int EPI, int NFRAG, int MBLK, int W, int OPS>
hipError_t launch_stream_short(const GemmArgs& p, dim3 g, hipStream_t s) {
  hipLaunchKernelGGL((grouped_gemm_stream_kernel<EPI, NFRAG, MBLK, 0, W, OPS>), g, dim3(64 * W), 0, s, p);
  return hipGetLastError();
}

template <int EPI, int NFRAG, int MBLK, int W, int OPS>
hipError_t launch_stream_w(const GemmArgs& p, dim3 g, hipStream_t s) {
  const dim3 b(64 * W);
  if ((p.K / ops_step_k(OPS) / W) % 2 == 0)
    hipLaunchKernelGGL((grouped_gemm_stream_kernel<EPI, NFRAG, MBLK, 2, W, OPS>), g, b, 0, s, p);
  else
    hipLaunchKernelGGL((grouped_gemm_stream_kernel<EPI, NFRAG, MBLK, 1, W, OPS>), g, b, 0, s, p);
  return hipGetLastError();
}

// Grid from the row bound; the K split from the expected rows (rows_hint) when given.
template <int EPI, int NFRAG, int MBLK, int OPS>
hipError_t launch_stream_cfg(const GemmArgs& p, int max_rows, int rows, hipStream_t s) {
  const long long grid = stream_tasks_bound(p, max_rows, NFRAG, MBLK, EPI);
  if (grid > 0x7fffffffll) return hipErrorInvalidValue;
  const dim3 g(static_cast<unsigned>(grid > 0 ? grid : 1));
  const long long tasks = stream_tasks_bound(p, rows, NFRAG, MBLK, EPI);
  // Split K over the workgroup's waves only while each wave keeps >= 16 steps: shorter
  // streams spend a large share of their time filling and draining the register ring.
  const int ks = p.K / ops_step_k(OPS);
  const int w = (ks % 4 == 0 && ks / 4 >= 16) ? 4 : (ks % 2 == 0 && ks / 2 >= 16) ? 2 : 1;
  if constexpr (NFRAG == 2) {
    // Grids of fewer than ~8 waves per CU (a few tokens) are latency-bound: each wave's
    // stream is a chain of memory round trips.  Split K over 4 or 8 waves so each holds
    // at most kShortSteps steps, all in flight at once.
    if (tasks * w < 8ll * kNumCu) {
      if (ks % 4 == 0 && ks / 4 <= kShortSteps) return launch_stream_short<EPI, NFRAG, MBLK, 4, OPS>(p, g, s);
      if (ks % 8 == 0 && ks / 8 <= kShortSteps) return launch_stream_short<EPI, NFRAG, MBLK, 8, OPS>(p, g, s);
    }
  }
  if (w == 4) return launch_stream_w<EPI, NFRAG, MBLK, 4, OPS>(p, g, s);
  if (w == 2) return launch_stream_w<EPI, NFRAG, MBLK, 2, OPS>(p, g, s);
  return launch_stream_w<EPI, NFRAG, MBLK, 1, OPS>(p, g, s);
}

template <int EPI, int NFRAG, int OPS>
hipError_t launch_stream_nf(const GemmArgs& p, int max_rows, int rows, int mblk, hipStream_t s) {
  return mblk == 1 ? launch_stream_cfg<EPI, NFRAG, 1, OPS>(p, max_rows, rows, s)
                   : launch_stream_cfg<EPI, NFRAG, 2, OPS>(p, max_rows, rows, s);
}

// Fragments per wave: as many as the output width allows, up to 8 (each activation load
// then feeds 8 weight fragments: measured the fastest on large decode layers), but no more
// than keeps about 4 workgroups per CU in the grid (small layers are latency-bound).
int stream_nfrag(const GemmArgs& p, int epi, int max_rows, int mblk, bool fp8) {
  const int per = epi == kEpiSiluBF16 ? 8 : 16;   // output columns per fragment
  const int cap = fp8 ? 4 : 8;                    // e4m3: half the steps per task; 4 measured ~7 % faster
  int best = 0;
  for (int nf = 2; nf <= cap; nf *= 2) {
    if (p.N % (per * nf) != 0) continue;
    if (best == 0 || stream_tasks_bound(p, max_rows, nf, mblk, epi) >= 4ll * kNumCu) best = nf;
  }
  return best;
}

}  // namespace

bool stream_gemm_supported(const GemmArgs& p, int epi, int ops) {
  return p.K % ops_step_k(ops) == 0 && stream_nfrag(p, epi, 0, 1, ops != kOpsBF16) > 0;
}

int stream_out_cols(int N, int epi, bool fp8) {
  const int per = epi == kEpiSiluBF16 ? 8 : 16;
  for (int nf = fp8 ? 4 : 8; nf >= 2; nf /= 2)
    if (N % (per * nf) == 0) return per * nf;
  return 0;
}

hipError_t launch_stream_gemm(const GemmArgs& p, int epi, int ops, int max_rows, int mblk, hipStream_t s) {
  const int rows = p.rows_hint > 0 ? std::min(p.rows_hint, max_rows) : max_rows;   // expected rows
  const int nf = stream_nfrag(p, epi, rows, mblk, ops != kOpsBF16);
  if (p.K % ops_step_k(ops) != 0 || nf == 0) return hipErrorInvalidValue;
#define EIMOE_STREAM_NF(E, O)                                               \
  switch (nf) {                                                             \
    case 8: return launch_stream_nf<E, 8, O>(p, max_rows, rows, mblk, s);   \
    case 4: return launch_stream_nf<E, 4, O>(p, max_rows, rows, mblk, s);   \
    default: return launch_stream_nf<E, 2, O>(p, max_rows, rows, mblk, s);  \
  }
#define EIMOE_STREAM_EPI(O)                                           \
  if (epi == kEpiSiluBF16) { EIMOE_STREAM_NF(kEpiSiluBF16, O) }      \
  if (epi == kEpiStoreBF16) { EIMOE_STREAM_NF(kEpiStoreBF16, O) }    \
  EIMOE_STREAM_NF(kEpiStoreF32, O)
  if (ops == kOpsW8A8) { EIMOE_STREAM_EPI(kOpsW8A8) }
  if (ops == kOpsW8A16) { EIMOE_STREAM_EPI(kOpsW8A16) }
  EIMOE_STREAM_EPI(kOpsBF16)
#undef EIMOE_STREAM_EPI
#undef EIMOE_STREAM_NF
}

}  // namespace eimoe
