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

template <int NFRAG, int MBLK>
struct StreamStage {
  bf16x8_t b[NFRAG][2];
  bf16x8_t a[MBLK][2];
};

template <int NFRAG, int MBLK>
__device__ __forceinline__ void stream_load(StreamStage<NFRAG, MBLK>& st, __amdgpu_buffer_rsrc_t ra,
                                            __amdgpu_buffer_rsrc_t rb, const uint32_t (&a_voff)[MBLK],
                                            const uint32_t (&b_voff)[NFRAG], int step) {
#if defined(__HIP_DEVICE_COMPILE__)
  const int soff = step * 128;   // 64 bf16 per k step
#pragma unroll
  for (int f = 0; f < NFRAG; ++f)
#pragma unroll
    for (int h = 0; h < 2; ++h)
      st.b[f][h] = __builtin_bit_cast(bf16x8_t, __builtin_amdgcn_raw_buffer_load_b128(rb, b_voff[f], soff + h * 64, 0));
#pragma unroll
  for (int m = 0; m < MBLK; ++m)
#pragma unroll
    for (int h = 0; h < 2; ++h)
      st.a[m][h] = __builtin_bit_cast(bf16x8_t, __builtin_amdgcn_raw_buffer_load_b128(ra, a_voff[m], soff + h * 64, 0));
#endif
}

template <int NFRAG, int MBLK>
__device__ __forceinline__ void stream_mma(f32x4_t (&acc)[MBLK][NFRAG], const StreamStage<NFRAG, MBLK>& st) {
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int m = 0; m < MBLK; ++m)
#pragma unroll
      for (int f = 0; f < NFRAG; ++f)
        acc[m][f] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(st.a[m][h], st.b[f][h], acc[m][f], 0, 0, 0);
}

// EPI kEpiSiluBF16: fragments [0, NFRAG/2) are gate rows col0 + 16f + (0..15), fragments
// [NFRAG/2, NFRAG) the matching up rows; else NFRAG fragments of 16 consecutive output
// columns.  W waves split K (K/64 is a multiple of W*U: the launcher picks W and U).
template <int EPI, int NFRAG, int MBLK, int U, int W>
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
  const uint32_t kq = static_cast<uint32_t>((lane >> 4) * 16);   // this lane's 16-byte k chunk
  const __amdgpu_buffer_rsrc_t ra =
      make_rsrc(static_cast<const uint16_t*>(p.a) + k0, (p.a_rows_cap * p.lda - k0) * 2);
  const __amdgpu_buffer_rsrc_t rb =
      make_rsrc(static_cast<const uint16_t*>(p.b) + static_cast<long long>(expert) * p.b_estride + k0,
                (p.b_estride - k0) * 2);
  uint32_t a_voff[MBLK], b_voff[NFRAG];
#pragma unroll
  for (int m = 0; m < MBLK; ++m) {
    const int r = min(row0 + m * 16 + lr, row_end - 1);
    const long long src = p.a_rows ? static_cast<long long>(p.a_rows[r]) : static_cast<long long>(r);
    a_voff[m] = static_cast<uint32_t>(src * p.lda * 2) + kq;
  }
#pragma unroll
  for (int f = 0; f < NFRAG; ++f) {
    const int wr = SILU ? (f < G ? col0 + f * 16 + lr : p.up_off + col0 + (f - G) * 16 + lr) : col0 + f * 16 + lr;
    b_voff[f] = static_cast<uint32_t>(static_cast<long long>(wr) * p.ldb * 2) + kq;
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
  const int KW = p.K / 64 / W;   // k steps of this wave
  const int s0 = wave * KW;
  const int s_last = s0 + KW - 1;
  StreamStage<NFRAG, MBLK> st[U];
#pragma unroll
  for (int u = 0; u < U - 1; ++u) {
    stream_load<NFRAG, MBLK>(st[u], ra, rb, a_voff, b_voff, min(s0 + u, s_last));
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_sched_barrier(0);   // stage order must match the loop's for exact vmcnt waits
#endif
  }
  for (int s = s0; s <= s_last; s += U) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      stream_load<NFRAG, MBLK>(st[(u + U - 1) % U], ra, rb, a_voff, b_voff, min(s + u + U - 1, s_last));
      stream_mma<NFRAG, MBLK>(acc, st[u]);
#if defined(__HIP_DEVICE_COMPILE__)
      __builtin_amdgcn_sched_barrier(0);   // keep the ring order: the scheduler would batch all loads
#endif
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
#pragma unroll
  for (int m = 0; m < MBLK; ++m) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = row0 + m * 16 + lq * 4 + r;
      if (row >= row_end) continue;
      const float rs = p.a_scale ? p.a_scale[p.a_rows ? p.a_rows[row] : row] : 1.f;
      if constexpr (SILU) {
#pragma unroll
        for (int f = 0; f < G; ++f) {
          const float g = acc[m][f][r] * rs;
          const float u = acc[m][G + f][r] * rs;
          static_cast<uint16_t*>(p.c)[static_cast<long long>(row) * p.ldc + col0 + f * 16 + lr] =
              f32_to_bf16(silu_f32(g) * u);
        }
      } else {
#pragma unroll
        for (int f = 0; f < NFRAG; ++f) {
          const int col = col0 + f * 16 + lr;
          const long long off =
              static_cast<long long>(split) * p.c_split_stride + static_cast<long long>(row) * p.ldc + col;
          const float v = acc[m][f][r] * rs;
          if constexpr (EPI == kEpiStoreF32) static_cast<float*>(p.c)[off] = v;
          else static_cast<uint16_t*>(p.c)[off] = f32_to_bf16(v);
        }
      }
    }
  }
}

template <int EPI, int NFRAG, int MBLK, int W>
hipError_t launch_stream_w(const GemmArgs& p, dim3 g, hipStream_t s) {
  const dim3 b(64 * W);
  if ((p.K / 64 / W) % 2 == 0) hipLaunchKernelGGL((grouped_gemm_stream_kernel<EPI, NFRAG, MBLK, 2, W>), g, b, 0, s, p);
  else hipLaunchKernelGGL((grouped_gemm_stream_kernel<EPI, NFRAG, MBLK, 1, W>), g, b, 0, s, p);
  return hipGetLastError();
}

template <int EPI, int NFRAG, int MBLK>
hipError_t launch_stream_cfg(const GemmArgs& p, int max_rows, hipStream_t s) {
  constexpr int BM = 16 * MBLK;
  constexpr int COLS = (EPI == kEpiSiluBF16) ? 8 * NFRAG : 16 * NFRAG;
  const long long chunks = (static_cast<long long>(max_rows) + BM - 1) / BM + p.S;   // bound
  const long long tasks = chunks * (p.N / COLS) * p.k_split;
  if (tasks > 0x7fffffffll) return hipErrorInvalidValue;
  const dim3 g(static_cast<unsigned>(tasks > 0 ? tasks : 1));
  if ((p.K / 64) % 4 == 0) return launch_stream_w<EPI, NFRAG, MBLK, 4>(p, g, s);
  return launch_stream_w<EPI, NFRAG, MBLK, 1>(p, g, s);
}

template <int EPI, int NFRAG>
hipError_t launch_stream_nf(const GemmArgs& p, int max_rows, int mblk, hipStream_t s) {
  return mblk == 1 ? launch_stream_cfg<EPI, NFRAG, 1>(p, max_rows, s) : launch_stream_cfg<EPI, NFRAG, 2>(p, max_rows, s);
}

// Fragments per wave: 8 (measured best: each activation load feeds 8 weight fragments),
// fewer when the output width does not divide.
int stream_nfrag(const GemmArgs& p, int epi) {
  const int per = epi == kEpiSiluBF16 ? 8 : 16;   // output columns per fragment
  for (int nf = 8; nf >= 2; nf /= 2)
    if (p.N % (per * nf) == 0) return nf;
  return 0;
}

}  // namespace

bool stream_gemm_supported(const GemmArgs& p, int epi) { return p.K % 64 == 0 && stream_nfrag(p, epi) > 0; }

int stream_out_cols(int N, int epi) {
  GemmArgs p{};
  p.N = N;
  const int nf = stream_nfrag(p, epi);
  return nf * (epi == kEpiSiluBF16 ? 8 : 16);
}

hipError_t launch_stream_gemm(const GemmArgs& p, int epi, int max_rows, int mblk, hipStream_t s) {
  const int nf = stream_nfrag(p, epi);
  if (p.K % 64 != 0 || nf == 0) return hipErrorInvalidValue;
#define EIMOE_STREAM_NF(E)                                                   \
  switch (nf) {                                                              \
    case 8: return launch_stream_nf<E, 8>(p, max_rows, mblk, s);             \
    case 4: return launch_stream_nf<E, 4>(p, max_rows, mblk, s);             \
    default: return launch_stream_nf<E, 2>(p, max_rows, mblk, s);            \
  }
  if (epi == kEpiSiluBF16) { EIMOE_STREAM_NF(kEpiSiluBF16) }
  if (epi == kEpiStoreBF16) { EIMOE_STREAM_NF(kEpiStoreBF16) }
  EIMOE_STREAM_NF(kEpiStoreF32)
#undef EIMOE_STREAM_NF
}

}  // namespace eimoe
