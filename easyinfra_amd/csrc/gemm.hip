// Grouped GEMM on gfx950 bf16 MFMA (v_mfma_f32_16x16x32_bf16), used for the
// expert gate/up projection (with the SiLU*mul epilogue fused) and the down
// projection.
//
// Replaces fused_moe_kernel / invoke_fused_moe_triton_kernel
// (easyinfra/generation/modules/moe/fused_moe.py:213-296, 299-367) as called at
// fused_moe.py:445-459 (gate/up, then silu(g)*u at :458-459) and :463-476 (down),
// and the grouped_gemm_single op contract (single_group_gemm_moe.py:81, 90).
//
// Both operands are K-contiguous ("TN"): A rows are tokens (optionally gathered
// through a row map, so the permute never materialises), B rows are weight output
// channels in nn.Linear layout.  Work decomposition:
//   * Segments (experts) own contiguous row ranges; each workgroup derives the
//     per-segment M-tile prefix on the device from the segment offsets, so the
//     launch needs no host sync; the grid is an upper bound and surplus workgroups
//     exit at once.
//   * Tile order: segment-major, then groups of GM m-tiles swept across all n-tiles,
//     so concurrently running workgroups share weight panels (B) and A tiles.
//   * XCD-aware: workgroups are dispatched round-robin over the 8 XCDs; logical
//     tile ids are assigned so that consecutive ids run on the same XCD (own L2).
//   * LDS double buffering with register prefetch of the next K-slab; 16-byte
//     chunks are XOR-swizzled so the MFMA fragment reads are bank-conflict free.
//   * Output column interleave: lane column c of fragment j maps to output column
//     c*NI + j, so each lane owns NI adjacent output columns and stores are wide.
//   * SiLU epilogue: a tile holds gate rows [n0, n0+BN/2) and the matching up rows
//     [I+n0, ...); h = silu(g)*u is formed in registers and stored as bf16.
//   * fp8-e4m3 weights (W8A16): B slabs are converted to bf16 exactly while being
//     staged into LDS; the per-output-channel scale is applied in the epilogue.
#include "common.h"
#include "kernels.h"

namespace eimoe {

template <int CNT>
__device__ __forceinline__ void store_f32(float* dst, const float* v) {
  if constexpr (CNT % 4 == 0) {
#pragma unroll
    for (int q = 0; q < CNT; q += 4) {
      f32x4_t t = {v[q], v[q + 1], v[q + 2], v[q + 3]};
      *reinterpret_cast<f32x4_t*>(dst + q) = t;
    }
  } else if constexpr (CNT % 2 == 0) {
#pragma unroll
    for (int q = 0; q < CNT; q += 2) {
      f32x2_t t = {v[q], v[q + 1]};
      *reinterpret_cast<f32x2_t*>(dst + q) = t;
    }
  } else {
#pragma unroll
    for (int q = 0; q < CNT; ++q) dst[q] = v[q];
  }
}

template <int CNT>
__device__ __forceinline__ void store_bf16(uint16_t* dst, const float* v) {
  if constexpr (CNT % 8 == 0) {
#pragma unroll
    for (int q = 0; q < CNT; q += 8) {
      u32x4_t t = {pack_bf16x2(v[q], v[q + 1]), pack_bf16x2(v[q + 2], v[q + 3]), pack_bf16x2(v[q + 4], v[q + 5]),
                   pack_bf16x2(v[q + 6], v[q + 7])};
      *reinterpret_cast<u32x4_t*>(dst + q) = t;
    }
  } else if constexpr (CNT % 4 == 0) {
#pragma unroll
    for (int q = 0; q < CNT; q += 4) {
      u32x2_t t = {pack_bf16x2(v[q], v[q + 1]), pack_bf16x2(v[q + 2], v[q + 3])};
      *reinterpret_cast<u32x2_t*>(dst + q) = t;
    }
  } else if constexpr (CNT % 2 == 0) {
#pragma unroll
    for (int q = 0; q < CNT; q += 2) *reinterpret_cast<uint32_t*>(dst + q) = pack_bf16x2(v[q], v[q + 1]);
  } else {
#pragma unroll
    for (int q = 0; q < CNT; ++q) dst[q] = f32_to_bf16(v[q]);
  }
}

template <int BM, int BN, int WGM, int WGN, int EPI, bool BFP8, int GM>
__global__ void __launch_bounds__(WGM * WGN * 64) grouped_gemm_kernel(GemmArgs p) {
  constexpr int BK = 64;                       // K per LDS slab (8 chunks of 8 bf16)
  constexpr int NT = WGM * WGN * 64;
  constexpr int WM = BM / WGM;
  constexpr int WN = BN / WGN;
  constexpr int MB = WM / 16;
  constexpr int NB = WN / 16;
  constexpr bool SILU = (EPI == kEpiSiluBF16);
  constexpr int NI = SILU ? NB / 2 : NB;       // adjacent output columns per lane
  constexpr int SHB = Log2<NI>::value;
  constexpr int OUT_BN = SILU ? BN / 2 : BN;
  constexpr int A_CH = BM * 8;                 // 16-byte chunks in an A slab
  constexpr int A_LD = (A_CH + NT - 1) / NT;
  constexpr int B_KPL = BFP8 ? 16 : 8;         // k elements per 16-byte global load
  constexpr int B_CPR = BK / B_KPL;            // global chunks per B row
  constexpr int B_CH = BN * B_CPR;
  constexpr int B_LD = (B_CH + NT - 1) / NT;
  static_assert(WM % 16 == 0 && WN % 16 == 0, "wave tile");
  static_assert(!SILU || (NB % 2 == 0), "silu pairs gate/up fragments");

  __shared__ __attribute__((aligned(16))) uint16_t sA[2][BM * BK];
  __shared__ __attribute__((aligned(16))) uint16_t sB[2][BN * BK];
  __shared__ int s_pref[kMaxSeg + 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int S = p.S;

  // ---- device-side tile schedule
  if (wave == 0) {
    int run = 0;
    for (int base = 0; base < S; base += 64) {
      const int s = base + lane;
      int mt = 0;
      if (s < S) {
        const int r0 = min(max(p.seg_off[s], 0), p.max_rows);
        const int r1 = min(max(p.seg_off[s + 1], r0), p.max_rows);
        mt = (r1 - r0 + BM - 1) / BM;
      }
      const int incl = wave_incl_scan(mt);
      if (s < S) s_pref[s + 1] = run + incl;
      run += __shfl(incl, 63, 64);
    }
    if (lane == 0) s_pref[0] = 0;
  }
  __syncthreads();
  const int mt_total = s_pref[S];
  const int n_tiles = p.N / OUT_BN;
  const int per_split = mt_total * n_tiles;
  const int total = per_split * p.k_split;
  const int per_xcd = (total + kNumXcd - 1) / kNumXcd;
  const int slot = blockIdx.x / kNumXcd;
  if (slot >= per_xcd) return;
  const int logical = (blockIdx.x % kNumXcd) * per_xcd + slot;
  if (logical >= total) return;

  const int split = logical / per_split;
  const int rest = logical - split * per_split;
  const int q = rest / n_tiles;
  int lo = 0, hi = S - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (s_pref[mid] <= q) lo = mid;
    else hi = mid - 1;
  }
  const int seg = lo;
  const int local = rest - s_pref[seg] * n_tiles;
  const int mt_s = s_pref[seg + 1] - s_pref[seg];
  const int grp = local / (GM * n_tiles);
  const int gm = min(GM, mt_s - grp * GM);
  const int r_in = local - grp * GM * n_tiles;
  const int n_tile = r_in / gm;
  const int m_tile = grp * GM + (r_in - n_tile * gm);
  const int seg_r0 = min(max(p.seg_off[seg], 0), p.max_rows);
  const int seg_r1 = min(max(p.seg_off[seg + 1], seg_r0), p.max_rows);
  const int row0 = seg_r0 + m_tile * BM;
  const int row_end = min(row0 + BM, seg_r1);
  const int expert = seg % p.e_mod;
  const long long k0 = static_cast<long long>(split) * p.K;

  // ---- global load addressing
  const uint16_t* a_ptr[A_LD];
  int a_lds[A_LD];
#pragma unroll
  for (int i = 0; i < A_LD; ++i) {
    const int qc = tid + NT * i;
    const int row = (qc < A_CH ? qc : 0) >> 3;
    const int c = qc & 7;
    const int gr = min(row0 + row, row_end - 1);
    const long long src = p.a_rows ? static_cast<long long>(p.a_rows[gr]) : static_cast<long long>(gr);
    a_ptr[i] = static_cast<const uint16_t*>(p.a) + src * p.lda + k0 + c * 8;
    a_lds[i] = row * BK + ((c ^ (row & 7)) << 3);
  }
  const uint8_t* b_ptr[B_LD];
  int b_lds[B_LD];
  const int bsz = BFP8 ? 1 : 2;
#pragma unroll
  for (int i = 0; i < B_LD; ++i) {
    const int qc = tid + NT * i;
    const int R = (qc < B_CH ? qc : 0) / B_CPR;
    const int c = qc % B_CPR;
    int wr;
    if constexpr (SILU) wr = (R < BN / 2) ? n_tile * (BN / 2) + R : p.up_off + n_tile * (BN / 2) + (R - BN / 2);
    else wr = n_tile * BN + R;
    b_ptr[i] = static_cast<const uint8_t*>(p.b) +
               (static_cast<long long>(expert) * p.b_estride + static_cast<long long>(wr) * p.ldb + k0 +
                static_cast<long long>(c) * B_KPL) * bsz;
    const int cb = BFP8 ? 2 * c : c;  // first bf16 chunk this load fills
    b_lds[i] = R * BK + ((cb ^ ((R >> SHB) & 7)) << 3);
  }

  u32x4_t ra[A_LD];
  u32x4_t rb[B_LD];
  auto gload = [&](int kt) {
#pragma unroll
    for (int i = 0; i < A_LD; ++i)
      if (A_CH % NT == 0 || tid + NT * i < A_CH)
        ra[i] = *reinterpret_cast<const u32x4_t*>(a_ptr[i] + static_cast<long long>(kt) * BK);
#pragma unroll
    for (int i = 0; i < B_LD; ++i)
      if (B_CH % NT == 0 || tid + NT * i < B_CH)
        rb[i] = *reinterpret_cast<const u32x4_t*>(b_ptr[i] + static_cast<long long>(kt) * BK * bsz);
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_LD; ++i)
      if (A_CH % NT == 0 || tid + NT * i < A_CH) *reinterpret_cast<u32x4_t*>(&sA[buf][a_lds[i]]) = ra[i];
#pragma unroll
    for (int i = 0; i < B_LD; ++i) {
      if (B_CH % NT == 0 || tid + NT * i < B_CH) {
        if constexpr (BFP8) {
          const int qc = tid + NT * i;
          const int R = qc / B_CPR;
          const int c = qc % B_CPR;
          const int sw = (R >> SHB) & 7;
          const u32x2_t w0 = fp8x4_to_bf16x4(rb[i][0]);
          const u32x2_t w1 = fp8x4_to_bf16x4(rb[i][1]);
          const u32x2_t w2 = fp8x4_to_bf16x4(rb[i][2]);
          const u32x2_t w3 = fp8x4_to_bf16x4(rb[i][3]);
          u32x4_t lo4 = {w0[0], w0[1], w1[0], w1[1]};
          u32x4_t hi4 = {w2[0], w2[1], w3[0], w3[1]};
          *reinterpret_cast<u32x4_t*>(&sB[buf][R * BK + (((2 * c) ^ sw) << 3)]) = lo4;
          *reinterpret_cast<u32x4_t*>(&sB[buf][R * BK + (((2 * c + 1) ^ sw) << 3)]) = hi4;
        } else {
          *reinterpret_cast<u32x4_t*>(&sB[buf][b_lds[i]]) = rb[i];
        }
      }
    }
  };

  const int wm = wave % WGM;
  const int wn = wave / WGM;
  const int lr = lane & 15;
  const int lq = lane >> 4;
  int a_off[MB];
#pragma unroll
  for (int i = 0; i < MB; ++i) a_off[i] = (wm * WM + i * 16 + lr) * BK;
  int b_row[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    if constexpr (SILU) {
      const int jj = j % NI;
      const int half = j / NI;
      b_row[j] = half * (BN / 2) + wn * (WN / 2) + lr * NI + jj;
    } else {
      b_row[j] = wn * WN + lr * NI + j;
    }
  }

  f32x4_t acc[MB][NB];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int KT = p.K / BK;
  gload(0);
  lstore(0);
  __syncthreads();
  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < KT) gload(kt + 1);
#pragma unroll
    for (int kk = 0; kk < BK / 32; ++kk) {
      const int c = kk * 4 + lq;
      bf16x8_t af[MB];
      bf16x8_t bfr[NB];
#pragma unroll
      for (int i = 0; i < MB; ++i) {
        const int R = wm * WM + i * 16 + lr;
        af[i] = *reinterpret_cast<const bf16x8_t*>(&sA[cur][a_off[i] + ((c ^ (R & 7)) << 3)]);
      }
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const int R = b_row[j];
        bfr[j] = *reinterpret_cast<const bf16x8_t*>(&sB[cur][R * BK + ((c ^ ((R >> SHB) & 7)) << 3)]);
      }
#pragma unroll
      for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < KT) lstore(cur ^ 1);
    __syncthreads();
  }

  // ---- epilogue: lane owns rows 4*lq + r of each 16-row fragment, NI adjacent columns
  const float* scale = (BFP8 && p.b_scale) ? p.b_scale + static_cast<long long>(expert) * p.nb_rows : nullptr;
#pragma unroll
  for (int i = 0; i < MB; ++i) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = row0 + wm * WM + i * 16 + lq * 4 + r;
      if (row >= row_end) continue;
      if constexpr (SILU) {
        const int col0 = n_tile * OUT_BN + wn * (WN / 2) + lr * NI;
        float h[NI];
#pragma unroll
        for (int j = 0; j < NI; ++j) {
          float g = acc[i][j][r];
          float u = acc[i][j + NI][r];
          if (scale) {
            g *= scale[col0 + j];
            u *= scale[p.up_off + col0 + j];
          }
          h[j] = silu_f32(g) * u;
        }
        store_bf16<NI>(static_cast<uint16_t*>(p.c) + static_cast<long long>(row) * p.ldc + col0, h);
      } else {
        const int col0 = n_tile * OUT_BN + wn * WN + lr * NI;
        float v[NI];
#pragma unroll
        for (int j = 0; j < NI; ++j) v[j] = acc[i][j][r] * (scale ? scale[col0 + j] : 1.f);
        const long long off = static_cast<long long>(split) * p.c_split_stride + static_cast<long long>(row) * p.ldc + col0;
        if constexpr (EPI == kEpiStoreF32) store_f32<NI>(static_cast<float*>(p.c) + off, v);
        else store_bf16<NI>(static_cast<uint16_t*>(p.c) + off, v);
      }
    }
  }
}

// ---------------------------------------------------------------------------- launch
template <int BM, int BN, int WGM, int WGN, int EPI, bool BFP8, int GM>
static hipError_t launch_cfg(const GemmArgs& p, int max_rows, hipStream_t s) {
  constexpr int OUT_BN = (EPI == kEpiSiluBF16) ? BN / 2 : BN;
  const int n_tiles = p.N / OUT_BN;
  const long long max_mt = (static_cast<long long>(max_rows) + BM - 1) / BM + p.S;
  long long total = max_mt * n_tiles * p.k_split;
  long long grid = (total + kNumXcd - 1) / kNumXcd * kNumXcd;
  if (grid < kNumXcd) grid = kNumXcd;
  if (grid > 0x7fffffffll) return hipErrorInvalidValue;
  hipLaunchKernelGGL((grouped_gemm_kernel<BM, BN, WGM, WGN, EPI, BFP8, GM>), dim3(static_cast<unsigned>(grid)),
                     dim3(WGM * WGN * 64), 0, s, p);
  return hipGetLastError();
}

template <int EPI, bool BFP8>
static hipError_t launch_epi(const GemmArgs& p, int max_rows, int tile, hipStream_t s) {
  switch (tile) {
    case kTileL: return launch_cfg<256, 256, 2, 2, EPI, BFP8, 4>(p, max_rows, s);
    case kTileM: return launch_cfg<128, 128, 2, 2, EPI, BFP8, 4>(p, max_rows, s);
    case kTileS: return launch_cfg<32, 128, 1, 4, EPI, BFP8, 1>(p, max_rows, s);
    case kTileXS: return launch_cfg<16, 64, 1, 2, EPI, BFP8, 1>(p, max_rows, s);
    default: return hipErrorInvalidValue;
  }
}

int gemm_out_cols_per_tile(int tile, int epi) {
  int bn = 0;
  switch (tile) {
    case kTileL: bn = 256; break;
    case kTileM: bn = 128; break;
    case kTileS: bn = 128; break;
    case kTileXS: bn = 64; break;
    default: return 0;
  }
  return epi == kEpiSiluBF16 ? bn / 2 : bn;
}

// Tile heuristic from the average rows per segment (the host knows only the bound).
int gemm_pick_tile(int epi, int max_rows, int S, int N) {
  const double avg = static_cast<double>(max_rows) / (S > 0 ? S : 1);
  int t;
  if (avg >= 1024) t = kTileL;
  else if (avg >= 96) t = kTileM;
  else if (avg >= 24) t = kTileS;
  else t = kTileXS;
  while (t != kTileXS && N % gemm_out_cols_per_tile(t, epi) != 0) ++t;
  return t;
}

hipError_t launch_grouped_gemm(const GemmArgs& p, int epi, bool b_fp8, int max_rows, int tile, hipStream_t s) {
  if (tile == kTileAuto) tile = gemm_pick_tile(epi, max_rows, p.S, p.N);
  if (epi == kEpiSiluBF16) return b_fp8 ? launch_epi<kEpiSiluBF16, true>(p, max_rows, tile, s)
                                        : launch_epi<kEpiSiluBF16, false>(p, max_rows, tile, s);
  if (epi == kEpiStoreBF16) return b_fp8 ? launch_epi<kEpiStoreBF16, true>(p, max_rows, tile, s)
                                         : launch_epi<kEpiStoreBF16, false>(p, max_rows, tile, s);
  return b_fp8 ? launch_epi<kEpiStoreF32, true>(p, max_rows, tile, s)
               : launch_epi<kEpiStoreF32, false>(p, max_rows, tile, s);
}

}  // namespace eimoe
