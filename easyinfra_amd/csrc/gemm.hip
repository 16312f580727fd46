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
//   * The 256x256 tile runs persistent for launches of up to 64 segments: one
//     workgroup per CU walks its XCD's share of the logical tiles, decoding them
//     from segment bounds held in registers and issuing each next tile's first
//     loads before the current tile's epilogue.
//   * Loads are buffer loads through SGPR resources (32-bit per-lane offsets, K
//     advanced through soffset, out-of-range reads return 0 instead of faulting).
//     bf16 weights go straight to LDS (buffer_load_dwordx4 ... lds, 1 KiB per wave
//     instruction); fp8-e4m3 weights (W8A16) are staged through registers and
//     converted to bf16 exactly on the way into LDS, with the per-output-channel
//     scale applied in the epilogue.
//   * LDS: 64-wide K slabs, double buffered; 16-byte chunks XOR-swizzled so the
//     MFMA fragment reads (ds_read_b128) are bank-conflict free.
//   * Output column interleave: lane column c of fragment j maps to output column
//     c*NI + j, so each lane owns NI adjacent output columns and stores are wide.
//   * SiLU epilogue: a tile holds gate rows [n0, n0+BN/2) and the matching up rows
//     [I+n0, ...); h = silu(g)*u is formed in registers and stored as bf16.
#include <algorithm>
#include <cmath>

#include "common.h"
#include "kernels.h"

namespace eimoe {

typedef __attribute__((address_space(3))) void lds_void_t;

// A buffer window: base address and byte size (bounds the hardware buffer resource).
struct BufRef {
  const void* base;
  long long bytes;
};

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

// ---------------------------------------------------------------------------- tile schedule
struct TileCoord {
  int expert, row0, row_end, n_tile, split;
  int one_mt;   // the segment is this one m-tile (its weight panels are read by no other tile)
};

// Tile `rest` of a split given its segment (clamped rows [seg_r0, seg_r1)) and the segment's first
// m-tile over all segments (pref).  Groups of GM m-tiles sweep the n-tiles together (sharing each
// weight panel through L2); the last group takes the segment's remaining 1..2*GM-1 m-tiles, so a
// short remainder tile shares the panels of the group before it instead of reading them alone.
template <int BM, int GM>
__device__ __forceinline__ void place_tile(const GemmArgs& p, int seg, int seg_r0, int seg_r1, int pref, int rest,
                                           int n_tiles, int split, TileCoord& tc) {
  const int local = rest - pref * n_tiles;
  const int mt_s = (seg_r1 - seg_r0 + BM - 1) / BM;
  const int n_grp = max(1, mt_s / GM);
  const int grp = min(local / (GM * n_tiles), n_grp - 1);
  const int gm = grp < n_grp - 1 ? GM : mt_s - grp * GM;
  const int r_in = local - grp * GM * n_tiles;
  const int n_tile = r_in / gm;
  const int m_tile = grp * GM + (r_in - n_tile * gm);
  tc.row0 = uniform(seg_r0 + m_tile * BM);
  tc.row_end = uniform(min(seg_r0 + m_tile * BM + BM, seg_r1));
  tc.expert = uniform(seg % p.e_mod);
  tc.split = uniform(split);
  tc.n_tile = uniform(n_tile);
  tc.one_mt = uniform(mt_s == 1 ? 1 : 0);
}

// Decodes this workgroup's tile; returns false (uniformly) if the workgroup has no work.
// Must be reached by every thread of the workgroup (contains a barrier).
template <int BM, int OUT_BN, int GM>
__device__ __forceinline__ bool decode_tile(const GemmArgs& p, int* s_pref, TileCoord& tc) {
  const int lane = threadIdx.x & 63;
  const int S = p.S;
  if (threadIdx.x < 64) {
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
  if (slot >= per_xcd) return false;
  const int logical = (blockIdx.x % kNumXcd) * per_xcd + slot;
  if (logical >= total) return false;
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
  const int seg_r0 = min(max(p.seg_off[seg], 0), p.max_rows);
  const int seg_r1 = min(max(p.seg_off[seg + 1], seg_r0), p.max_rows);
  place_tile<BM, GM>(p, seg, seg_r0, seg_r1, s_pref[seg], rest, n_tiles, split, tc);
  return true;
}

// Tile schedule of a launch with at most 64 segments, held in registers (lane s: segment s):
// a persistent workgroup decodes each of its tiles with a ballot and lane reads, no memory access.
struct RegSched {
  int r0, r1, incl;                         // lane s: clamped rows, inclusive m-tile prefix
  int n_tiles, per_split, total, per_xcd;   // uniform
};

template <int BM, int OUT_BN>
__device__ __forceinline__ RegSched reg_sched(const GemmArgs& p, int lane) {
  RegSched s;
  s.r0 = 0;
  s.r1 = 0;
  if (lane < p.S) {
    s.r0 = min(max(p.seg_off[lane], 0), p.max_rows);
    s.r1 = min(max(p.seg_off[lane + 1], s.r0), p.max_rows);
  }
  s.incl = wave_incl_scan((s.r1 - s.r0 + BM - 1) / BM);
  s.n_tiles = p.N / OUT_BN;
  s.per_split = uniform(__shfl(s.incl, 63, 64)) * s.n_tiles;
  s.total = s.per_split * p.k_split;
  s.per_xcd = (s.total + kNumXcd - 1) / kNumXcd;
  return s;
}

// Coordinates of logical tile `logical` (uniform); false past the end.
template <int BM, int GM>
__device__ __forceinline__ bool reg_decode(const GemmArgs& p, const RegSched& s, int logical, TileCoord& tc) {
  if (logical >= s.total) return false;
  const int split = logical / s.per_split;
  const int rest = logical - split * s.per_split;
  const int q = rest / s.n_tiles;   // m-tile over all segments
  // the first lane whose inclusive prefix passes q holds the segment (lanes past S hold the total)
  const int seg = uniform(static_cast<int>(__popcll(__ballot(s.incl <= q))));
  const int seg_r0 = __builtin_amdgcn_readlane(s.r0, seg);
  const int seg_r1 = __builtin_amdgcn_readlane(s.r1, seg);
  const int pref = __builtin_amdgcn_readlane(s.incl, seg) - (seg_r1 - seg_r0 + BM - 1) / BM;
  place_tile<BM, GM>(p, seg, seg_r0, seg_r1, pref, rest, s.n_tiles, split, tc);
  return true;
}

// ---------------------------------------------------------------------------- shared pieces
template <int BM, int BN, int WGM, int WGN, int EPI>
struct Geo {
  static constexpr int BK = 64;
  static constexpr int NW = WGM * WGN;
  static constexpr int NT = NW * 64;
  static constexpr int WM = BM / WGM;
  static constexpr int WN = BN / WGN;
  static constexpr int MB = WM / 16;
  static constexpr int NB = WN / 16;
  static constexpr bool SILU = epi_silu(EPI);
  static constexpr int NI = SILU ? NB / 2 : NB;   // output columns per lane
  static constexpr int OUT_BN = SILU ? BN / 2 : BN;
  // A lane's NI columns come in runs of CH adjacent columns, run g of lane column c starting at
  // column g*16*CH + c*CH of the wave's block.  One run (CH = NI) but for fp32 outputs of 8
  // columns per lane, which take runs of 4: each 16-byte store then writes 256 contiguous bytes
  // of a row across the 16 lane columns, where one run of 8 left every store instruction's row
  // half-written, in 16-byte pieces 32 bytes apart.
  static constexpr int CH = (EPI == kEpiStoreF32 && !SILU && NI % 4 == 0) ? 4 : NI;
  static __device__ __forceinline__ int col_in_run(int j) { return (j / CH) * 16 * CH + j % CH; }
  static_assert(WM % 16 == 0 && WN % 16 == 0, "wave tile");
  static_assert(!SILU || (NB % 2 == 0), "silu pairs gate/up fragments");

  // B is stored in fragment order: LDS row L = wn*WN + j*16 + c feeds fragment j of wave
  // column wn at lane column c, so the 16 lanes of a fragment read 16 consecutive rows.
  // Lane column c of fragment j produces output column c*CH + col_in_run(j % NI) of the
  // wave's block; in the SiLU tile, fragments j < NI are gate rows and j >= NI the matching
  // up rows.  Returns the weight row (within the expert).
  static __device__ __forceinline__ int weight_row_of_lds(int L, int n_tile, int up_off) {
    const int wn = L / WN;
    const int j = (L % WN) >> 4;
    const int c = L & 15;
    if constexpr (SILU) {
      const int col = n_tile * (BN / 2) + wn * (WN / 2) + c * NI + (j % NI);
      return j < NI ? col : up_off + col;
    } else {
      return n_tile * BN + wn * WN + c * CH + col_in_run(j);
    }
  }
};

// 16-byte chunk swizzle inside a 128-byte LDS row.  A fragment read (ds_read_b128)
// touches 16 consecutive rows at chunk q (lanes 0-15), q+1 (16-31), ...; XOR with row&7
// makes it conflict-free on gfx950 (measured with SQ_LDS_BANK_CONFLICT: 4 cycles per
// instruction, the 1 KiB/4-cycle floor; swizzles mixing in higher row bits measured
// 2-way conflicts).  It depends on R mod 8 only, so all fragments of a wave share one
// address pattern and differ by immediate offsets.
__device__ __forceinline__ int swz(int R) { return R & 7; }

// MBE: 16-row A fragments per wave in this tile (G::MB for a full-height tile, fewer for a
// segment's short remainder tile: the wave's rows are then wm * 16 * MBE + [0, 16 * MBE)).
template <class G, int MBE>
__device__ __forceinline__ void read_frags(const uint16_t* sA, const uint16_t* sB, int kk, int wm, int wn, int lane,
                                           bf16x8_t (&af)[MBE], bf16x8_t (&bfr)[G::NB]) {
  const int lr = lane & 15;
  const int c = kk * 4 + (lane >> 4);
#pragma unroll
  for (int i = 0; i < MBE; ++i) {
    const int R = wm * 16 * MBE + i * 16 + lr;
    af[i] = *reinterpret_cast<const bf16x8_t*>(&sA[R * G::BK + ((c ^ swz(R)) << 3)]);
  }
#pragma unroll
  for (int j = 0; j < G::NB; ++j) {
    const int R = wn * G::WN + j * 16 + lr;
    bfr[j] = *reinterpret_cast<const bf16x8_t*>(&sB[R * G::BK + ((c ^ swz(R)) << 3)]);
  }
}

template <class G, int MBE>
__device__ __forceinline__ void mma(f32x4_t (&acc)[MBE][G::NB], const bf16x8_t (&af)[MBE],
                                    const bf16x8_t (&bfr)[G::NB]) {
#pragma unroll
  for (int i = 0; i < MBE; ++i)
#pragma unroll
    for (int j = 0; j < G::NB; ++j)
      acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
}

// fp32 operands: a fragment's 16 bytes are 4 floats at k = 4c..4c+3 (c its chunk), one per
// v_mfma_f32_16x16x4f32; MFMA j takes float j of every lane, so lane group q contributes k =
// 4c+j and A and B agree on it.  Four MFMAs per fragment pair cover the 16 k of the chunk pair.
template <class G, int MBE>
__device__ __forceinline__ void mma_f32(f32x4_t (&acc)[MBE][G::NB], const bf16x8_t (&af)[MBE],
                                        const bf16x8_t (&bfr)[G::NB]) {
#pragma unroll
  for (int i = 0; i < MBE; ++i) {
    const f32x4_t a = __builtin_bit_cast(f32x4_t, af[i]);
#pragma unroll
    for (int j = 0; j < G::NB; ++j) {
      const f32x4_t b = __builtin_bit_cast(f32x4_t, bfr[j]);
#pragma unroll
      for (int q = 0; q < 4; ++q) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[q], b[q], acc[i][j], 0, 0, 0);
    }
  }
}

// One 64-wide K slab: two 32-wide MFMA steps, each reading its fragments first.
template <class G, int MBE, bool F32 = false>
__device__ __forceinline__ void slab_mma(f32x4_t (&acc)[MBE][G::NB], const uint16_t* sA, const uint16_t* sB, int wm,
                                         int wn, int lane) {
#pragma unroll
  for (int kk = 0; kk < G::BK / 32; ++kk) {
    bf16x8_t af[MBE], bfr[G::NB];
    read_frags<G, MBE>(sA, sB, kk, wm, wn, lane, af, bfr);
    if constexpr (F32) mma_f32<G, MBE>(acc, af, bfr);
    else mma<G, MBE>(acc, af, bfr);
  }
}

// Epilogue: lane owns rows 4*(lane/16)+r of each 16-row fragment and NI adjacent columns.
// Scales: per-output-channel weight scales (scale) and per-row activation scales (a_scale);
// either may be null, and the bf16 kernels pass compile-time nulls, so their epilogue has no
// scale arithmetic.  All are loaded before the first store: loaded between stores (which may
// alias them, as far as the compiler knows) each row's loads would wait for the previous row's,
// a chain of 16 memory latencies that measured ~12 us per 256x256 e4m3 tile.
template <class G, int MBE>
struct EpiScales {
  float cs[G::NI], cs_up[G::SILU ? G::NI : 1];   // weight scales of the lane's output columns
  float rs[MBE][4];                              // activation scale of each of the lane's rows
};

template <class G, int MBE>
__device__ __forceinline__ int epi_col0(const TileCoord& tc, int wn, int lane) {
  return G::SILU ? tc.n_tile * G::OUT_BN + wn * (G::WN / 2) + (lane & 15) * G::NI
                 : tc.n_tile * G::OUT_BN + wn * G::WN + (lane & 15) * G::CH;
}

// Two steps, so that a caller can put other loads between them: the weight scales and the
// row map (rows past the segment take the last row, whose scale is never stored: no per-row
// branch, so the row-map loads issue back to back; with a branch per row the compiler waited for
// each row's dependent pair in turn, 16 round trips, ~3.5 us per 256x256 tile), then the
// activation scales of the mapped rows.
// The null tests sit outside the loops: tested per element, they split the loads into one
// block each, and the wait inserted at every block waited for the loads in flight before it.
// mbe: the tile's 16-row fragments per wave (MBE for a tile of the full MBE class; a persistent
// kernel loads the scales of its next tile, whose class it knows only at run time, into the
// full-size arrays: rows past the tile's are clamped to its last).
template <class G, int MBE>
__device__ __forceinline__ void epi_load_scales_1(const GemmArgs& p, const TileCoord& tc, int wm, int wn, int lane,
                                                  const float* scale, const float* a_scale, EpiScales<G, MBE>& sc,
                                                  int (&src_row)[MBE][4], int mbe = MBE) {
  const int col0 = epi_col0<G, MBE>(tc, wn, lane);
  if (scale) {
#pragma unroll
    for (int j = 0; j < G::NI; ++j) {
      sc.cs[j] = scale[col0 + G::col_in_run(j)];
      if constexpr (G::SILU) sc.cs_up[j] = scale[p.up_off + col0 + j];
    }
  } else {
#pragma unroll
    for (int j = 0; j < G::NI; ++j) {
      sc.cs[j] = 1.f;
      if constexpr (G::SILU) sc.cs_up[j] = 1.f;
    }
  }
#pragma unroll
  for (int i = 0; i < MBE; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      src_row[i][r] = min(tc.row0 + wm * 16 * mbe + i * 16 + (lane >> 4) * 4 + r, tc.row_end - 1);
  if (a_scale && p.a_rows) {
#pragma unroll
    for (int i = 0; i < MBE; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) src_row[i][r] = p.a_rows[src_row[i][r]];
  }
}

template <class G, int MBE>
__device__ __forceinline__ void epi_load_scales_2(const float* a_scale, EpiScales<G, MBE>& sc,
                                                  const int (&src_row)[MBE][4]) {
  if (a_scale) {
#pragma unroll
    for (int i = 0; i < MBE; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) sc.rs[i][r] = a_scale[src_row[i][r]];
  } else {
#pragma unroll
    for (int i = 0; i < MBE; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) sc.rs[i][r] = 1.f;
  }
}

template <class G, int EPI, int MBE, int MBS>
__device__ __forceinline__ void epilogue(const GemmArgs& p, const TileCoord& tc, f32x4_t (&acc)[MBE][G::NB], int wm,
                                         int wn, int lane, const EpiScales<G, MBS>& sc) {
  static_assert(MBS >= MBE, "scales of every fragment row");
  const int lq = lane >> 4;
  const int col0 = epi_col0<G, MBE>(tc, wn, lane);
  const auto& cs = sc.cs;
  const auto& cs_up = sc.cs_up;
  const auto& rs = sc.rs;
#pragma unroll
  for (int i = 0; i < MBE; ++i) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = tc.row0 + wm * 16 * MBE + i * 16 + lq * 4 + r;
      if (row >= tc.row_end) continue;
      if constexpr (G::SILU) {
        float h[G::NI];
#pragma unroll
        for (int j = 0; j < G::NI; ++j) {
          const float g = acc[i][j][r] * rs[i][r] * cs[j];
          const float u = acc[i][j + G::NI][r] * rs[i][r] * cs_up[j];
          h[j] = silu_f32(g) * u;
        }
        const long long off = static_cast<long long>(row) * p.ldc + col0;
        if constexpr (EPI == kEpiSiluF32) {
          store_f32<G::NI>(static_cast<float*>(p.c) + off, h);
          continue;
        }
        store_bf16<G::NI>(static_cast<uint16_t*>(p.c) + off, h);
        if (p.c_lo) {   // the residual of the bf16 rounding, itself in bf16
#pragma unroll
          for (int j = 0; j < G::NI; ++j) h[j] -= bf16_to_f32(f32_to_bf16(h[j]));
          store_bf16<G::NI>(static_cast<uint16_t*>(p.c_lo) + off, h);
        }
      } else {
        float v[G::NI];
#pragma unroll
        for (int j = 0; j < G::NI; ++j) v[j] = acc[i][j][r] * rs[i][r] * cs[j];
        const long long off =
            static_cast<long long>(tc.split) * p.c_split_stride + static_cast<long long>(row) * p.ldc + col0;
        if constexpr (EPI == kEpiStoreF32) {
#pragma unroll
          for (int g = 0; g < G::NI / G::CH; ++g)
            store_f32<G::CH>(static_cast<float*>(p.c) + off + g * 16 * G::CH, v + g * G::CH);
        } else {
          store_bf16<G::NI>(static_cast<uint16_t*>(p.c) + off, v);
        }
      }
    }
  }
}

template <class G, int EPI, int MBE>
__device__ __forceinline__ void epilogue(const GemmArgs& p, const TileCoord& tc, f32x4_t (&acc)[MBE][G::NB], int wm,
                                         int wn, int lane, const float* scale, const float* a_scale) {
  EpiScales<G, MBE> sc;
  int src_row[MBE][4];
  epi_load_scales_1<G, MBE>(p, tc, wm, wn, lane, scale, a_scale, sc, src_row);
  epi_load_scales_2<G, MBE>(a_scale, sc, src_row);
  epilogue<G, EPI, MBE>(p, tc, acc, wm, wn, lane, sc);
}

// Issues one K slab of A and B straight into LDS: each wave instruction fills one
// contiguous 1 KiB block (16 bytes per lane).
// Keeps the next slab's loads at the top of the current slab's MFMA work.  Without it the
// machine scheduler sinks them towards the barrier, whose vmcnt(0) then exposes their whole
// latency on every other slab.
__device__ __forceinline__ void pin_issue() {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_sched_barrier(0);
#endif
}

// A's 1 KiB blocks (8 rows each) are interleaved over the NW waves, block i * NW + wave, so the
// first A_CNT of them per wave cover the first 8 * NW * A_CNT rows: a short tile loads only its
// rows.  B's blocks are contiguous per wave.
// b_nt (uniform): the weight loads carry the non-temporal hint.  When every weight panel is read by
// one m-tile only (decode batches: a segment's rows fit one tile), streaming them past the caches
// measured 13-20 % faster (Mixtral-8x7B 64 tokens, cold: bf16 down 176 -> 142 us on 128x128 tiles,
// W8A8 gate/up 186 -> 167 us and down 82.5 -> 74.6 us on 32x128; a plain 1 KiB-per-instruction HBM
// read 6.0-6.3 -> 6.7-7.0 TB/s); where a panel serves several m-tiles it costs the L2 reuse (W8A8
// 256-token down on 32x128 tiles 150 -> 195 us), so the launcher sets it only for one m-tile per
// segment.
template <int A_CNT, int B_PW, int NW, int A_PW>
__device__ __forceinline__ void issue_slab_dma(const BufRef& a, const BufRef& b, const uint32_t (&a_voff)[A_PW],
                                               const uint32_t (&b_voff)[B_PW], uint16_t* sA, uint16_t* sB, int wave,
                                               int soff, bool b_nt) {
#if defined(__HIP_DEVICE_COMPILE__)  // device-only builtins; the host pass only needs the declaration
  const auto rA = make_rsrc(a.base, a.bytes);
  const auto rB = make_rsrc(b.base, b.bytes);
#pragma unroll
  for (int i = 0; i < A_CNT; ++i)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rA, (lds_void_t*)(sA + (i * NW + wave) * 512), 16, a_voff[i], soff, 0,
                                             0);
  if (b_nt) {
#pragma unroll
    for (int i = 0; i < B_PW; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rB, (lds_void_t*)(sB + (wave * B_PW + i) * 512), 16, b_voff[i], soff,
                                               0, 2);
  } else {
#pragma unroll
    for (int i = 0; i < B_PW; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rB, (lds_void_t*)(sB + (wave * B_PW + i) * 512), 16, b_voff[i], soff,
                                               0, 0);
  }
#endif
}

template <int A_CNT, int NW, int A_PW>
__device__ __forceinline__ void issue_a_dma(const BufRef& a, const uint32_t (&a_voff)[A_PW], uint16_t* sA, int wave,
                                            int soff) {
#if defined(__HIP_DEVICE_COMPILE__)
  const auto rA = make_rsrc(a.base, a.bytes);
#pragma unroll
  for (int i = 0; i < A_CNT; ++i)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rA, (lds_void_t*)(sA + (i * NW + wave) * 512), 16, a_voff[i], soff, 0,
                                             0);
#endif
}

template <int B_LD, int B_CH, int NT>
__device__ __forceinline__ void load_b_fp8(const BufRef& b, const uint32_t (&b_voff)[B_LD], u32x4_t (&rb)[B_LD],
                                           int soff) {
  const auto rB = make_rsrc(b.base, b.bytes);
#pragma unroll
  for (int i = 0; i < B_LD; ++i)
    if (B_CH % NT == 0 || static_cast<int>(threadIdx.x) + NT * i < B_CH)
      rb[i] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rB, b_voff[i], soff, 0));
}

// fp8 B chunk (16 values of one row) -> two swizzled bf16 LDS chunks.
template <class G, int B_LD, int B_CH, int NT>
__device__ __forceinline__ void store_b_fp8(const u32x4_t (&rb)[B_LD], const int (&b_R)[B_LD], const int (&b_c)[B_LD],
                                            uint16_t* sB) {
#pragma unroll
  for (int i = 0; i < B_LD; ++i) {
    if (B_CH % NT == 0 || static_cast<int>(threadIdx.x) + NT * i < B_CH) {
      const int R = b_R[i];
      const int sw = swz(R);
      const u32x2_t w0 = fp8x4_to_bf16x4(rb[i][0]);
      const u32x2_t w1 = fp8x4_to_bf16x4(rb[i][1]);
      const u32x2_t w2 = fp8x4_to_bf16x4(rb[i][2]);
      const u32x2_t w3 = fp8x4_to_bf16x4(rb[i][3]);
      const u32x4_t lo4 = {w0[0], w0[1], w1[0], w1[1]};
      const u32x4_t hi4 = {w2[0], w2[1], w3[0], w3[1]};
      *reinterpret_cast<u32x4_t*>(&sB[R * G::BK + (((2 * b_c[i]) ^ sw) << 3)]) = lo4;
      *reinterpret_cast<u32x4_t*>(&sB[R * G::BK + (((2 * b_c[i] + 1) ^ sw) << 3)]) = hi4;
    }
  }
}

// ---------------------------------------------------------------------------- row-height classes
// A segment's tiles are BM rows except its last, which takes the smallest of BM/4, BM/2 and BM
// rows that covers the remainder (when the slab split gives every wave whole 1 KiB A blocks at
// that height): the waves keep their 2-D layout with MBE = MB/4 or MB/2 fragment rows each, so
// a 2-row remainder of a Mixtral expert costs a quarter of a full tile's MFMAs, not all of them.
template <int MB, int A_PW>
struct Heights {
  static constexpr bool kQuarter = MB % 4 == 0 && A_PW % 4 == 0;
  static constexpr bool kHalf = MB % 2 == 0 && A_PW % 2 == 0;
};

// Calls body.template operator()<MBE>() with the MBE of this tile's rows (uniform per workgroup).
template <int BM, int MB, int A_PW, class Body>
__device__ __forceinline__ void by_height(int rows, Body&& body) {
  if constexpr (Heights<MB, A_PW>::kQuarter) {
    if (rows <= BM / 4) {
      body.template operator()<MB / 4>();
      return;
    }
  }
  if constexpr (Heights<MB, A_PW>::kHalf) {
    if (rows <= BM / 2) {
      body.template operator()<MB / 2>();
      return;
    }
  }
  body.template operator()<MB>();
}

// The MBE by_height picks for a tile of `rows` rows, at run time (a persistent kernel loads its
// next tile's e4m3 scales before it dispatches on that tile's height).
template <int BM, int MB, int A_PW>
__device__ __forceinline__ int mbe_of_rows(int rows) {
  if constexpr (Heights<MB, A_PW>::kQuarter)
    if (rows <= BM / 4) return MB / 4;
  if constexpr (Heights<MB, A_PW>::kHalf)
    if (rows <= BM / 2) return MB / 2;
  return MB;
}

// Per-lane A source offsets for the A_PW blocks of this wave (block i*NW + wave: rows 8 * that
// + lrow, clamped to the tile's last row), 16-byte chunks pre-swizzled; elem_bytes per element.
template <int A_PW, int NW>
__device__ __forceinline__ void a_offsets(const GemmArgs& p, const TileCoord& tc, int wave, int lane, int elem_bytes,
                                          uint32_t (&a_voff)[A_PW]) {
  const int lrow = lane >> 3;
#pragma unroll
  for (int i = 0; i < A_PW; ++i) {
    const int row = (i * NW + wave) * 8 + lrow;
    const int gr = min(tc.row0 + row, tc.row_end - 1);
    const long long src = p.a_rows ? static_cast<long long>(p.a_rows[gr]) : static_cast<long long>(gr);
    a_voff[i] = static_cast<uint32_t>(src * p.lda * elem_bytes + (((lane & 7) ^ swz(row)) << 4));
  }
}

// ---------------------------------------------------------------------------- bf16 (or fp32) weights: direct-to-LDS
// F32: fp32 A and B.  An LDS row is 128 bytes either way (64 bf16 or 32 fp32 of K per slab), so
// the DMA, the swizzle and the fragment reads are the same bytes; only the MFMA differs.
template <int BM, int BN, int WGM, int WGN, int EPI, int GM, bool F32 = false>
__global__ void __launch_bounds__(WGM * WGN * 64) grouped_gemm_dma_kernel(GemmArgs p) {
  using G = Geo<BM, BN, WGM, WGN, EPI>;
  constexpr int EB = F32 ? 4 : 2;             // bytes per element
  constexpr int BK = G::BK;
  constexpr int NW = G::NW;
  constexpr int A_PW = BM / 8 / G::NW;   // 1 KiB LDS blocks per wave per slab (8 rows each)
  constexpr int B_PW = BN / 8 / G::NW;
  static_assert(A_PW * 8 * G::NW == BM && B_PW * 8 * G::NW == BN, "slab split over waves");

  // The two LDS stages are distinct objects, and the loop below is unrolled by two so
  // the stage being read is known statically: alias analysis can then prove the DMA
  // into one stage does not touch the other, and the compiler does not wait for the
  // in-flight DMA before reading the current stage.
  __shared__ __attribute__((aligned(1024))) uint16_t sA0[BM * BK];
  __shared__ __attribute__((aligned(1024))) uint16_t sA1[BM * BK];
  __shared__ __attribute__((aligned(1024))) uint16_t sB0[BN * BK];
  __shared__ __attribute__((aligned(1024))) uint16_t sB1[BN * BK];
  __shared__ int s_pref[kMaxSeg + 1];

  TileCoord tc;
  if (!decode_tile<BM, G::OUT_BN, GM>(p, s_pref, tc)) return;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lrow = lane >> 3;                 // row of the lane inside an 8-row block
  const long long k0 = static_cast<long long>(tc.split) * p.K;

  // A: lane fetches logical chunk (lane&7)^(row&7) so LDS position == swizzled position.
  const BufRef rA{static_cast<const uint8_t*>(p.a) + k0 * EB, (p.a_rows_cap * p.lda - k0) * EB};
  uint32_t a_voff[A_PW];
  a_offsets<A_PW, NW>(p, tc, wave, lane, EB, a_voff);
  const uint8_t* b_base = expert_weights(p, tc.expert, EB) + k0 * EB;
  const BufRef rB{b_base, (p.b_estride - k0) * EB};
  uint32_t b_voff[B_PW];
#pragma unroll
  for (int i = 0; i < B_PW; ++i) {
    const int R = (wave * B_PW + i) * 8 + lrow;
    const int wr = G::weight_row_of_lds(R, tc.n_tile, p.up_off);
    b_voff[i] = static_cast<uint32_t>(static_cast<long long>(wr) * p.ldb * EB + (((lane & 7) ^ swz(R)) << 4));
  }

  const int wm = wave % WGM;
  const int wn = wave / WGM;
  const int KT = p.K * EB / (BK * 2);         // 128-byte slabs
  // weight DMA non-temporal: the launcher's choice, or this tile's segment is one m-tile (the only
  // reader of its weight panels)
  const bool b_nt = p.b_nt != 0 || tc.one_mt != 0;
  by_height<BM, G::MB, A_PW>(tc.row_end - tc.row0, [&]<int MBE>() {
    constexpr int A_CNT = A_PW * MBE / G::MB;
    f32x4_t acc[MBE][G::NB];
#pragma unroll
    for (int i = 0; i < MBE; ++i)
#pragma unroll
      for (int j = 0; j < G::NB; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    issue_slab_dma<A_CNT, B_PW, NW>(rA, rB, a_voff, b_voff, sA0, sB0, wave, 0, b_nt);
    __syncthreads();
    int kt = 0;
    // Slab kt is in buffer 0 at the top of each iteration.  The second load is unconditional
    // (on the last iteration of an even slab count it re-reads slab KT-1 into buffer 0, which is
    // not read again and which the closing barrier waits for) so that it is not split into its
    // own basic block, where the scheduler would queue the previous slab's MFMAs ahead of it.
    for (; kt + 1 < KT; kt += 2) {
      issue_slab_dma<A_CNT, B_PW, NW>(rA, rB, a_voff, b_voff, sA1, sB1, wave, (kt + 1) * BK * 2, b_nt);
      pin_issue();
      slab_mma<G, MBE, F32>(acc, sA0, sB0, wm, wn, lane);
      __syncthreads();
      issue_slab_dma<A_CNT, B_PW, NW>(rA, rB, a_voff, b_voff, sA0, sB0, wave, min(kt + 2, KT - 1) * BK * 2,
                                      b_nt);
      pin_issue();
      slab_mma<G, MBE, F32>(acc, sA1, sB1, wm, wn, lane);
      __syncthreads();
    }
    if (kt < KT) slab_mma<G, MBE, F32>(acc, sA0, sB0, wm, wn, lane);   // odd slab count: last slab in buffer 0
    epilogue<G, EPI, MBE>(p, tc, acc, wm, wn, lane, nullptr, nullptr);
  });
}

// ---------------------------------------------------------------------------- e4m3 fragments (W8A8)
// Both operands OCP e4m3fn on v_mfma_scale_f32_16x16x128_f8f6f4 (block scales fixed at
// 1.0; the per-row activation scale and per-output-channel weight scale are applied in
// the epilogue).  A 128-wide fp8 K slab is one 128-byte LDS row, so slab loading,
// swizzle and staging are those of the bf16 kernels.  Each lane feeds 32 bytes per
// operand: 16-byte chunks q and q+4 of its row (lane group q = lane/16); A and B use the
// same K assignment, so the K sum is exact whatever order the instruction adds.
__device__ __forceinline__ i32x8_t frag_fp8(const uint8_t* s, int R, int q) {
  const u32x4_t lo = *reinterpret_cast<const u32x4_t*>(&s[R * 128 + ((q ^ swz(R)) << 4)]);
  const u32x4_t hi = *reinterpret_cast<const u32x4_t*>(&s[R * 128 + (((q + 4) ^ swz(R)) << 4)]);
  return i32x8_t{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
}

__device__ __forceinline__ f32x4_t mfma_fp8(const i32x8_t& a, const i32x8_t& b, const f32x4_t& c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
}

// One 128-wide slab in two halves of the B fragments: the A fragments and half of the B
// fragments are live at once (64 VGPRs for the 256x256 tile, not 96).
template <class G, int MBE>
__device__ __forceinline__ void slab_mma_fp8(f32x4_t (&acc)[MBE][G::NB], const uint8_t* sA, const uint8_t* sB,
                                             int wm, int wn, int lane) {
  constexpr int NH = G::NB % 2 == 0 ? G::NB / 2 : G::NB;
  const int lr = lane & 15;
  const int q = lane >> 4;
  i32x8_t af[MBE];
#pragma unroll
  for (int i = 0; i < MBE; ++i) af[i] = frag_fp8(sA, wm * 16 * MBE + i * 16 + lr, q);
#pragma unroll
  for (int h = 0; h < G::NB; h += NH) {
    i32x8_t bfr[NH];
#pragma unroll
    for (int j = 0; j < NH; ++j) bfr[j] = frag_fp8(sB, wn * G::WN + (h + j) * 16 + lr, q);
#pragma unroll
    for (int i = 0; i < MBE; ++i)
#pragma unroll
      for (int j = 0; j < NH; ++j) acc[i][h + j] = mfma_fp8(af[i], bfr[j], acc[i][h + j]);
  }
}

// ---------------------------------------------------------------------------- bf16 ping-pong
// The 256x256 tile with its 8 waves in two groups of four, one wave of each group per SIMD
// (waves w and w + 4).  The groups run one phase apart: while one group multiplies the slab
// whose fragments it already holds in registers, the other reads its fragments of the same
// slab from LDS (and, in its first read phase of a slab, issues its share of the next slab's
// DMA), so each SIMD's MFMA pipe is fed by one wave while the other waits on LDS.  A phase
// is half a slab (32-wide K) and ends with a workgroup barrier; group 1 enters one phase late
// and group 0 adds one barrier at the end, so both groups execute 4*KT + 2 of them.  Same
// tiles, LDS layout and accumulation order as grouped_gemm_dma_kernel<256, 256, 4, 2>:
// bit-identical results, 3-4 % faster on the Mixtral-8x7B prefill GEMMs (MI355X) with two B
// stages; the third B stage below gains another 1-4 % there (A/B on one box: gate/up 3.31 ->
// 3.28 ms, down with K split 2 1.685 -> 1.645 ms, DeepSeek-V2-Lite 1-2 %).
// Workgroup barrier without a memory fence: a fence would wait for the DMA still in flight
// (it writes LDS).  The callers wait for what must be complete (lgkmcnt for their fragment
// reads, vmcnt for their DMA) explicitly; the asm's memory clobber keeps the compiler from
// moving LDS accesses across the barrier.
__device__ __forceinline__ void pp_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_barrier" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}
__device__ __forceinline__ void pp_wait_vm0() { __builtin_amdgcn_s_waitcnt(0x0F70); }     // vmcnt(0)
__device__ __forceinline__ void pp_wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xC07F); }   // lgkmcnt(0)

// ---------------------------------------------------------------------------- bf16: deeper LDS ring
// s_waitcnt vmcnt(N), the other counters untouched (gfx9 encoding: vmcnt bits 3:0 and 15:14).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

// Fragment reads of the ring kernel as inline ds_read_b128: the compiler's own waits for LDS DMA
// cannot tell the ring's stages apart (with a DMA in flight into another stage it waited for all of
// it before each read, whatever the barrier or the object layout), so the reads are hidden from it.
// One asm statement issues all of a slab's N reads and waits for them (lgkmcnt(0)), so nothing the
// compiler places between the reads and their use can see a register before its data has landed.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  typedef const __attribute__((address_space(3))) void* lds_cptr_t;
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_cptr_t)p));
}
template <int N>
__device__ __forceinline__ void lds_read_wait(const uint32_t (&a)[N], bf16x8_t (&f)[N]) {
  static_assert(N == 6 || N == 8 || N == 10 || N == 12 || N == 16, "fragment count of a ring slab");
  if constexpr (N == 6) {
    asm volatile("ds_read_b128 %0, %6\n ds_read_b128 %1, %7\n ds_read_b128 %2, %8\n ds_read_b128 %3, %9\n"
                 " ds_read_b128 %4, %10\n ds_read_b128 %5, %11\n s_waitcnt lgkmcnt(0)"
                 : "=&v"(f[0]), "=&v"(f[1]), "=&v"(f[2]), "=&v"(f[3]), "=&v"(f[4]), "=&v"(f[5])
                 : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(a[4]), "v"(a[5]));
  } else if constexpr (N == 8) {
    asm volatile("ds_read_b128 %0, %8\n ds_read_b128 %1, %9\n ds_read_b128 %2, %10\n ds_read_b128 %3, %11\n"
                 " ds_read_b128 %4, %12\n ds_read_b128 %5, %13\n ds_read_b128 %6, %14\n ds_read_b128 %7, %15\n"
                 " s_waitcnt lgkmcnt(0)"
                 : "=&v"(f[0]), "=&v"(f[1]), "=&v"(f[2]), "=&v"(f[3]), "=&v"(f[4]), "=&v"(f[5]), "=&v"(f[6]),
                   "=&v"(f[7])
                 : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(a[4]), "v"(a[5]), "v"(a[6]), "v"(a[7]));
  } else if constexpr (N == 10) {
    asm volatile("ds_read_b128 %0, %10\n ds_read_b128 %1, %11\n ds_read_b128 %2, %12\n ds_read_b128 %3, %13\n"
                 " ds_read_b128 %4, %14\n ds_read_b128 %5, %15\n ds_read_b128 %6, %16\n ds_read_b128 %7, %17\n"
                 " ds_read_b128 %8, %18\n ds_read_b128 %9, %19\n s_waitcnt lgkmcnt(0)"
                 : "=&v"(f[0]), "=&v"(f[1]), "=&v"(f[2]), "=&v"(f[3]), "=&v"(f[4]), "=&v"(f[5]), "=&v"(f[6]),
                   "=&v"(f[7]), "=&v"(f[8]), "=&v"(f[9])
                 : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(a[4]), "v"(a[5]), "v"(a[6]), "v"(a[7]),
                   "v"(a[8]), "v"(a[9]));
  } else if constexpr (N == 16) {
    asm volatile("ds_read_b128 %0, %16\n ds_read_b128 %1, %17\n ds_read_b128 %2, %18\n ds_read_b128 %3, %19\n"
                 " ds_read_b128 %4, %20\n ds_read_b128 %5, %21\n ds_read_b128 %6, %22\n ds_read_b128 %7, %23\n"
                 " ds_read_b128 %8, %24\n ds_read_b128 %9, %25\n ds_read_b128 %10, %26\n ds_read_b128 %11, %27\n"
                 " ds_read_b128 %12, %28\n ds_read_b128 %13, %29\n ds_read_b128 %14, %30\n ds_read_b128 %15, %31\n"
                 " s_waitcnt lgkmcnt(0)"
                 : "=&v"(f[0]), "=&v"(f[1]), "=&v"(f[2]), "=&v"(f[3]), "=&v"(f[4]), "=&v"(f[5]), "=&v"(f[6]),
                   "=&v"(f[7]), "=&v"(f[8]), "=&v"(f[9]), "=&v"(f[10]), "=&v"(f[11]), "=&v"(f[12]), "=&v"(f[13]),
                   "=&v"(f[14]), "=&v"(f[15])
                 : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(a[4]), "v"(a[5]), "v"(a[6]), "v"(a[7]),
                   "v"(a[8]), "v"(a[9]), "v"(a[10]), "v"(a[11]), "v"(a[12]), "v"(a[13]), "v"(a[14]), "v"(a[15]));
  } else {
    asm volatile("ds_read_b128 %0, %12\n ds_read_b128 %1, %13\n ds_read_b128 %2, %14\n ds_read_b128 %3, %15\n"
                 " ds_read_b128 %4, %16\n ds_read_b128 %5, %17\n ds_read_b128 %6, %18\n ds_read_b128 %7, %19\n"
                 " ds_read_b128 %8, %20\n ds_read_b128 %9, %21\n ds_read_b128 %10, %22\n ds_read_b128 %11, %23\n"
                 " s_waitcnt lgkmcnt(0)"
                 : "=&v"(f[0]), "=&v"(f[1]), "=&v"(f[2]), "=&v"(f[3]), "=&v"(f[4]), "=&v"(f[5]), "=&v"(f[6]),
                   "=&v"(f[7]), "=&v"(f[8]), "=&v"(f[9]), "=&v"(f[10]), "=&v"(f[11])
                 : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(a[4]), "v"(a[5]), "v"(a[6]), "v"(a[7]),
                   "v"(a[8]), "v"(a[9]), "v"(a[10]), "v"(a[11]));
  }
}

// LDS byte addresses of a slab's fragments (both K halves: A then B of half 0, then of half 1), as
// read_frags addresses them.
template <class G, int MBE>
__device__ __forceinline__ void ring_frag_addrs(uint32_t aA, uint32_t aB, int wm, int wn, int lane,
                                                uint32_t (&ad)[2 * (MBE + G::NB)]) {
  const int lr = lane & 15;
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) {
    const int c = kk * 4 + (lane >> 4);
#pragma unroll
    for (int i = 0; i < MBE; ++i) {
      const int R = wm * 16 * MBE + i * 16 + lr;
      ad[kk * (MBE + G::NB) + i] = aA + 2 * (R * G::BK + ((c ^ swz(R)) << 3));
    }
#pragma unroll
    for (int j = 0; j < G::NB; ++j) {
      const int R = wn * G::WN + j * 16 + lr;
      ad[kk * (MBE + G::NB) + MBE + j] = aB + 2 * (R * G::BK + ((c ^ swz(R)) << 3));
    }
  }
}

// grouped_gemm_dma_kernel on a ring of NS LDS stages: NS - 1 slabs in flight per workgroup instead
// of one.  The two-stage loop's __syncthreads() fences wait for every DMA in flight at each slab
// end; here each slab ends waiting for its wave's next slab only (loads complete in issue order)
// and a barrier without a fence publishes it.  Same tiles, LDS layout per stage and accumulation
// order: bit-identical results.  For launches whose tiles fit the GPU at the ring's occupancy.
template <int BM, int BN, int WGM, int WGN, int EPI, int GM, int NS>
__global__ void __launch_bounds__(WGM * WGN * 64) grouped_gemm_ring_kernel(GemmArgs p) {
  static_assert(NS == 3, "three stages");
  using G = Geo<BM, BN, WGM, WGN, EPI>;
  constexpr int EB = 2;
  constexpr int BK = G::BK;
  constexpr int NW = G::NW;
  constexpr int A_PW = BM / 8 / G::NW;
  constexpr int B_PW = BN / 8 / G::NW;
  static_assert(A_PW * 8 * G::NW == BM && B_PW * 8 * G::NW == BN, "slab split over waves");
  // One object per stage (A then B), read with static indices, so alias analysis proves that the
  // DMA into one stage does not touch the one being read (with a separate object per operand and
  // stage, nine in all, the compiler waited for the DMA just issued before every fragment read).
  struct Stage {
    uint16_t a[BM * BK];
    uint16_t b[BN * BK];
  };
  __shared__ __attribute__((aligned(1024))) Stage t0;
  __shared__ __attribute__((aligned(1024))) Stage t1;
  __shared__ __attribute__((aligned(1024))) Stage t2;
  __shared__ int s_pref[kMaxSeg + 1];

  TileCoord tc;
  if (!decode_tile<BM, G::OUT_BN, GM>(p, s_pref, tc)) return;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lrow = lane >> 3;
  const long long k0 = static_cast<long long>(tc.split) * p.K;
  const BufRef rA{static_cast<const uint8_t*>(p.a) + k0 * EB, (p.a_rows_cap * p.lda - k0) * EB};
  uint32_t a_voff[A_PW];
  a_offsets<A_PW, NW>(p, tc, wave, lane, EB, a_voff);
  const uint8_t* b_base = expert_weights(p, tc.expert, EB) + k0 * EB;
  const BufRef rB{b_base, (p.b_estride - k0) * EB};
  uint32_t b_voff[B_PW];
#pragma unroll
  for (int i = 0; i < B_PW; ++i) {
    const int R = (wave * B_PW + i) * 8 + lrow;
    const int wr = G::weight_row_of_lds(R, tc.n_tile, p.up_off);
    b_voff[i] = static_cast<uint32_t>(static_cast<long long>(wr) * p.ldb * EB + (((lane & 7) ^ swz(R)) << 4));
  }
  const int wm = wave % WGM;
  const int wn = wave / WGM;
  const int KT = p.K * EB / (BK * 2);
  const bool b_nt = p.b_nt != 0 || tc.one_mt != 0;
  by_height<BM, G::MB, A_PW>(tc.row_end - tc.row0, [&]<int MBE>() {
    constexpr int A_CNT = A_PW * MBE / G::MB;
    constexpr int L = A_CNT + B_PW;   // DMA instructions per slab per wave
    f32x4_t acc[MBE][G::NB];
#pragma unroll
    for (int i = 0; i < MBE; ++i)
#pragma unroll
      for (int j = 0; j < G::NB; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    // slabs 0 and 1 into stages 0 and 1 (clamped to the last slab: stages not read again)
    issue_slab_dma<A_CNT, B_PW, NW>(rA, rB, a_voff, b_voff, t0.a, t0.b, wave, 0, b_nt);
    issue_slab_dma<A_CNT, B_PW, NW>(rA, rB, a_voff, b_voff, t1.a, t1.b, wave, min(1, KT - 1) * BK * 2, b_nt);
    wait_vm<(NS - 2) * L>();   // this wave's slab 0
    pp_barrier();
    // slab kt + J: read stage J, load slab kt + J + NS - 1 into the stage slab kt + J - 1 read (every
    // wave finished reading it before the barrier that ended that slab).
    // The slab's DMA goes first, then its fragment reads and their wait (lds_read_wait), its MFMAs, and
    // the wait for the next slab's data.
#define EIMOE_RING_SLAB(J, SA, SB, SAN, SBN)                                                                \
  if (kt + J < KT) {                                                                                        \
    issue_slab_dma<A_CNT, B_PW, NW>(rA, rB, a_voff, b_voff, SAN, SBN, wave, min(kt + J + NS - 1, KT - 1) * BK * 2, \
                                    b_nt);                                                                  \
    uint32_t ad[2 * (MBE + G::NB)];                                                                         \
    ring_frag_addrs<G, MBE>(lds_addr(SA), lds_addr(SB), wm, wn, lane, ad);                                  \
    bf16x8_t fr[2 * (MBE + G::NB)];                                                                         \
    lds_read_wait(ad, fr);                                                                                  \
    mma<G, MBE>(acc, *reinterpret_cast<bf16x8_t(*)[MBE]>(fr), *reinterpret_cast<bf16x8_t(*)[G::NB]>(fr + MBE)); \
    mma<G, MBE>(acc, *reinterpret_cast<bf16x8_t(*)[MBE]>(fr + MBE + G::NB),                                 \
                *reinterpret_cast<bf16x8_t(*)[G::NB]>(fr + 2 * MBE + G::NB));                               \
    wait_vm<(NS - 2) * L>();                                                                                \
    pp_barrier();                                                                                           \
  }
    for (int kt = 0; kt < KT; kt += NS) {
      EIMOE_RING_SLAB(0, t0.a, t0.b, t2.a, t2.b)
      EIMOE_RING_SLAB(1, t1.a, t1.b, t0.a, t0.b)
      EIMOE_RING_SLAB(2, t2.a, t2.b, t1.a, t1.b)
    }
#undef EIMOE_RING_SLAB
    pp_wait_vm0();   // the clamped loads near the end land before the workgroup's LDS is released
    epilogue<G, EPI, MBE>(p, tc, acc, wm, wn, lane, nullptr, nullptr);
  });
}

// ---------------------------------------------------------------------------- ping-pong, three B stages (bf16 or e4m3)
// The ping-pong kernel with the weight panel (B, the operand streamed from HBM) fetched two slabs
// ahead: A in two stages, B in three, 5 x 32 KiB = the whole 160 KiB of LDS (the segment prefix
// lives in the third B stage until that stage's first load).  Each wave issues A(kt+1) at the top
// of its first phase of slab kt and B(kt+2) at the top of its second: issuing both in one phase
// made that phase longer than the other group's multiply (the ping-pong's MFMA-idle gap; moving B
// to the second phase took the Mixtral-8x7B prefill layer from 4.84 to 4.43 ms, A/B on one box).
// The slab ends waiting for all but the last B_PW loads of the wave (vmcnt(4): loads complete in
// issue order), so A(kt+1) and B(kt+1) have landed and B(kt+2) may still be in flight.  Unrolled by
// six so every stage index is static.
__device__ __forceinline__ void pp_wait_vm4() { __builtin_amdgcn_s_waitcnt(0x0F74); }   // vmcnt(4)

// BAUX: cache-policy bits of the weight loads (2: non-temporal).
template <int A_CNT, int B_PW, int NW, int A_PW, int BAUX = 0>
__device__ __forceinline__ void issue_ab_dma(const BufRef& a, const BufRef& b, const uint32_t (&a_voff)[A_PW],
                                             const uint32_t (&b_voff)[B_PW], uint16_t* sA, uint16_t* sB, int wave,
                                             int soff_a, int soff_b) {
#if defined(__HIP_DEVICE_COMPILE__)
  const auto rA = make_rsrc(a.base, a.bytes);
  const auto rB = make_rsrc(b.base, b.bytes);
#pragma unroll
  for (int i = 0; i < A_CNT; ++i)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rA, (lds_void_t*)(sA + (i * NW + wave) * 512), 16, a_voff[i], soff_a,
                                             0, 0);
#pragma unroll
  for (int i = 0; i < B_PW; ++i)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rB, (lds_void_t*)(sB + (wave * B_PW + i) * 512), 16, b_voff[i], soff_b,
                                             0, BAUX);
#endif
}

// Phases of the ping-pong loop.  bf16: phase KK reads the A and B fragments of K half KK (32
// wide) and runs MBE x NB MFMAs.  e4m3 (one 16x16x128 MFMA covers a 128-byte row): phase 0
// reads the A fragments and the first half of the B fragments, phase 1 the other half of B,
// and each runs MBE x NB/2 MFMAs of twice the bf16 MFMA's cycles, so a phase is the same MFMA
// time either way and the live fragments stay at 64 VGPRs.
template <bool FP8, class G, int MBE>
struct PpFrags;
template <class G, int MBE>
struct PpFrags<false, G, MBE> {
  bf16x8_t a[MBE], b[G::NB];
};
template <class G, int MBE>
struct PpFrags<true, G, MBE> {
  i32x8_t a[MBE], b[G::NB / 2];
};

template <bool FP8, class G, int MBE, int KK>
__device__ __forceinline__ void pp_read(PpFrags<FP8, G, MBE>& f, const uint16_t* sA, const uint16_t* sB, int wm,
                                        int wn, int lane) {
  if constexpr (!FP8) {
    read_frags<G, MBE>(sA, sB, KK, wm, wn, lane, f.a, f.b);
  } else {
    const int lr = lane & 15;
    const int q = lane >> 4;
    if constexpr (KK == 0) {
#pragma unroll
      for (int i = 0; i < MBE; ++i)
        f.a[i] = frag_fp8(reinterpret_cast<const uint8_t*>(sA), wm * 16 * MBE + i * 16 + lr, q);
    }
#pragma unroll
    for (int j = 0; j < G::NB / 2; ++j)
      f.b[j] = frag_fp8(reinterpret_cast<const uint8_t*>(sB), wn * G::WN + (KK * G::NB / 2 + j) * 16 + lr, q);
  }
}

template <bool FP8, class G, int MBE, int KK>
__device__ __forceinline__ void pp_mma(f32x4_t (&acc)[MBE][G::NB], const PpFrags<FP8, G, MBE>& f) {
  if constexpr (!FP8) {
    mma<G, MBE>(acc, f.a, f.b);
  } else {
#pragma unroll
    for (int i = 0; i < MBE; ++i)
#pragma unroll
      for (int j = 0; j < G::NB / 2; ++j)
        acc[i][KK * G::NB / 2 + j] = mfma_fp8(f.a[i], f.b[j], acc[i][KK * G::NB / 2 + j]);
    // Phase 0's accumulators are not read again until the next slab, and the machine sinking
    // pass would move their MFMAs past the phase barrier into phase 1 (measured: all 32 MFMAs
    // of a slab then run in one phase).  An empty asm that takes them as operands keeps them here.
    if constexpr (KK == 0) {
#pragma unroll
      for (int i = 0; i < MBE; ++i)
#pragma unroll
        for (int j = 0; j < G::NB / 2; ++j) asm volatile("" ::"v"(acc[i][j]));
    }
  }
}

// The five LDS stages of the ping-pong kernels: A in two, B in three (5 x 32 KiB).
struct PpStages {
  uint16_t *a0, *a1, *b0, *b1, *b2;
};

// Operand windows and per-lane B offsets of one 256x256 ping-pong tile; EB bytes per weight, EA
// per activation (bf16 activations against e4m3 weights in W8A16).
template <class G, int EB, int FR = 16, int EA = EB>
struct PpOperands {
  static constexpr int B_PW = 256 / 8 / G::NW;
  BufRef rA, rB;
  uint32_t b_voff[B_PW];
  __device__ __forceinline__ PpOperands(const GemmArgs& p, const TileCoord& tc, int wave, int lane) {
    const long long k0 = static_cast<long long>(tc.split) * p.K;
    // uniform by construction, taken from the first lane so that the compiler keeps them in
    // SGPRs: in the persistent kernel's tile loop it could not prove it and wrapped every
    // buffer load in a readfirstlane loop (measured: MFMA busy 63 % against 79 %)
    rA = BufRef{uniform(static_cast<const uint8_t*>(p.a) + k0 * EA), uniform((p.a_rows_cap * p.lda - k0) * EA)};
    rB = BufRef{uniform(expert_weights(p, tc.expert, EB) + k0 * EB), uniform((p.b_estride - k0) * EB)};
#pragma unroll
    for (int i = 0; i < B_PW; ++i) {
      const int R = (wave * B_PW + i) * 8 + (lane >> 3);
      const int wr = G::weight_row_of_lds(R, tc.n_tile, p.up_off);
      b_voff[i] = static_cast<uint32_t>(static_cast<long long>(wr) * p.ldb * EB + (((lane & 7) ^ swz(R)) << 4));
    }
  }
};

// The K loop of one tile, from the first slab's data in (A0, B0) and B of the second slab in B1
// (waited for and published by the caller's barrier) to every wave's last LDS read.  Group 1
// enters one phase late; both groups execute 4*KT + 2 barriers including the caller's one.
// FP8: e4m3 activations and weights (W8A8); an LDS row is 128 bytes either way (64 bf16 or 128
// e4m3 of K per slab), so the DMA, the swizzle and the stages are the same bytes.
template <bool FP8, class G, int MBE, int A_CNT, int A_PW, int B_PW, int BAUX = 0>
__device__ __forceinline__ void pp3_kloop(f32x4_t (&acc)[MBE][G::NB], const BufRef& rA, const BufRef& rB,
                                          const uint32_t (&a_voff)[A_PW], const uint32_t (&b_voff)[B_PW], int KT,
                                          int wave, int lane, const PpStages& st) {
  constexpr int BK = G::BK;
  constexpr int NW = G::NW;
  const int grp = wave >> 2;
  const int wm = wave % 4;
  const int wn = wave / 4;
  uint16_t* const sA0 = st.a0;
  uint16_t* const sA1 = st.a1;
  uint16_t* const sB0 = st.b0;
  uint16_t* const sB1 = st.b1;
  uint16_t* const sB2 = st.b2;
  if (grp == 1) pp_barrier();
  PpFrags<FP8, G, MBE> fr;
  // The phase's DMA goes ahead of its fragment reads for bf16, after them for e4m3 (A/B on one
  // box: bf16 prefill 4.47 vs 4.50 ms; W8A8 prefill 2.76 vs 2.65 ms).
#define EIMOE_PP3_HALF(SA, SB, KK, DMA)                   \
  if constexpr (!FP8) DMA;                                \
  pp_read<FP8, G, MBE, KK>(fr, SA, SB, wm, wn, lane);     \
  if constexpr (FP8) {                                    \
    pin_issue();                                          \
    DMA;                                                  \
    pin_issue();                                          \
  }                                                       \
  pp_wait_lgkm0();                                        \
  if (KK == 1 && grp == 1) pp_wait_vm4();                 \
  pp_barrier();                                           \
  pp_mma<FP8, G, MBE, KK>(acc, fr);                       \
  if (KK == 1 && grp == 0) pp_wait_vm4();                 \
  pp_barrier();
  // slab kt + J: read (SA, SB); load A(kt+J+1) into SAN and B(kt+J+2) into SBN (clamped to
  // the last slab near the end: those stages are not read again)
#define EIMOE_PP3_SLAB(J, SA, SB, SAN, SBN)                                                              \
  if (kt + J < KT) {                                                                                     \
    EIMOE_PP3_HALF(SA, SB, 0, (issue_a_dma<A_CNT, NW>(rA, a_voff, SAN, wave, min(kt + J + 1, KT - 1) * BK * 2))) \
    EIMOE_PP3_HALF(SA, SB, 1,                                                                            \
                   (issue_ab_dma<0, B_PW, NW, A_PW, BAUX>(rA, rB, a_voff, b_voff, SAN, SBN, wave, 0,      \
                                                          min(kt + J + 2, KT - 1) * BK * 2)))            \
  }
  for (int kt = 0; kt < KT; kt += 6) {
    EIMOE_PP3_SLAB(0, sA0, sB0, sA1, sB2)
    EIMOE_PP3_SLAB(1, sA1, sB1, sA0, sB0)
    EIMOE_PP3_SLAB(2, sA0, sB2, sA1, sB1)
    EIMOE_PP3_SLAB(3, sA1, sB0, sA0, sB2)
    EIMOE_PP3_SLAB(4, sA0, sB1, sA1, sB0)
    EIMOE_PP3_SLAB(5, sA1, sB2, sA0, sB1)
  }
#undef EIMOE_PP3_SLAB
#undef EIMOE_PP3_HALF
  if (grp == 0) pp_barrier();   // matches group 1's late start: every wave has read its last slab
}

// Eight e4m3 weights (two 32-bit words, bytes in k order) widened to bf16 with gfx950's
// v_cvt_scalef32_pk_bf16_fp8 at scale 1: exact (e4m3 values are bf16 values), and bit-identical to
// widening through fp32 on all 65536 byte pairs (NaNs included; compared on gfx950).
__device__ __forceinline__ bf16x8_t widen_fp8x8(uint32_t w0, uint32_t w1) {
  const bf16x2_t a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(static_cast<int>(w0), 1.0f, false);
  const bf16x2_t b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(static_cast<int>(w0), 1.0f, true);
  const bf16x2_t c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(static_cast<int>(w1), 1.0f, false);
  const bf16x2_t d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(static_cast<int>(w1), 1.0f, true);
  return bf16x8_t{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// The K loop of the W8A16 ping-pong tile: bf16 activations against e4m3 weights on the bf16 MFMA.
// A stage is a 64-wide k slab of activations (128-byte rows of bf16, as for bf16); a B stage holds
// 128 k of weights (128-byte rows of e4m3), so weight chunk c serves slabs 2c and 2c+1 and its DMA
// runs every other slab: chunk c+2 goes out in the second phase of slab 2c+1, into the stage of
// chunk c-1.  Within a slab lane group q takes k = 16q + 8*KK + (0..7) in phase KK (every k once):
// its activation fragment is chunk 2q+KK of the row, and one 16-byte weight read per slab in phase
// 0 (chunk 4*(slab%2) + q) covers both phases, widened half by half.  So each slab reads 16 1-KiB
// LDS blocks per wave instead of 24 and fetches half the weight bytes.  Slab ends wait for all but
// the latest B DMA after an odd slab (vmcnt(4)), for everything after an even one (the chunk issued
// a slab earlier is then complete 1.5 slabs after its issue, as the bf16 loop's B).  K % 128 == 0.
template <class G, int MBE, int A_CNT, int A_PW, int B_PW>
__device__ __forceinline__ void pp3w_kloop(f32x4_t (&acc)[MBE][G::NB], const BufRef& rA, const BufRef& rB,
                                           const uint32_t (&a_voff)[A_PW], const uint32_t (&b_voff)[B_PW], int KT,
                                           int wave, int lane, const PpStages& st) {
  constexpr int NW = G::NW;
  const int grp = wave >> 2;
  const int wm = wave % 4;
  const int wn = wave / 4;
  const int lr = lane & 15;
  const int q = lane >> 4;
  const int NC = KT / 2;   // 128-k weight chunks
  uint16_t* const sA0 = st.a0;
  uint16_t* const sA1 = st.a1;
  uint16_t* const sB0 = st.b0;
  uint16_t* const sB1 = st.b1;
  uint16_t* const sB2 = st.b2;
  if (grp == 1) pp_barrier();
  bf16x8_t af[MBE], bw[G::NB];
  u32x4_t braw[G::NB];
  auto read_a = [&](const uint16_t* sA, int KK) {
#pragma unroll
    for (int i = 0; i < MBE; ++i) {
      const int R = wm * 16 * MBE + i * 16 + lr;
      af[i] = *reinterpret_cast<const bf16x8_t*>(&sA[R * G::BK + (((2 * q + KK) ^ swz(R)) << 3)]);
    }
  };
  auto read_b = [&](const uint16_t* sB, int half) {
    const uint8_t* b8 = reinterpret_cast<const uint8_t*>(sB);
#pragma unroll
    for (int j = 0; j < G::NB; ++j) {
      const int R = wn * G::WN + j * 16 + lr;
      braw[j] = *reinterpret_cast<const u32x4_t*>(&b8[R * 128 + (((4 * half + q) ^ swz(R)) << 4)]);
    }
  };
  auto widen = [&](int KK) {
#pragma unroll
    for (int j = 0; j < G::NB; ++j) bw[j] = widen_fp8x8(braw[j][2 * KK], braw[j][2 * KK + 1]);
  };
  // slab kt + J reads activations from SA and weights from SB (its chunk's stage); loads A(kt+J+1)
  // into SAN and, for odd J, weight chunk (kt+J)/2 + 2 into SBN (clamped near the end: those
  // stages are not read again)
#define EIMOE_PPW_SLAB(J, SA, SB, SAN, SBN)                                                          \
  if (kt + J < KT) {                                                                                 \
    issue_a_dma<A_CNT, NW>(rA, a_voff, SAN, wave, min(kt + J + 1, KT - 1) * 128);                    \
    read_a(SA, 0);                                                                                   \
    read_b(SB, J % 2);                                                                               \
    pp_wait_lgkm0();                                                                                 \
    widen(0);                                                                                        \
    pp_barrier();                                                                                    \
    mma<G, MBE>(acc, af, bw);                                                                        \
    pp_barrier();                                                                                    \
    if (J % 2 == 1)                                                                                  \
      issue_ab_dma<0, B_PW, NW>(rA, rB, a_voff, b_voff, SAN, SBN, wave, 0,                           \
                                min((kt + J) / 2 + 2, NC - 1) * 128);                                \
    read_a(SA, 1);                                                                                   \
    widen(1);                                                                                        \
    pp_wait_lgkm0();                                                                                 \
    if (grp == 1) {                                                                                  \
      if (J % 2 == 1) pp_wait_vm4();                                                                 \
      else pp_wait_vm0();                                                                            \
    }                                                                                                \
    pp_barrier();                                                                                    \
    mma<G, MBE>(acc, af, bw);                                                                        \
    if (grp == 0) {                                                                                  \
      if (J % 2 == 1) pp_wait_vm4();                                                                 \
      else pp_wait_vm0();                                                                            \
    }                                                                                                \
    pp_barrier();                                                                                    \
  }
  for (int kt = 0; kt < KT; kt += 6) {
    EIMOE_PPW_SLAB(0, sA0, sB0, sA1, sB2)
    EIMOE_PPW_SLAB(1, sA1, sB0, sA0, sB2)
    EIMOE_PPW_SLAB(2, sA0, sB1, sA1, sB0)
    EIMOE_PPW_SLAB(3, sA1, sB1, sA0, sB0)
    EIMOE_PPW_SLAB(4, sA0, sB2, sA1, sB1)
    EIMOE_PPW_SLAB(5, sA1, sB2, sA0, sB1)
  }
#undef EIMOE_PPW_SLAB
  if (grp == 0) pp_barrier();   // matches group 1's late start: every wave has read its last slab
}

// Pins values in registers at this point (an empty asm that takes them as operands): loads
// issued early then complete here instead of being sunk by the compiler to their first use.
template <class G, int MBE>
__device__ __forceinline__ void pin_scales(EpiScales<G, MBE>& sc) {
  for (auto& x : sc.cs) asm volatile("" ::"v"(x));
  for (auto& x : sc.cs_up) asm volatile("" ::"v"(x));
  for (auto& row : sc.rs)
    for (auto& x : row) asm volatile("" ::"v"(x));
}

template <int EPI, int GM, bool FP8 = false>
__global__ void __launch_bounds__(512) grouped_gemm_pp3_kernel(GemmArgs p) {
  using G = Geo<256, 256, 4, 2, EPI>;
  constexpr int BK = G::BK;
  constexpr int EB = FP8 ? 1 : 2;             // bytes per element
  constexpr int NW = G::NW;
  constexpr int A_PW = 256 / 8 / G::NW;
  constexpr int B_PW = 256 / 8 / G::NW;
  static_assert(B_PW == 4, "the slab-end wait is vmcnt(B_PW)");
  static_assert(!FP8 || G::NB % 2 == 0, "e4m3 phases split the B fragments in two");
  static_assert((kMaxSeg + 1) * sizeof(int) <= 256 * BK * sizeof(uint16_t), "segment prefix fits a B stage");
  __shared__ __attribute__((aligned(1024))) uint16_t sA0[256 * BK];
  __shared__ __attribute__((aligned(1024))) uint16_t sA1[256 * BK];
  __shared__ __attribute__((aligned(1024))) uint16_t sB0[256 * BK];
  __shared__ __attribute__((aligned(1024))) uint16_t sB1[256 * BK];
  __shared__ __attribute__((aligned(1024))) uint16_t sB2[256 * BK];
  const PpStages st{sA0, sA1, sB0, sB1, sB2};

  TileCoord tc;
  if (!decode_tile<256, G::OUT_BN, GM>(p, reinterpret_cast<int*>(sB2), tc)) return;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  uint32_t a_voff[A_PW];
  a_offsets<A_PW, NW>(p, tc, wave, lane, EB, a_voff);
  const PpOperands<G, EB> op(p, tc, wave, lane);
  const float* scale = FP8 ? p.b_scale + static_cast<long long>(tc.expert) * p.nb_rows : nullptr;

  const int wm = wave % 4;
  const int wn = wave / 4;
  const int KT = p.K * EB / (BK * 2);        // 128-byte slabs
  by_height<256, G::MB, A_PW>(tc.row_end - tc.row0, [&]<int MBE>() {
    constexpr int A_CNT = A_PW * MBE / G::MB;
    f32x4_t acc[MBE][G::NB];
#pragma unroll
    for (int i = 0; i < MBE; ++i)
#pragma unroll
      for (int j = 0; j < G::NB; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    // e4m3: the epilogue's scales are loaded here, around the first slab's DMA, instead of after
    // the K loop (the activation scale is two dependent loads, row map then scale, ~5 us of a
    // ~60 us tile at the epilogue): the row map before the DMA, the scales after it, so their
    // round trip overlaps the DMA's.  24 VGPRs held through the loop.
    EpiScales<G, MBE> sc;
    int src_row[MBE][4];
    if constexpr (FP8) epi_load_scales_1<G, MBE>(p, tc, wm, wn, lane, scale, p.a_scale, sc, src_row);
    // slab 0 into (A0, B0), B of slab 1 into B1 (the prefix in B2 is no longer read: every
    // thread finished decode_tile before the barrier below, and B2's first load comes after it)
    issue_ab_dma<A_CNT, B_PW, NW>(op.rA, op.rB, a_voff, op.b_voff, sA0, sB0, wave, 0, 0);
    issue_ab_dma<0, B_PW, NW>(op.rA, op.rB, a_voff, op.b_voff, sA0, sB1, wave, 0, min(1, KT - 1) * BK * 2);
    if constexpr (FP8) epi_load_scales_2<G, MBE>(p.a_scale, sc, src_row);
    pp_wait_vm0();
    if constexpr (FP8) pin_scales(sc);   // the compiler would otherwise sink the loads to their use
    pp_barrier();
    pp3_kloop<FP8, G, MBE, A_CNT>(acc, op.rA, op.rB, a_voff, op.b_voff, KT, wave, lane, st);
    pp_wait_vm0();                // the clamped loads near the end land before the LDS is released
    if constexpr (FP8) epilogue<G, EPI, MBE>(p, tc, acc, wm, wn, lane, sc);
    else epilogue<G, EPI, MBE>(p, tc, acc, wm, wn, lane, nullptr, nullptr);
  });
}

// The ping-pong kernel as a persistent loop over tiles, for launches of at most 64 segments.
// One workgroup per CU (the LDS allows no more); workgroup b walks the tiles b / 8, b / 8 +
// grid / 8, ... of XCD b % 8's share, the XCD-major order of the one-tile-per-workgroup launch,
// so the tiles running at one time on an XCD still share weight panels in its L2.  Per tile the
// one-tile-per-workgroup kernel spends ~1.5 us decoding the schedule, ~2.5 us waiting for its
// first slabs and ~1.7 us between workgroups (timestamped per tile on the Mixtral-8x7B
// prefill); here the schedule lives in registers (reg_sched), the next tile's row map is
// loaded during the first slab of the current one, and the next tile's first DMA (and e4m3
// scales) is issued before the current tile's epilogue, into each wave's own LDS blocks, which
// no wave reads any more once the K loop's last barrier has passed.  Every workgroup's loop is
// bounded by its share of the tiles.  Same tiles, DMA and accumulation order as
// grouped_gemm_pp3_kernel: bit-identical results.
// MODE: 0 bf16 x bf16, 1 W8A8 (e4m3 x e4m3 on the fp8 MFMA), 2 W8A16 (bf16 activations x e4m3
// weights on the bf16 MFMA, pp3w_kloop; K % 128 == 0).
template <int EPI, int GM, int MODE = 0>
__global__ void __launch_bounds__(512) grouped_gemm_pp3p_kernel(GemmArgs p) {
  using G = Geo<256, 256, 4, 2, EPI>;
  constexpr int BK = G::BK;
  constexpr bool FP8 = MODE == 1;    // e4m3 activations and weights
  constexpr bool WFP8 = MODE != 0;   // e4m3 weights (per-channel scales)
  constexpr int EB = WFP8 ? 1 : 2;   // bytes per weight
  constexpr int EA = FP8 ? 1 : 2;    // bytes per activation
  constexpr int NW = G::NW;
  constexpr int A_PW = 256 / 8 / G::NW;
  constexpr int B_PW = 256 / 8 / G::NW;
  constexpr int MB = G::MB;
  static_assert(B_PW == 4, "the slab-end wait is vmcnt(B_PW)");
  __shared__ __attribute__((aligned(1024))) uint16_t sA0[256 * BK];
  __shared__ __attribute__((aligned(1024))) uint16_t sA1[256 * BK];
  __shared__ __attribute__((aligned(1024))) uint16_t sB0[256 * BK];
  __shared__ __attribute__((aligned(1024))) uint16_t sB1[256 * BK];
  __shared__ __attribute__((aligned(1024))) uint16_t sB2[256 * BK];
  const PpStages st{sA0, sA1, sB0, sB1, sB2};

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave % 4;
  const int wn = wave / 4;
  const int KT = p.K * EA / (BK * 2);        // 128-byte activation slabs
  const int B1 = MODE == 2 ? min(1, KT / 2 - 1) : min(1, KT - 1);   // the B stage loaded second
  const RegSched rsch = reg_sched<256, G::OUT_BN>(p, lane);
  const int xcd = blockIdx.x % kNumXcd;
  const int stride = gridDim.x / kNumXcd;   // the launch rounds the grid to whole XCD rounds
  auto logical_of = [&](int sl) { return sl < rsch.per_xcd ? xcd * rsch.per_xcd + sl : rsch.total; };
  int slot = blockIdx.x / kNumXcd;
  TileCoord tc;
  if (!reg_decode<256, GM>(p, rsch, logical_of(slot), tc)) return;
  // A short tile (a quarter or half of the rows) of a segment that is a single m-tile is the only
  // reader of its weight panels: its weight DMA takes the non-temporal hint, as the LDS-tiled
  // kernels' decode launches do (bf16 and W8A8; the W8A16 loop stages its weights elsewhere).
  // A/B on one box, with the LDS-tiled kernels' per-tile hint: layers timed back to back, Qwen3-30B-A3B
  // share at 2048 tokens (28 of its 32 experts one short tile each) 0.138 -> 0.126 ms and
  // DeepSeek-V2-Lite at 768 / 4096 tokens 0.327 -> 0.295 / 0.669 -> 0.649 ms; after a 512 MB write
  // (dirty lines in the last-level cache) 9-16 % and 4-5 % faster; after a 512 MB read within 1 %.
  // Full-height single tiles with the hint as well measured the same.
  auto nt_tile = [&](const TileCoord& t) {
    return MODE != 2 && t.one_mt != 0 && mbe_of_rows<256, MB, A_PW>(t.row_end - t.row0) < MB;
  };
  // A tile's first DMA: slab 0 of A and B, B of slab 1 (the K loop loads the rest).
  auto first_dma = [&](const PpOperands<G, EB, 16, EA>& o, const uint32_t (&av)[A_PW], bool nt) {
    if (nt) {
      issue_ab_dma<A_PW, B_PW, NW, A_PW, 2>(o.rA, o.rB, av, o.b_voff, sA0, sB0, wave, 0, 0);
      issue_ab_dma<0, B_PW, NW, A_PW, 2>(o.rA, o.rB, av, o.b_voff, sA0, sB1, wave, 0, B1 * BK * 2);
    } else {
      issue_ab_dma<A_PW, B_PW, NW>(o.rA, o.rB, av, o.b_voff, sA0, sB0, wave, 0, 0);
      issue_ab_dma<0, B_PW, NW>(o.rA, o.rB, av, o.b_voff, sA0, sB1, wave, 0, B1 * BK * 2);
    }
  };

  // first tile: its row map, scales and first slabs (every A block: a short tile's extra rows
  // repeat its last row and are not read)
  uint32_t a_voff[A_PW];
  a_offsets<A_PW, NW>(p, tc, wave, lane, EA, a_voff);
  const float* const a_scale = FP8 ? p.a_scale : nullptr;
  EpiScales<G, MB> sc;
  {
    const PpOperands<G, EB, 16, EA> op(p, tc, wave, lane);
    const float* scale = WFP8 ? p.b_scale + static_cast<long long>(tc.expert) * p.nb_rows : nullptr;
    int src_row[MB][4];
    if constexpr (WFP8)
      epi_load_scales_1<G, MB>(p, tc, wm, wn, lane, scale, a_scale, sc, src_row,
                               mbe_of_rows<256, MB, A_PW>(tc.row_end - tc.row0));
    first_dma(op, a_voff, nt_tile(tc));
    if constexpr (WFP8) epi_load_scales_2<G, MB>(a_scale, sc, src_row);
  }
  for (;;) {
    TileCoord tn;
    const bool more = reg_decode<256, GM>(p, rsch, logical_of(slot + stride), tn);
    // The lane index, opaque to the compiler once per tile: otherwise it hoists the lane address
    // arithmetic of all three height classes out of the tile loop, all live at once (256 VGPRs
    // and spills against 196 for one tile per workgroup).
    int ln = lane;
    asm volatile("" : "+v"(ln));
    auto body = [&]<int MBE, int BAUX>() {
      const int lane = ln;
      constexpr int A_CNT = A_PW * MBE / MB;
      f32x4_t acc[MBE][G::NB];
#pragma unroll
      for (int i = 0; i < MBE; ++i)
#pragma unroll
        for (int j = 0; j < G::NB; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      const PpOperands<G, EB, 16, EA> op(p, tc, wave, lane);
      pp_wait_vm0();   // this tile's first slabs and scales (and the previous tile's stores)
      if constexpr (WFP8) pin_scales(sc);
      pp_barrier();
      // the next tile's row map: in flight during the first slab, whose end wait covers it
      uint32_t an_voff[A_PW];
      if (more) a_offsets<A_PW, NW>(p, tn, wave, lane, EA, an_voff);
      if constexpr (MODE == 2) pp3w_kloop<G, MBE, A_CNT>(acc, op.rA, op.rB, a_voff, op.b_voff, KT, wave, lane, st);
      else pp3_kloop<FP8, G, MBE, A_CNT, A_PW, B_PW, BAUX>(acc, op.rA, op.rB, a_voff, op.b_voff, KT, wave, lane, st);
      pp_wait_vm0();   // this wave's clamped loads have landed in its own LDS blocks
      EpiScales<G, MB> sn;
      if (more) {
        const PpOperands<G, EB, 16, EA> on(p, tn, wave, lane);
        const float* scale_n = WFP8 ? p.b_scale + static_cast<long long>(tn.expert) * p.nb_rows : nullptr;
        int src_row[MB][4];
        if constexpr (WFP8)
          epi_load_scales_1<G, MB>(p, tn, wm, wn, lane, scale_n, a_scale, sn, src_row,
                                   mbe_of_rows<256, MB, A_PW>(tn.row_end - tn.row0));
        first_dma(on, an_voff, nt_tile(tn));
        if constexpr (WFP8) epi_load_scales_2<G, MB>(a_scale, sn, src_row);
#pragma unroll
        for (int i = 0; i < A_PW; ++i) a_voff[i] = an_voff[i];
      }
      if constexpr (WFP8) epilogue<G, EPI, MBE>(p, tc, acc, wm, wn, lane, sc);
      else epilogue<G, EPI, MBE>(p, tc, acc, wm, wn, lane, nullptr, nullptr);
      if constexpr (WFP8) sc = sn;
    };
    const bool nt = nt_tile(tc);
    by_height<256, MB, A_PW>(tc.row_end - tc.row0, [&]<int MBE>() {
      if constexpr (MBE < MB && MODE != 2) {
        if (nt) {
          body.template operator()<MBE, 2>();
          return;
        }
      }
      body.template operator()<MBE, 0>();
    });
    if (!more) break;
    tc = tn;
    slot += stride;
  }
}

template <int BM, int BN, int WGM, int WGN, int EPI, int GM>
__global__ void __launch_bounds__(WGM * WGN * 64) grouped_gemm_fp8_kernel(GemmArgs p) {
  using G = Geo<BM, BN, WGM, WGN, EPI>;
  constexpr int BKB = 128;                    // K per slab = bytes per LDS row
  constexpr int NW = G::NW;
  constexpr int A_PW = BM / 8 / G::NW;
  constexpr int B_PW = BN / 8 / G::NW;
  static_assert(A_PW * 8 * G::NW == BM && B_PW * 8 * G::NW == BN, "slab split over waves");

  __shared__ __attribute__((aligned(1024))) uint8_t sA0[BM * BKB];
  __shared__ __attribute__((aligned(1024))) uint8_t sA1[BM * BKB];
  __shared__ __attribute__((aligned(1024))) uint8_t sB0[BN * BKB];
  __shared__ __attribute__((aligned(1024))) uint8_t sB1[BN * BKB];
  __shared__ int s_pref[kMaxSeg + 1];

  TileCoord tc;
  if (!decode_tile<BM, G::OUT_BN, GM>(p, s_pref, tc)) return;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lrow = lane >> 3;
  const long long k0 = static_cast<long long>(tc.split) * p.K;

  const BufRef rA{static_cast<const uint8_t*>(p.a) + k0, p.a_rows_cap * p.lda - k0};
  uint32_t a_voff[A_PW];
  a_offsets<A_PW, NW>(p, tc, wave, lane, 1, a_voff);
  const uint8_t* b_base = expert_weights(p, tc.expert, 1) + k0;
  const BufRef rB{b_base, p.b_estride - k0};
  uint32_t b_voff[B_PW];
#pragma unroll
  for (int i = 0; i < B_PW; ++i) {
    const int R = (wave * B_PW + i) * 8 + lrow;
    const int wr = G::weight_row_of_lds(R, tc.n_tile, p.up_off);
    b_voff[i] = static_cast<uint32_t>(static_cast<long long>(wr) * p.ldb + (((lane & 7) ^ swz(R)) << 4));
  }

  const int wm = wave % WGM;
  const int wn = wave / WGM;
  // The slab DMA helper addresses LDS in bf16 units (512 per 1 KiB block).
  uint16_t* a0 = reinterpret_cast<uint16_t*>(sA0);
  uint16_t* a1 = reinterpret_cast<uint16_t*>(sA1);
  uint16_t* b0 = reinterpret_cast<uint16_t*>(sB0);
  uint16_t* b1 = reinterpret_cast<uint16_t*>(sB1);
  const int KT = p.K / BKB;
  const float* scale = p.b_scale + static_cast<long long>(tc.expert) * p.nb_rows;
  const bool b_nt = p.b_nt != 0 || tc.one_mt != 0;   // as in grouped_gemm_dma_kernel
  by_height<BM, G::MB, A_PW>(tc.row_end - tc.row0, [&]<int MBE>() {
    constexpr int A_CNT = A_PW * MBE / G::MB;
    f32x4_t acc[MBE][G::NB];
#pragma unroll
    for (int i = 0; i < MBE; ++i)
#pragma unroll
      for (int j = 0; j < G::NB; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    issue_slab_dma<A_CNT, B_PW, NW>(rA, rB, a_voff, b_voff, a0, b0, wave, 0, b_nt);
    __syncthreads();
    int kt = 0;
    for (; kt + 1 < KT; kt += 2) {
      issue_slab_dma<A_CNT, B_PW, NW>(rA, rB, a_voff, b_voff, a1, b1, wave, (kt + 1) * BKB, b_nt);
      pin_issue();
      slab_mma_fp8<G, MBE>(acc, sA0, sB0, wm, wn, lane);
      __syncthreads();
      issue_slab_dma<A_CNT, B_PW, NW>(rA, rB, a_voff, b_voff, a0, b0, wave, min(kt + 2, KT - 1) * BKB, b_nt);
      pin_issue();
      slab_mma_fp8<G, MBE>(acc, sA1, sB1, wm, wn, lane);
      __syncthreads();
    }
    if (kt < KT) slab_mma_fp8<G, MBE>(acc, sA0, sB0, wm, wn, lane);
    epilogue<G, EPI, MBE>(p, tc, acc, wm, wn, lane, scale, p.a_scale);
  });
}

// ---------------------------------------------------------------------------- fp8 weights (W8A16)
template <int BM, int BN, int WGM, int WGN, int EPI, int GM>
__global__ void __launch_bounds__(WGM * WGN * 64) grouped_gemm_fp8w_kernel(GemmArgs p) {
  using G = Geo<BM, BN, WGM, WGN, EPI>;
  constexpr int BK = G::BK;
  constexpr int NT = G::NT;
  constexpr int NW = G::NW;
  constexpr int A_PW = BM / 8 / G::NW;
  static_assert(A_PW * 8 * G::NW == BM, "slab split over waves");
  constexpr int B_CH = BN * 4;                  // 16-byte (16 x fp8) chunks per B slab
  constexpr int B_LD = (B_CH + NT - 1) / NT;

  __shared__ __attribute__((aligned(1024))) uint16_t sA[2][BM * BK];
  __shared__ __attribute__((aligned(1024))) uint16_t sB[2][BN * BK];
  __shared__ int s_pref[kMaxSeg + 1];

  TileCoord tc;
  if (!decode_tile<BM, G::OUT_BN, GM>(p, s_pref, tc)) return;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const long long k0 = static_cast<long long>(tc.split) * p.K;

  const BufRef rA{static_cast<const uint16_t*>(p.a) + k0, (p.a_rows_cap * p.lda - k0) * 2};
  uint32_t a_voff[A_PW];
  a_offsets<A_PW, NW>(p, tc, wave, lane, 2, a_voff);
  const uint8_t* b_base = expert_weights(p, tc.expert, 1) + k0;
  const BufRef rB{b_base, p.b_estride - k0};
  uint32_t b_voff[B_LD];
  int b_R[B_LD], b_c[B_LD];
#pragma unroll
  for (int i = 0; i < B_LD; ++i) {
    const int qc = tid + NT * i;
    const int R = (qc < B_CH ? qc : 0) >> 2;
    const int c = qc & 3;
    b_R[i] = R;
    b_c[i] = c;
    b_voff[i] =
        static_cast<uint32_t>(static_cast<long long>(G::weight_row_of_lds(R, tc.n_tile, p.up_off)) * p.ldb + c * 16);
  }
  const int wm = wave % WGM;
  const int wn = wave / WGM;
  const int KT = p.K / BK;
  const float* scale = p.b_scale + static_cast<long long>(tc.expert) * p.nb_rows;
  by_height<BM, G::MB, A_PW>(tc.row_end - tc.row0, [&]<int MBE>() {
    constexpr int A_CNT = A_PW * MBE / G::MB;
    u32x4_t rb[B_LD];
    f32x4_t acc[MBE][G::NB];
#pragma unroll
    for (int i = 0; i < MBE; ++i)
#pragma unroll
      for (int j = 0; j < G::NB; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    issue_a_dma<A_CNT, NW>(rA, a_voff, sA[0], wave, 0);
    load_b_fp8<B_LD, B_CH, NT>(rB, b_voff, rb, 0);
    store_b_fp8<G, B_LD, B_CH, NT>(rb, b_R, b_c, sB[0]);
    __syncthreads();
    for (int kt = 0; kt < KT; ++kt) {
      const int cur = kt & 1;
      if (kt + 1 < KT) {
        issue_a_dma<A_CNT, NW>(rA, a_voff, sA[cur ^ 1], wave, (kt + 1) * BK * 2);
        load_b_fp8<B_LD, B_CH, NT>(rB, b_voff, rb, (kt + 1) * BK);
      }
      bf16x8_t fa0[MBE], fb0[G::NB], fa1[MBE], fb1[G::NB];
      read_frags<G, MBE>(sA[cur], sB[cur], 0, wm, wn, lane, fa0, fb0);
      read_frags<G, MBE>(sA[cur], sB[cur], 1, wm, wn, lane, fa1, fb1);
      mma<G, MBE>(acc, fa0, fb0);
      mma<G, MBE>(acc, fa1, fb1);
      if (kt + 1 < KT) store_b_fp8<G, B_LD, B_CH, NT>(rb, b_R, b_c, sB[cur ^ 1]);
      __syncthreads();
    }
    epilogue<G, EPI, MBE>(p, tc, acc, wm, wn, lane, scale, nullptr);   // W8A16: bf16 activations
  });
}

// ---------------------------------------------------------------------------- fp8 weights (W8A16), direct-to-LDS
// The LDS tiles of W8A16 with the e4m3 weight rows DMA'd to LDS as they are (128 k per 128-byte row)
// and widened to bf16 at the fragment reads, the k assignment of the ping-pong W8A16 tile (within a
// 64-k activation slab lane group q takes k = 16q + 8*KK + 0..7 in MFMA step KK; one 16-byte weight
// read per slab covers both steps), so its sums are those of the 256x256 W8A16 tile, bit for bit.
// Tiles of at most 64 rows keep a whole 128-k chunk of both operands per stage (two activation
// slabs and one weight slab, one barrier per chunk: Mixtral-8x7B 64 tokens, 32x128, gate/up 180.9
// -> 162.7 us and down 98.3 -> 75.1 us against a barrier per activation slab).  The 128x128 tile,
// whose chunk stages would leave one workgroup per CU, keeps 64-k activation stages: a weight chunk
// serves two of them and its DMA goes out at the top of the odd slab before them, into the stage
// the chunk before last has left.  Both stages of each operand are distinct objects and the loops
// are unrolled, so every stage index is static.  K % 128 == 0.
template <class G, int MBE>
__device__ __forceinline__ void w8a16_slab_mma(f32x4_t (&acc)[MBE][G::NB], const uint16_t* sA, const uint16_t* sB,
                                               int half, int wm, int wn, int lane) {
  const int lr = lane & 15;
  const int q = lane >> 4;
  const uint8_t* b8 = reinterpret_cast<const uint8_t*>(sB);
  u32x4_t braw[G::NB];
#pragma unroll
  for (int j = 0; j < G::NB; ++j) {
    const int R = wn * G::WN + j * 16 + lr;
    braw[j] = *reinterpret_cast<const u32x4_t*>(&b8[R * 128 + (((4 * half + q) ^ swz(R)) << 4)]);
  }
#pragma unroll
  for (int KK = 0; KK < 2; ++KK) {
    bf16x8_t af[MBE], bw[G::NB];
#pragma unroll
    for (int i = 0; i < MBE; ++i) {
      const int R = wm * 16 * MBE + i * 16 + lr;
      af[i] = *reinterpret_cast<const bf16x8_t*>(&sA[R * G::BK + (((2 * q + KK) ^ swz(R)) << 3)]);
    }
#pragma unroll
    for (int j = 0; j < G::NB; ++j) bw[j] = widen_fp8x8(braw[j][2 * KK], braw[j][2 * KK + 1]);
    mma<G, MBE>(acc, af, bw);
  }
}

template <int B_PW, int NW>
__device__ __forceinline__ void issue_b8_dma(const BufRef& b, const uint32_t (&b_voff)[B_PW], uint16_t* sB, int wave,
                                             int soff, bool b_nt) {
#if defined(__HIP_DEVICE_COMPILE__)
  const auto rB = make_rsrc(b.base, b.bytes);
  if (b_nt) {
#pragma unroll
    for (int i = 0; i < B_PW; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rB, (lds_void_t*)(sB + (wave * B_PW + i) * 512), 16, b_voff[i], soff,
                                               0, 2);
  } else {
#pragma unroll
    for (int i = 0; i < B_PW; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rB, (lds_void_t*)(sB + (wave * B_PW + i) * 512), 16, b_voff[i], soff,
                                               0, 0);
  }
#endif
}

template <int BM, int BN, int WGM, int WGN, int EPI, int GM>
__global__ void __launch_bounds__(WGM * WGN * 64) grouped_gemm_w8a16_dma_kernel(GemmArgs p) {
  using G = Geo<BM, BN, WGM, WGN, EPI>;
  constexpr int BK = G::BK;
  constexpr int NW = G::NW;
  constexpr int A_PW = BM / 8 / NW;   // 1 KiB LDS blocks per wave per slab (8 rows each)
  constexpr int B_PW = BN / 8 / NW;
  static_assert(A_PW * 8 * NW == BM && B_PW * 8 * NW == BN, "slab split over waves");

  // CHUNK (tiles of at most 64 rows): a stage holds a whole 128-k chunk of both operands (two
  // activation slabs), one barrier per chunk; else a stage holds one 64-k activation slab.
  constexpr bool CHUNK = BM <= 64;
  __shared__ __attribute__((aligned(1024))) uint16_t sA0[(CHUNK ? 2 : 1) * BM * BK];
  __shared__ __attribute__((aligned(1024))) uint16_t sA1[(CHUNK ? 2 : 1) * BM * BK];
  __shared__ __attribute__((aligned(1024))) uint16_t sB0[BN * BK];   // BN rows of 128 e4m3 bytes
  __shared__ __attribute__((aligned(1024))) uint16_t sB1[BN * BK];
  __shared__ int s_pref[kMaxSeg + 1];

  TileCoord tc;
  if (!decode_tile<BM, G::OUT_BN, GM>(p, s_pref, tc)) return;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lrow = lane >> 3;
  const long long k0 = static_cast<long long>(tc.split) * p.K;

  const BufRef rA{static_cast<const uint8_t*>(p.a) + k0 * 2, (p.a_rows_cap * p.lda - k0) * 2};
  uint32_t a_voff[A_PW];
  a_offsets<A_PW, NW>(p, tc, wave, lane, 2, a_voff);
  const uint8_t* b_base = expert_weights(p, tc.expert, 1) + k0;
  const BufRef rB{b_base, p.b_estride - k0};
  uint32_t b_voff[B_PW];
#pragma unroll
  for (int i = 0; i < B_PW; ++i) {
    const int R = (wave * B_PW + i) * 8 + lrow;
    const int wr = G::weight_row_of_lds(R, tc.n_tile, p.up_off);
    b_voff[i] = static_cast<uint32_t>(static_cast<long long>(wr) * p.ldb + (((lane & 7) ^ swz(R)) << 4));
  }
  const int wm = wave % WGM;
  const int wn = wave / WGM;
  const int KT = p.K / BK;   // 64-k activation slabs (even)
  const int NC = KT / 2;     // 128-k weight chunks
  const bool nt = p.b_nt != 0 || tc.one_mt != 0;   // as in grouped_gemm_dma_kernel
  const float* scale = p.b_scale + static_cast<long long>(tc.expert) * p.nb_rows;
  by_height<BM, G::MB, A_PW>(tc.row_end - tc.row0, [&]<int MBE>() {
    constexpr int A_CNT = A_PW * MBE / G::MB;
    f32x4_t acc[MBE][G::NB];
#pragma unroll
    for (int i = 0; i < MBE; ++i)
#pragma unroll
      for (int j = 0; j < G::NB; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    if constexpr (CHUNK) {
      auto issue_chunk = [&](int c, uint16_t* sa, uint16_t* sb) __attribute__((always_inline)) {
        issue_a_dma<A_CNT, NW>(rA, a_voff, sa, wave, c * 256);
        issue_a_dma<A_CNT, NW>(rA, a_voff, sa + BM * BK, wave, c * 256 + 128);
        issue_b8_dma<B_PW, NW>(rB, b_voff, sb, wave, c * 128, nt);
      };
      auto chunk_mma = [&](const uint16_t* sa, const uint16_t* sb) __attribute__((always_inline)) {
        w8a16_slab_mma<G, MBE>(acc, sa, sb, 0, wm, wn, lane);
        w8a16_slab_mma<G, MBE>(acc, sa + BM * BK, sb, 1, wm, wn, lane);
      };
      // chunk c in stage 0 at the top of each iteration; the second load is unconditional (near
      // the end it re-reads the last chunk into stage 0, which is not read again and which the
      // closing barrier waits for)
      issue_chunk(0, sA0, sB0);
      __syncthreads();
      int c = 0;
      for (; c + 1 < NC; c += 2) {
        issue_chunk(c + 1, sA1, sB1);
        pin_issue();
        chunk_mma(sA0, sB0);
        __syncthreads();
        issue_chunk(min(c + 2, NC - 1), sA0, sB0);
        pin_issue();
        chunk_mma(sA1, sB1);
        __syncthreads();
      }
      if (c < NC) chunk_mma(sA0, sB0);
      epilogue<G, EPI, MBE>(p, tc, acc, wm, wn, lane, scale, nullptr);   // bf16 activations
      return;
    }
    issue_a_dma<A_CNT, NW>(rA, a_voff, sA0, wave, 0);
    issue_b8_dma<B_PW, NW>(rB, b_voff, sB0, wave, 0, nt);
    __syncthreads();
    // slab kt + J: activations in SA, its weight chunk in SB (half J % 2 of it); loads the next
    // slab's activations into SAN and, after an odd slab's issue, the chunk after next into SBN
    // (clamped near the end: those stages are not read again)
#define EIMOE_W8_SLAB(J, SA, SAN, SB, SBN)                                                             \
    if (kt + J < KT) {                                                                               \
      issue_a_dma<A_CNT, NW>(rA, a_voff, SAN, wave, min(kt + J + 1, KT - 1) * 128);                  \
      if (J % 2 == 1) issue_b8_dma<B_PW, NW>(rB, b_voff, SBN, wave, min((kt + J + 1) / 2, NC - 1) * 128, nt); \
      pin_issue();                                                                                   \
      w8a16_slab_mma<G, MBE>(acc, SA, SB, J % 2, wm, wn, lane);                                       \
      __syncthreads();                                                                               \
    }
    for (int kt = 0; kt < KT; kt += 4) {
      EIMOE_W8_SLAB(0, sA0, sA1, sB0, sB1)
      EIMOE_W8_SLAB(1, sA1, sA0, sB0, sB1)
      EIMOE_W8_SLAB(2, sA0, sA1, sB1, sB0)
      EIMOE_W8_SLAB(3, sA1, sA0, sB1, sB0)
    }
#undef EIMOE_W8_SLAB
    epilogue<G, EPI, MBE>(p, tc, acc, wm, wn, lane, scale, nullptr);   // bf16 activations
  });
}

// grouped_gemm_w8a16_dma_kernel's chunk loop (tiles of at most 64 rows) on a ring of three chunk
// stages: as grouped_gemm_ring_kernel does for bf16, the DMA goes two chunks ahead, the chunk's
// fragments (both halves: e4m3 weight rows, then the activations of each MFMA step) are read in one
// asm block that ends waiting for them, the weights are widened after it, and each chunk ends
// waiting for its wave's next chunk only.  Same MFMAs in the same order: bit-identical.  K % 128 == 0.
template <int BM, int BN, int WGM, int WGN, int EPI, int GM>
__global__ void __launch_bounds__(WGM * WGN * 64) grouped_gemm_w8a16_ring_kernel(GemmArgs p) {
  using G = Geo<BM, BN, WGM, WGN, EPI>;
  constexpr int BK = G::BK;
  constexpr int NW = G::NW;
  constexpr int A_PW = BM / 8 / NW;
  constexpr int B_PW = BN / 8 / NW;
  static_assert(A_PW * 8 * NW == BM && B_PW * 8 * NW == BN, "slab split over waves");
  static_assert(BM <= 64, "chunk stages");
  struct Stage {
    uint16_t a[2 * BM * BK];   // two 64-k activation slabs
    uint16_t b[BN * BK];       // BN rows of 128 e4m3 bytes
  };
  __shared__ __attribute__((aligned(1024))) Stage t0;
  __shared__ __attribute__((aligned(1024))) Stage t1;
  __shared__ __attribute__((aligned(1024))) Stage t2;
  __shared__ int s_pref[kMaxSeg + 1];

  TileCoord tc;
  if (!decode_tile<BM, G::OUT_BN, GM>(p, s_pref, tc)) return;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lrow = lane >> 3;
  const long long k0 = static_cast<long long>(tc.split) * p.K;
  const BufRef rA{static_cast<const uint8_t*>(p.a) + k0 * 2, (p.a_rows_cap * p.lda - k0) * 2};
  uint32_t a_voff[A_PW];
  a_offsets<A_PW, NW>(p, tc, wave, lane, 2, a_voff);
  const uint8_t* b_base = expert_weights(p, tc.expert, 1) + k0;
  const BufRef rB{b_base, p.b_estride - k0};
  uint32_t b_voff[B_PW];
#pragma unroll
  for (int i = 0; i < B_PW; ++i) {
    const int R = (wave * B_PW + i) * 8 + lrow;
    const int wr = G::weight_row_of_lds(R, tc.n_tile, p.up_off);
    b_voff[i] = static_cast<uint32_t>(static_cast<long long>(wr) * p.ldb + (((lane & 7) ^ swz(R)) << 4));
  }
  const int wm = wave % WGM;
  const int wn = wave / WGM;
  const int NC = p.K / 128;   // 128-k chunks
  const bool nt = p.b_nt != 0 || tc.one_mt != 0;
  const float* scale = p.b_scale + static_cast<long long>(tc.expert) * p.nb_rows;
  const int lr = lane & 15;
  const int q = lane >> 4;
  by_height<BM, G::MB, A_PW>(tc.row_end - tc.row0, [&]<int MBE>() {
    constexpr int A_CNT = A_PW * MBE / G::MB;
    constexpr int L = 2 * A_CNT + B_PW;          // DMA instructions per chunk per wave
    constexpr int NF = 2 * (G::NB + 2 * MBE);    // fragment reads per chunk
    f32x4_t acc[MBE][G::NB];
#pragma unroll
    for (int i = 0; i < MBE; ++i)
#pragma unroll
      for (int j = 0; j < G::NB; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    auto issue_chunk = [&](int c, Stage& st) __attribute__((always_inline)) {
      issue_a_dma<A_CNT, NW>(rA, a_voff, st.a, wave, c * 256);
      issue_a_dma<A_CNT, NW>(rA, a_voff, st.a + BM * BK, wave, c * 256 + 128);
      issue_b8_dma<B_PW, NW>(rB, b_voff, st.b, wave, c * 128, nt);
    };
    // fragment addresses of a stage: per half h, the NB weight rows, then the MBE activation
    // fragments of step 0 and of step 1 (the k assignment of w8a16_slab_mma)
    auto chunk_mma = [&](const Stage& st) __attribute__((always_inline)) {
      const uint32_t aA = lds_addr(st.a);
      const uint32_t aB = lds_addr(st.b);
      uint32_t ad[NF];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        constexpr int PH = G::NB + 2 * MBE;
#pragma unroll
        for (int j = 0; j < G::NB; ++j) {
          const int R = wn * G::WN + j * 16 + lr;
          ad[h * PH + j] = aB + R * 128 + (((4 * h + q) ^ swz(R)) << 4);
        }
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
#pragma unroll
          for (int i = 0; i < MBE; ++i) {
            const int R = wm * 16 * MBE + i * 16 + lr;
            ad[h * PH + G::NB + kk * MBE + i] = aA + 2 * (h * BM * BK + R * BK + (((2 * q + kk) ^ swz(R)) << 3));
          }
      }
      bf16x8_t fr[NF];
      lds_read_wait(ad, fr);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        constexpr int PH = G::NB + 2 * MBE;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          bf16x8_t af[MBE], bw[G::NB];
#pragma unroll
          for (int i = 0; i < MBE; ++i) af[i] = fr[h * PH + G::NB + kk * MBE + i];
#pragma unroll
          for (int j = 0; j < G::NB; ++j) {
            const u32x4_t raw = __builtin_bit_cast(u32x4_t, fr[h * PH + j]);
            bw[j] = widen_fp8x8(raw[2 * kk], raw[2 * kk + 1]);
          }
          mma<G, MBE>(acc, af, bw);
        }
      }
    };
    issue_chunk(0, t0);
    issue_chunk(min(1, NC - 1), t1);
    wait_vm<L>();   // this wave's chunk 0
    pp_barrier();
#define EIMOE_W8R_CHUNK(J, ST, STN)                  \
  if (c + J < NC) {                                 \
    issue_chunk(min(c + J + 2, NC - 1), STN);       \
    chunk_mma(ST);                                  \
    wait_vm<L>();                                   \
    pp_barrier();                                   \
  }
    for (int c = 0; c < NC; c += 3) {
      EIMOE_W8R_CHUNK(0, t0, t2)
      EIMOE_W8R_CHUNK(1, t1, t0)
      EIMOE_W8R_CHUNK(2, t2, t1)
    }
#undef EIMOE_W8R_CHUNK
    pp_wait_vm0();   // the clamped loads near the end land before the workgroup's LDS is released
    epilogue<G, EPI, MBE>(p, tc, acc, wm, wn, lane, scale, nullptr);   // bf16 activations
  });
}

// grouped_gemm_fp8_kernel (W8A8, e4m3 x e4m3) on the three-stage ring of grouped_gemm_ring_kernel:
// a 128-k slab is a 128-byte row of either operand, a fragment two 16-byte chunks of it (frag_fp8),
// read in one asm block; each accumulator takes one MFMA per slab, as in slab_mma_fp8, so results
// are bit-identical.
template <int BM, int BN, int WGM, int WGN, int EPI, int GM>
__global__ void __launch_bounds__(WGM * WGN * 64) grouped_gemm_fp8_ring_kernel(GemmArgs p) {
  using G = Geo<BM, BN, WGM, WGN, EPI>;
  constexpr int BKB = 128;   // K per slab = bytes per LDS row
  constexpr int NW = G::NW;
  constexpr int A_PW = BM / 8 / NW;
  constexpr int B_PW = BN / 8 / NW;
  static_assert(A_PW * 8 * NW == BM && B_PW * 8 * NW == BN, "slab split over waves");
  struct Stage {
    uint16_t a[BM * 64];   // BM rows of 128 e4m3 bytes (the DMA helpers count in 2-byte units)
    uint16_t b[BN * 64];
  };
  __shared__ __attribute__((aligned(1024))) Stage t0;
  __shared__ __attribute__((aligned(1024))) Stage t1;
  __shared__ __attribute__((aligned(1024))) Stage t2;
  __shared__ int s_pref[kMaxSeg + 1];

  TileCoord tc;
  if (!decode_tile<BM, G::OUT_BN, GM>(p, s_pref, tc)) return;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lrow = lane >> 3;
  const long long k0 = static_cast<long long>(tc.split) * p.K;
  const BufRef rA{static_cast<const uint8_t*>(p.a) + k0, p.a_rows_cap * p.lda - k0};
  uint32_t a_voff[A_PW];
  a_offsets<A_PW, NW>(p, tc, wave, lane, 1, a_voff);
  const uint8_t* b_base = expert_weights(p, tc.expert, 1) + k0;
  const BufRef rB{b_base, p.b_estride - k0};
  uint32_t b_voff[B_PW];
#pragma unroll
  for (int i = 0; i < B_PW; ++i) {
    const int R = (wave * B_PW + i) * 8 + lrow;
    const int wr = G::weight_row_of_lds(R, tc.n_tile, p.up_off);
    b_voff[i] = static_cast<uint32_t>(static_cast<long long>(wr) * p.ldb + (((lane & 7) ^ swz(R)) << 4));
  }
  const int wm = wave % WGM;
  const int wn = wave / WGM;
  const int KT = p.K / BKB;
  const bool b_nt = p.b_nt != 0 || tc.one_mt != 0;
  const float* scale = p.b_scale + static_cast<long long>(tc.expert) * p.nb_rows;
  const int lr = lane & 15;
  const int q = lane >> 4;
  by_height<BM, G::MB, A_PW>(tc.row_end - tc.row0, [&]<int MBE>() {
    constexpr int A_CNT = A_PW * MBE / G::MB;
    constexpr int L = A_CNT + B_PW;
    constexpr int NF = 2 * (MBE + G::NB);   // 16-byte reads per slab
    f32x4_t acc[MBE][G::NB];
#pragma unroll
    for (int i = 0; i < MBE; ++i)
#pragma unroll
      for (int j = 0; j < G::NB; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    auto slab = [&](const Stage& st) __attribute__((always_inline)) {
      const uint32_t aA = lds_addr(st.a);
      const uint32_t aB = lds_addr(st.b);
      uint32_t ad[NF];
#pragma unroll
      for (int i = 0; i < MBE; ++i) {
        const int R = wm * 16 * MBE + i * 16 + lr;
        ad[2 * i] = aA + R * 128 + ((q ^ swz(R)) << 4);
        ad[2 * i + 1] = aA + R * 128 + (((q + 4) ^ swz(R)) << 4);
      }
#pragma unroll
      for (int j = 0; j < G::NB; ++j) {
        const int R = wn * G::WN + j * 16 + lr;
        ad[2 * (MBE + j)] = aB + R * 128 + ((q ^ swz(R)) << 4);
        ad[2 * (MBE + j) + 1] = aB + R * 128 + (((q + 4) ^ swz(R)) << 4);
      }
      bf16x8_t fr[NF];
      lds_read_wait(ad, fr);
      i32x8_t af[MBE], bf[G::NB];
#pragma unroll
      for (int i = 0; i < MBE; ++i) {
        const u32x4_t lo = __builtin_bit_cast(u32x4_t, fr[2 * i]);
        const u32x4_t hi = __builtin_bit_cast(u32x4_t, fr[2 * i + 1]);
        af[i] = i32x8_t{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
      }
#pragma unroll
      for (int j = 0; j < G::NB; ++j) {
        const u32x4_t lo = __builtin_bit_cast(u32x4_t, fr[2 * (MBE + j)]);
        const u32x4_t hi = __builtin_bit_cast(u32x4_t, fr[2 * (MBE + j) + 1]);
        bf[j] = i32x8_t{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
      }
#pragma unroll
      for (int i = 0; i < MBE; ++i)
#pragma unroll
        for (int j = 0; j < G::NB; ++j) acc[i][j] = mfma_fp8(af[i], bf[j], acc[i][j]);
    };
    issue_slab_dma<A_CNT, B_PW, NW>(rA, rB, a_voff, b_voff, t0.a, t0.b, wave, 0, b_nt);
    issue_slab_dma<A_CNT, B_PW, NW>(rA, rB, a_voff, b_voff, t1.a, t1.b, wave, min(1, KT - 1) * BKB, b_nt);
    wait_vm<L>();   // this wave's slab 0
    pp_barrier();
#define EIMOE_F8R_SLAB(J, ST, STN)                                                                 \
  if (kt + J < KT) {                                                                              \
    issue_slab_dma<A_CNT, B_PW, NW>(rA, rB, a_voff, b_voff, STN.a, STN.b, wave,                     \
                                    min(kt + J + 2, KT - 1) * BKB, b_nt);                         \
    slab(ST);                                                                                     \
    wait_vm<L>();                                                                                 \
    pp_barrier();                                                                                 \
  }
    for (int kt = 0; kt < KT; kt += 3) {
      EIMOE_F8R_SLAB(0, t0, t2)
      EIMOE_F8R_SLAB(1, t1, t0)
      EIMOE_F8R_SLAB(2, t2, t1)
    }
#undef EIMOE_F8R_SLAB
    pp_wait_vm0();   // the clamped loads near the end land before the workgroup's LDS is released
    epilogue<G, EPI, MBE>(p, tc, acc, wm, wn, lane, scale, p.a_scale);
  });
}

// ---------------------------------------------------------------------------- launch
// bf16 LDS tiles of at most 64 rows: the three-stage ring (grouped_gemm_ring_kernel) holds two slabs
// in flight per workgroup instead of one, but at fewer workgroups per CU (LDS: 32x128 3 -> 2,
// 64x128 3 -> 2, 16x64 6 -> 4).  Taken unless the two-stage kernel would run the launch's tiles in
// one round and the ring would not: estimated tiles (expected rows, as the tile rules use them) above
// the two-stage slots, or within the ring's with a third to spare for skewed routing.  A/B on one
// box, all bit-identical, the ring on every such tile: DeepSeek-V2-Lite 64 / 256 tokens 0.184 ->
// 0.170 / 0.222 -> 0.200 ms cold, Qwen3-30B-A3B share 256 tokens 95 -> 93 us, but the share at 768
// tokens 90 -> 92 us (its down projection, ~640 tiles of 64x128, one round of the two-stage kernel's
// 768 slots and 1.25 of the ring's 512).
// Workgroups per CU that a tile's LDS allows: `stages` stages of stage_bytes and the segment prefix.
static int lds_tile_wgs(int stage_bytes, int stages) {
  const int bytes = stages * stage_bytes + (kMaxSeg + 1) * 4;
  const int kib = (bytes + 1023) / 1024;
  return 160 / kib;
}

// stage_bytes: one stage of the tile (bf16: a 64-k slab of A and B; W8A16: a 128-k chunk of both).
static bool use_ring_tile(const GemmArgs& p, int bm, int stage_bytes, int n_tiles) {
  const int S = p.S > 0 ? p.S : 1;
  const double avg = static_cast<double>(p.rows_hint > 0 ? std::min(p.rows_hint, p.max_rows) : p.max_rows) / S;
  const double est = static_cast<double>(S) * std::ceil(avg / bm) * n_tiles * p.k_split;
  const double slots2 = static_cast<double>(lds_tile_wgs(stage_bytes, 2)) * kNumCu;
  const double slots3 = static_cast<double>(lds_tile_wgs(stage_bytes, 3)) * kNumCu;
  return est > slots2 || est * 1.3 <= slots3;
}

template <int BM, int BN, int WGM, int WGN, int EPI, bool BFP8, int GM>
static hipError_t launch_cfg(const GemmArgs& p, int max_rows, bool a_fp8, hipStream_t s) {
  constexpr int OUT_BN = epi_silu(EPI) ? BN / 2 : BN;
  const int n_tiles = p.N / OUT_BN;
  const long long max_mt = (static_cast<long long>(max_rows) + BM - 1) / BM + p.S;
  long long total = max_mt * n_tiles * p.k_split;
  long long grid = (total + kNumXcd - 1) / kNumXcd * kNumXcd;
  if (grid < kNumXcd) grid = kNumXcd;
  if (grid > 0x7fffffffll) return hipErrorInvalidValue;
  // A plain runtime branch: the kernels of a configuration are instantiated together.
  if (BFP8 && a_fp8) {
    if constexpr (BM <= 64) {
      if (use_ring_tile(p, BM, (BM + BN) * 128, n_tiles)) {
        hipLaunchKernelGGL((grouped_gemm_fp8_ring_kernel<BM, BN, WGM, WGN, EPI, GM>),
                           dim3(static_cast<unsigned>(grid)), dim3(WGM * WGN * 64), 0, s, p);
        return hipGetLastError();
      }
    }
    hipLaunchKernelGGL((grouped_gemm_fp8_kernel<BM, BN, WGM, WGN, EPI, GM>), dim3(static_cast<unsigned>(grid)),
                       dim3(WGM * WGN * 64), 0, s, p);
  } else if (BFP8) {
    // W8A16: the e4m3 weights DMA'd to LDS and widened at the fragment reads when K allows, else
    // widened through registers on their way to LDS
    if constexpr (BM <= 128) {
      if (p.K % 128 == 0) {
        if constexpr (BM <= 64) {
          if (use_ring_tile(p, BM, (2 * BM + BN) * 128, n_tiles)) {
            hipLaunchKernelGGL((grouped_gemm_w8a16_ring_kernel<BM, BN, WGM, WGN, EPI, GM>),
                               dim3(static_cast<unsigned>(grid)), dim3(WGM * WGN * 64), 0, s, p);
            return hipGetLastError();
          }
        }
        hipLaunchKernelGGL((grouped_gemm_w8a16_dma_kernel<BM, BN, WGM, WGN, EPI, GM>),
                           dim3(static_cast<unsigned>(grid)), dim3(WGM * WGN * 64), 0, s, p);
        return hipGetLastError();
      }
    }
    hipLaunchKernelGGL((grouped_gemm_fp8w_kernel<BM, BN, WGM, WGN, EPI, GM>), dim3(static_cast<unsigned>(grid)),
                       dim3(WGM * WGN * 64), 0, s, p);
  } else {
    if constexpr (BM <= 64) {
      if (use_ring_tile(p, BM, (BM + BN) * 128, n_tiles)) {
        hipLaunchKernelGGL((grouped_gemm_ring_kernel<BM, BN, WGM, WGN, EPI, GM, 3>), dim3(static_cast<unsigned>(grid)),
                           dim3(WGM * WGN * 64), 0, s, p);
        return hipGetLastError();
      }
    }
    hipLaunchKernelGGL((grouped_gemm_dma_kernel<BM, BN, WGM, WGN, EPI, GM>), dim3(static_cast<unsigned>(grid)),
                       dim3(WGM * WGN * 64), 0, s, p);
  }
  return hipGetLastError();
}

// 256x256 tiles: the ping-pong kernel (bf16: 3-4 % faster than the lock-step 8-wave kernel on
// the Mixtral-8x7B prefill GEMMs, bit-identical results; e4m3 W8A8: with the epilogue's scale
// loads hoisted, gate/up 2.32 -> 1.95 ms and down (K split 2) 1.08 -> 0.89 ms against the
// lock-step kernel, A/B on one box).  W8A16 keeps the lock-step kernel (its B goes through
// registers for the conversion).
// Tile grouping depth 8: on the current kernels (persistent tile walk, hardware-reciprocal SiLU)
// depth 8 and 16 both run the Mixtral-8x7B 8192-token layer ~1 % faster than 4 (4.25 vs 4.29 ms,
// W8A8 2.40-2.42 vs 2.43-2.44 ms; DeepSeek-V2-Lite within noise, two repeats on one box).
// MODE as grouped_gemm_pp3p_kernel's.  W8A16 runs the ping-pong kernel persistent only (launches
// of at most 64 segments, K % 128 == 0); otherwise the lock-step kernel that widens the weights
// through registers.
template <int EPI, int MODE = 0, int GMX = 8>
static hipError_t launch_pp(const GemmArgs& p, int max_rows, hipStream_t s) {
  if constexpr (MODE == 2)
    if (p.S > 64 || p.K % 128 != 0) return launch_cfg<256, 256, 4, 2, EPI, true, 4>(p, max_rows, false, s);
  constexpr int OUT_BN = epi_silu(EPI) ? 128 : 256;
  const int n_tiles = p.N / OUT_BN;
  const long long max_mt = (static_cast<long long>(max_rows) + 255) / 256 + p.S;
  long long total = max_mt * n_tiles * p.k_split;
  long long grid = (total + kNumXcd - 1) / kNumXcd * kNumXcd;
  if (grid < kNumXcd) grid = kNumXcd;
  if (grid > 0x7fffffffll) return hipErrorInvalidValue;
  if (p.S <= 64) {
    // persistent: one workgroup per CU at most (the grid stays a whole number of XCD rounds).
    // Against one tile per workgroup (A/B on one box): Mixtral-8x7B W8A8 gate/up 1524 -> 1485 us
    // under counters, layers within 0-1 % (the bf16 GEMMs run at the chip's power-limited clock
    // either way, so hiding the per-tile latencies buys them nothing).
    const long long pgrid = std::min<long long>(grid, kNumCu);
    hipLaunchKernelGGL((grouped_gemm_pp3p_kernel<EPI, GMX, MODE>), dim3(static_cast<unsigned>(pgrid)), dim3(512), 0,
                       s, p);
    return hipGetLastError();
  }
  if constexpr (MODE != 2) {
    hipLaunchKernelGGL((grouped_gemm_pp3_kernel<EPI, GMX, MODE == 1>), dim3(static_cast<unsigned>(grid)), dim3(512),
                       0, s, p);
  }
  return hipGetLastError();
}

template <int EPI, bool BFP8>
static hipError_t launch_epi(const GemmArgs& p, int max_rows, int tile, bool a_fp8, hipStream_t s) {
  switch (tile) {
    case kTileL:
      if constexpr (BFP8) {
        if (a_fp8) return launch_pp<EPI, 1>(p, max_rows, s);
        return launch_pp<EPI, 2>(p, max_rows, s);
      } else {
        return launch_pp<EPI, 0>(p, max_rows, s);
      }
    case kTileM: return launch_cfg<128, 128, 2, 2, EPI, BFP8, 4>(p, max_rows, a_fp8, s);
    case kTileMS: return launch_cfg<64, 128, 2, 2, EPI, BFP8, 4>(p, max_rows, a_fp8, s);
    case kTileS: return launch_cfg<32, 128, 1, 4, EPI, BFP8, 1>(p, max_rows, a_fp8, s);
    case kTileXS: return launch_cfg<16, 64, 1, 2, EPI, BFP8, 1>(p, max_rows, a_fp8, s);
    default: return hipErrorInvalidValue;
  }
}

int gemm_out_cols_per_tile(int tile, int epi) {
  if (tile == kTileStream) return epi_silu(epi) ? 16 : 32;   // narrowest task; wider when N allows
  int bn = 0;
  switch (tile) {
    case kTileL: bn = 256; break;
    case kTileM: bn = 128; break;
    case kTileMS: bn = 128; break;
    case kTileS: bn = 128; break;
    case kTileXS: bn = 64; break;
    default: return 0;
  }
  return epi_silu(epi) ? bn / 2 : bn;
}

// Routed launches (8 or more segments) of bf16 experts that stay in cache, from 8 to a few
// hundred expected rows per segment.  What decides is whether a tile shape spreads the weight
// panels over all CUs: the 256x256 tile is the fastest per tile (persistent, ping-pong) but with
// few experts and narrow outputs it leaves CUs idle, the 64x128 tile (three workgroups per CU,
// one m-tile for most segments) covers the CUs where 128x128 makes too few tiles and 32x128 reads
// each weight panel once per 32 rows.  Tile counts are estimated at the expected rows.  Measured
// per GEMM, single launches on the routed segments (cold, one box; us):
//  * Qwen3-30B-A3B 32-expert share, 768 tokens (46 rows per expert, 198 at most): gate/up 52.8 on
//    64x128 against 63.2 / 63.7 / 62.7 on 128x128 / 32x128 / 256x256, down 35.9 against 49.1 /
//    48.2 / 41.4; 256 tokens (15 rows): gate/up 51.0 on 32x128 (64x128 52.9, 128x128 54.4), down
//    33.4 on 128x128 (32x128 34.9);
//  * DeepSeek-V2-Lite, 768 tokens (72 rows, zipf routing): gate/up 152.9 on 256x256 against
//    174.3 / 178.6 / 218.9 on 64x128 / 128x128 / 32x128, down 88.2 against 99.5 / 105.1 / 115.3
//    (uniform routing: 168.7 and 87.2 on 256x256); 128 tokens (12 rows): gate/up 112.6 on 128x128
//    against 125.3 streamed and 128.4 on 32x128.
static int routed_small_gate_up_tile(const GemmArgs& p, int S, double avg, int t, bool fp8) {
  const long long tiles_l = static_cast<long long>(S) * static_cast<long long>((avg + 255) / 256) * (p.N / 128);
  const long long tiles_m = static_cast<long long>(S) * static_cast<long long>((avg + 127) / 128) * (p.N / 64);
  const long long tiles_ms = static_cast<long long>(S) * static_cast<long long>((avg + 63) / 64) * (p.N / 64);
  if (avg >= 40 && tiles_l >= kNumCu) return kTileL;
  if (avg >= 20 && avg < 64 && (!fp8 || tiles_ms <= 3 * kNumCu)) return kTileMS;
  if (avg >= 8 && avg < 20 && tiles_m >= 2 * kNumCu) return kTileM;
  return t;
}

// e4m3 (W8A8) tiles do half the MFMA work per weight byte: the 64x128 band reaches to 80 rows, the
// 256x256 tile takes over from 64, and below 40 rows the 32x128 tile (t) stays.
static int routed_small_down_tile(const GemmArgs& p, int S, double avg, int t, bool fp8) {
  const long long tiles_ms = static_cast<long long>(S) * static_cast<long long>((avg + 63) / 64) * (p.N / 128);
  const long long tiles_l = static_cast<long long>(S) * static_cast<long long>((avg + 255) / 256) * (p.N / 256);
  if (avg >= 20 && avg < (fp8 ? 80 : 64) && tiles_ms <= 3 * kNumCu) return kTileMS;   // one round of 64x128 workgroups
  if (avg >= (fp8 ? 64 : 36) && tiles_l >= 2 * kNumCu) return kTileL;
  if (fp8 && avg < 40) return t;
  return kTileM;
}

// Tile heuristic (the host knows only the row bound, or a caller's estimate, and the shapes).
// Measured on the routed offsets of the workloads (cold caches; us, gate/up + down):
//  * experts of >= 32 MiB of weights (Mixtral-8x7B) are read from HBM once per row chunk of
//    a segment, so the tile should cover a segment in one chunk: the 32x128 and 64x128 tiles
//    (on the three-stage ring) while the expected rows fit one 32- or 64-row chunk with room
//    for the spread, the bf16 down projection on 128x128 with K split 2, 256x256 from 64 rows
//    (the figures beside each rule below);
//  * small experts (DeepSeek-V2-Lite, Qwen3 local share) stay in cache: gate/up keeps the
//    256x256 tile from ~256 rows per segment of the bound (DeepSeek 4096 tokens 717 vs 710
//    us skewed, 580 vs 657 uniform against 128x128); the down projection (short K) wants
//    more, smaller tiles: 128x128 below ~384 expected rows per segment (Qwen3 2048 tokens:
//    46 vs 62 us), 32x128 below ~96.  Routed bf16 launches of 8 or more segments between 8
//    and 384 expected rows take routed_small_gate_up_tile / routed_small_down_tile instead.
int gemm_pick_tile(const GemmArgs& p, int epi, bool b_fp8) {
  const int S = p.S > 0 ? p.S : 1;
  const double avg_bound = static_cast<double>(p.max_rows) / S;
  const double avg = static_cast<double>(p.rows_hint > 0 ? std::min(p.rows_hint, p.max_rows) : p.max_rows) / S;
  const double expert_bytes = static_cast<double>(p.nb_rows) * p.K * p.k_split * (b_fp8 ? 1 : 2);
  const bool silu = epi_silu(epi);
  int t;
  if (expert_bytes >= 32.0 * 1024 * 1024) {
    // (W8A8 gate/up at 16 rows per expert on the routed, gathered rows of a Mixtral-8x7B
    // decode batch: 182 us on 32x128 tiles, 190 us streamed.  bf16 down projection on 128x128
    // with its K split 2, first from 4 expected rows: Mixtral-8x7B layers at 16 / 20 /
    // 24 / 28 tokens 488 / 499 / 492 / 499 -> 459 / 456 / 462 / 458 us cold, where streaming with a
    // K split of 8 had run to 8 rows; 12 and 32 tokens unchanged.  bf16 gate/up on 256x256 from 64
    // rows: layers at 256 / 320 / 384 / 448 tokens 524 / 543 / 555 / 578 -> 511 / 516 / 544 / 552 us
    // cold against 128x128 up to 128 rows; 192 tokens unchanged.  W8A8 likewise on 256x256 from 64
    // rows: 256 / 320 / 384 / 448 tokens 323 / 340 / 355 / 368 -> 316 / 316 / 334 / 342 us)
    // (W8A8 on 32x128, the three-stage ring, to 24 rows included: 96 tokens 262 -> 244 us cold against
    // 128x128; 16x64 rather than 32x128 below 8 rows, equal on the ring at 4-32 tokens; 64x128, the
    // ring, to 56 rows: 104 / 128 / 160 / 192 / 224 tokens 265 / 273 / 282 / 293 / 301 -> 246 / 253 /
    // 262 / 272 / 281 us against 128x128, but 240 tokens, 60 rows, 313 -> 334)
    if (b_fp8) t = avg < 8 ? kTileXS : avg < 25 ? kTileS : avg < 58 ? kTileMS : avg < 64 ? kTileM : kTileL;
    // bf16 from 0.7 expected rows per expert (3 Mixtral-8x7B tokens 334 -> 318 us; 2 tokens, half a
    // row, 204 -> 229 on the tiles): the gate/up on 32x128 tiles (the three-stage ring) to
    // 24 rows, the down projection on 128x128 (Mixtral-8x7B layers, cold, one box, at 4 / 8 / 12 / 16
    // / 32 / 64 / 96 tokens 332 / 395 / 458 / 460 / 460 / 468 / 464 -> 318 / 353 / 394 / 419 / 421 /
    // 427 / 435 us against streaming both below 24 / 4 rows; at 128 tokens, 32 rows, half the
    // experts take a second 32-row m-tile whose weight panel comes again from HBM: 482 -> 650 us),
    // then on 64x128 tiles (the ring) to 64 rows (104 / 128 / 160 / 192 / 224 / 240 tokens 470 / 480 /
    // 491 / 503 / 515 / 525 -> 438 / 449 / 457 / 469 / 480 / 517 us against 128x128)
    else if (silu) t = avg < 0.7 ? kTileXS : avg < 25 ? kTileS : avg < 64 ? kTileMS : kTileL;
    else t = avg < 0.7 ? kTileXS : avg < 128 ? kTileM : kTileL;
  } else if (silu) {
    // From the row bound, not the expected rows: the Qwen3-30B-A3B 32-expert share at 2048
    // tokens (~3900 local rows, 56-551 per expert) measured 72 us on 256x256 tiles and 89 us on
    // 128x128 (the expected 125 rows per expert would pick the latter).
    t = avg_bound >= 256 ? kTileL : avg_bound >= 96 ? kTileM : avg_bound >= 24 ? kTileS : kTileXS;
    if (S >= 8 && avg_bound < 256) t = routed_small_gate_up_tile(p, S, avg, t, b_fp8);
  } else {
    t = avg < 6 ? kTileXS : avg < 96 ? kTileS : avg < 384 ? kTileM : kTileL;
    if (S >= 8 && avg >= (b_fp8 ? 20 : 8) && avg < 384) t = routed_small_down_tile(p, S, avg, t, b_fp8);
  }
  if (t == kTileL) {
    // fewer 256x256 tiles than CUs (a dense shared-expert launch, say) leaves CUs idle: step down
    const long long mt = static_cast<long long>(p.max_rows) / 256 + S;
    const int oc = gemm_out_cols_per_tile(kTileL, epi);
    if (p.N % oc == 0 && mt * (p.N / oc) * p.k_split < kNumCu) t = kTileM;
  }
  while (t != kTileXS && p.N % gemm_out_cols_per_tile(t, epi) != 0) t = tile_step_down(t);
  return t;
}

int gemm_choose_tile(const GemmArgs& p, int epi, bool b_fp8, bool a_fp8) {
  const int ops = !b_fp8 ? 0 : a_fp8 ? 1 : 2;   // the streaming kernel's operand mode
  const bool stream_ok = stream_gemm_supported(p, epi, ops);
  const double avg = static_cast<double>(p.rows_hint > 0 ? std::min(p.rows_hint, p.max_rows) : p.max_rows) /
                     (p.S > 0 ? p.S : 1);
  const double expert_bytes = static_cast<double>(p.nb_rows) * p.K * p.k_split * (b_fp8 ? 1 : 2);
  int tile;
  bool keep_xs = false;   // a 16x64 choice that is not to be streamed
  if (ops == 2) {
    // W8A16: the LDS tiles DMA the e4m3 weights and widen them at the fragment reads, the
    // streaming kernel widens them in registers on the way to the MFMA.  Experts too large for
    // the caches, measured on the routed Mixtral-8x7B segments (cold, one box; us): streaming
    // below one expected row per segment (1-3 tokens), then 32x128 (64 tokens, single GEMMs:
    // gate/up 162.7 against 208.7 streamed, down with K split 2 75.1 against 106.5), 64x128 from
    // 24 rows (128 tokens: 186.1 / 87.2 against 214.2 / 108.7 on 128x128; 192 tokens: layer 334 ->
    // 304 us against 128x128 from 48 rows), 128x128 from 56 (256 tokens: 248.8 / 117.3 against
    // 257.3 / 140.5 on 64x128); layers at 4 / 8 / 32 / 64 / 128 tokens 206 / 207 / 273 / 293 / 327 ->
    // 185 / 190 / 233 / 260 / 302 us against streaming below 12 rows.
    // Experts that stay in cache read half the bytes of their bf16 form, so the smaller tiles keep
    // the CUs busy longer: 16x64 from one row (not streamed), 32x128 from 4, 64x128 from 20, the
    // down projection on 128x128 from 100 and both on 256x256 from 256 (gate/up / down us,
    // single GEMMs, cold: Qwen3-30B-A3B share 256 tokens 26.1 / 17.9 on 32x128 against 37.3 /
    // 22.8 streamed, 768 tokens 29.7 / 27.3 on 64x128 against 39.8 / 36.2 on 128x128, 2048 tokens
    // 48.9 on 64x128 / 39.0 on 128x128 against 53.8 / 52.6 on 256x256; DeepSeek-V2-Lite 768 tokens
    // 108.8 / 66.9 on 64x128 against 125.9 / 78.9 on 128x128).
    if (expert_bytes >= 32.0 * 1024 * 1024) {
      tile = avg < 1 ? kTileXS : avg < 24 ? kTileS : avg < 56 ? kTileMS : avg < 128 ? kTileM : kTileL;
    } else {
      tile = avg < 4 ? kTileXS : avg < 20 ? kTileS : avg < 100 ? kTileMS : avg < 256 ? (epi_silu(epi) ? kTileMS : kTileM)
                                                                                       : kTileL;
      keep_xs = avg >= 1;
    }
    if (tile == kTileL && (static_cast<long long>(p.max_rows) / 256 + p.S) * (p.N / gemm_out_cols_per_tile(kTileL, epi)) *
                                  p.k_split < kNumCu)
      tile = kTileM;
    while (tile != kTileXS && p.N % gemm_out_cols_per_tile(tile, epi) != 0) tile = tile_step_down(tile);
  } else {
    tile = gemm_pick_tile(p, epi, b_fp8);
    // The bf16 down projection of experts that stay in cache, from one expected row per segment:
    // the 16x64 LDS tile rather than streaming (single launches, cold, one box: DeepSeek-V2-Lite 16
    // / 32 tokens 32.9 / 39.0 us against 43.2 / 43.2 streamed, the Qwen3-30B-A3B share at 32 / 64
    // tokens 25.2 / 28.9 against 25.9 / 31.1; at half a row streaming stays ahead, 19.8 against 21.8).
    keep_xs = ops == 0 && !epi_silu(epi) && expert_bytes < 32.0 * 1024 * 1024 && avg >= 1;
  }
  // a few rows per segment: stream the weights instead of tiling them through LDS, except W8A8 on
  // experts too large for the caches, whose LDS tiles read the weights non-temporally: from two
  // expected rows per expert the 16x64 tile beat streaming (Mixtral-8x7B 8 / 16 tokens, cold: gate/up
  // 113 / 160 us against 131 / 170, down 58 / 73 against 65 / 84; the layers 0.208 / 0.279 ->
  // 0.184-0.194 / 0.260 ms); 1 and 2 tokens stream (their layers 7 and 31 us slower on the LDS
  // tiles), 4 tokens measured either way by 10 % on two boxes.
  const bool w8a8_lds = ops == 1 && expert_bytes >= 32.0 * 1024 * 1024 && avg >= 2.0;
  if (tile == kTileXS && stream_ok && !w8a8_lds && !keep_xs) tile = kTileStream;
  return tile;
}

hipError_t launch_grouped_gemm(const GemmArgs& p, int epi, bool b_fp8, bool a_fp8, int max_rows, int tile,
                               hipStream_t s) {
  if (a_fp8 && !b_fp8) return hipErrorInvalidValue;
  const int ops = !b_fp8 ? 0 : a_fp8 ? 1 : 2;   // the streaming kernel's operand mode
  const bool stream_ok = stream_gemm_supported(p, epi, ops);
  if (tile == kTileAuto) tile = gemm_choose_tile(p, epi, b_fp8, a_fp8);
  if (tile == kTileStream) {
    if (!stream_ok) return hipErrorInvalidValue;
    const double avg = static_cast<double>(max_rows) / (p.S > 0 ? p.S : 1);
    return launch_stream_gemm(p, epi, ops, max_rows, avg > 8 ? 2 : 1, s);
  }
  // Non-temporal weight DMA on the smaller LDS tiles when a segment's expected rows (with half
  // again for skew) fit one m-tile, so each weight panel is read once (decode batches).  Not on
  // the 64x128 tile, which runs mid-size batches of cache-resident experts (with the hint: the
  // Qwen3 share at 384 tokens 86.5 -> 94.9 us warm, DeepSeek-V2-Lite at 256 tokens 222 -> 231 us
  // cold, within noise elsewhere; one box).
  GemmArgs q = p;
  {
    const int bm = tile == kTileM ? 128 : tile == kTileS ? 32 : tile == kTileXS ? 16 : 0;
    const double avg =
        static_cast<double>(p.rows_hint > 0 ? std::min(p.rows_hint, p.max_rows) : p.max_rows) / (p.S > 0 ? p.S : 1);
    q.b_nt = bm > 0 && 3.0 * avg <= 2.0 * bm ? 1 : 0;
  }
  if (epi == kEpiSiluBF16) return b_fp8 ? launch_epi<kEpiSiluBF16, true>(q, max_rows, tile, a_fp8, s)
                                        : launch_epi<kEpiSiluBF16, false>(q, max_rows, tile, false, s);
  if (epi == kEpiStoreBF16) return b_fp8 ? launch_epi<kEpiStoreBF16, true>(q, max_rows, tile, a_fp8, s)
                                         : launch_epi<kEpiStoreBF16, false>(q, max_rows, tile, false, s);
  return b_fp8 ? launch_epi<kEpiStoreF32, true>(q, max_rows, tile, a_fp8, s)
               : launch_epi<kEpiStoreF32, false>(q, max_rows, tile, false, s);
}

template <int BM, int BN, int WGM, int WGN, int EPI, int GM>
static hipError_t launch_cfg_f32(const GemmArgs& p, int max_rows, hipStream_t s) {
  constexpr int OUT_BN = epi_silu(EPI) ? BN / 2 : BN;
  const int n_tiles = p.N / OUT_BN;
  const long long max_mt = (static_cast<long long>(max_rows) + BM - 1) / BM + p.S;
  long long grid = (max_mt * n_tiles * p.k_split + kNumXcd - 1) / kNumXcd * kNumXcd;
  if (grid < kNumXcd) grid = kNumXcd;
  if (grid > 0x7fffffffll) return hipErrorInvalidValue;
  hipLaunchKernelGGL((grouped_gemm_dma_kernel<BM, BN, WGM, WGN, EPI, GM, true>), dim3(static_cast<unsigned>(grid)),
                     dim3(WGM * WGN * 64), 0, s, p);
  return hipGetLastError();
}

template <int EPI>
static hipError_t launch_epi_f32(const GemmArgs& p, int max_rows, int tile, hipStream_t s) {
  switch (tile) {
    case kTileM: return launch_cfg_f32<128, 128, 2, 2, EPI, 4>(p, max_rows, s);
    case kTileS: return launch_cfg_f32<32, 128, 1, 4, EPI, 1>(p, max_rows, s);
    case kTileXS: return launch_cfg_f32<16, 64, 1, 2, EPI, 1>(p, max_rows, s);
    default: return hipErrorInvalidValue;
  }
}

// The fp32 MFMA runs at 1/16 of the bf16 rate, so LDS and memory are far from the limit: the
// 128x128 tile from 32 rows per segment, 32x128 and 16x64 below.
hipError_t launch_grouped_gemm_f32(const GemmArgs& p, int epi, int max_rows, int tile, hipStream_t s) {
  if (epi != kEpiSiluF32 && epi != kEpiStoreF32) return hipErrorInvalidValue;
  if (tile == kTileAuto) {
    const double avg = static_cast<double>(p.rows_hint > 0 ? std::min(p.rows_hint, p.max_rows) : p.max_rows) /
                       (p.S > 0 ? p.S : 1);
    tile = avg >= 32 ? kTileM : avg >= 12 ? kTileS : kTileXS;
  }
  // No 256x256, 64x128 or streaming fp32 kernel: those requests take the 128x128 tile.  Whatever
  // the start, step down until the tile's output columns divide N (the tile's columns are its
  // grid's only bound on N), and refuse a tile that still does not fit rather than leave columns
  // unwritten.
  if (tile == kTileL || tile == kTileMS || tile == kTileStream) tile = kTileM;
  while (tile != kTileXS && p.N % gemm_out_cols_per_tile(tile, epi) != 0) tile = tile_step_down(tile);
  if (p.N % gemm_out_cols_per_tile(tile, epi) != 0) return hipErrorInvalidValue;
  return epi == kEpiSiluF32 ? launch_epi_f32<kEpiSiluF32>(p, max_rows, tile, s)
                            : launch_epi_f32<kEpiStoreF32>(p, max_rows, tile, s);
}

}  // namespace eimoe
