// Internal launcher declarations shared by the kernel files and the C-ABI layer.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace eimoe {

constexpr int kMaxSeg = 1024;  // segments (local experts x source ranks) per grouped GEMM

enum Epilogue : int { kEpiStoreF32 = 0, kEpiStoreBF16 = 1, kEpiSiluBF16 = 2, kEpiSiluF32 = 3 };
constexpr bool epi_silu(int epi) { return epi == kEpiSiluBF16 || epi == kEpiSiluF32; }

// One grouped GEMM launch: for each segment s (rows [seg_off[s], seg_off[s+1]) of A),
// C[rows, :] = A[rows, :] . B[s % e_mod]^T  (B in nn.Linear layout [N_b, K]).
struct GemmArgs {
  const void* a;             // bf16 [*, lda]
  const int32_t* a_rows;     // optional gather map: logical row r reads a[a_rows[r]]
  long long lda;
  const void* b;             // bf16 or fp8-e4m3 [E][N_b][K]
  long long b_estride;       // elements between experts
  const void* const* b_ptrs; // optional: expert e's [N_b][K] weights at b_ptrs[e] (b, b_estride unused
                             // for addressing; b_estride still bounds one expert's elements)
  long long ldb;
  const float* b_scale;      // fp8: per-output-channel scale [E][N_b]; null for bf16
  int nb_rows;               // N_b, rows per expert in b (scale indexing)
  int N;                     // output columns (silu: I)
  int K;                     // reduction length per split
  int up_off;                // silu: first 'up' row in b (= I)
  const int32_t* seg_off;    // [S+1] device
  int S;
  int e_mod;
  void* c;
  void* c_lo;                // SiLU epilogue: also store bf16(h - bf16(h)) here (same layout as c); may be null
  long long ldc;
  long long c_split_stride;  // elements between split-K partial outputs
  int k_split;
  int max_rows;              // rows of A (non-gathered) / of C; segment bounds are clamped to it
  long long a_rows_cap;      // rows in the A buffer (bounds the buffer resource)
  const float* a_scale;      // fp8 A: per-row dequantisation scale, indexed like A (through a_rows)
  int rows_hint;             // expected rows in the segments (tile choice only); 0: max_rows
  int b_nt;                  // set by the launcher: weight DMA non-temporal (each weight read by one m-tile)
};

// Tile shape selector; the launcher maps it to a kernel instantiation.
enum TileCfg : int { kTileAuto = 0, kTileL = 1, kTileM = 2, kTileS = 3, kTileXS = 4, kTileStream = 5, kTileMS = 6 };
// The next smaller LDS tile (256x256 -> 128x128 -> 32x128 -> 16x64; 64x128 -> 32x128), for a tile
// whose output columns do not divide N.
constexpr int tile_step_down(int t) { return t == kTileMS ? kTileS : t + 1; }

hipError_t launch_router_topk(const float* logits, int T, int E, int k, int renorm, int32_t* ids, float* w,
                              hipStream_t s);
// DeepSeek-V3 grouped top-k router (sigmoid, correction bias, group-limited), E <= 512.
hipError_t launch_router_grouped(const float* logits, int T, int E, int k, int n_group, int topk_group,
                                 const float* bias, int renorm, float scaling, int32_t* ids, float* w,
                                 hipStream_t s);
// EPLB logical -> physical ids (replica i mod count of each flat slot i); in place allowed.
hipError_t launch_eplb_map(const int32_t* ids, int n, const int32_t* log2phy, int n_logical, int max_rep,
                           const int32_t* replica_count, int32_t* phys, hipStream_t s);
size_t align_lds_bytes(int n_loc);
// Align: one workgroup, or from kAlignMbMinIds flat ids with a hist buffer of
// align_plan(N, n_loc).hist_ints ints, two launches over align_plan(...).blocks workgroups.
constexpr int kAlignMbMinIds = 4096;
constexpr int kAlignMbIdsPerBlock = 1024;
constexpr int kAlignMbMaxBlocks = 256;
constexpr int kAlignMbMaxCells = 16384;   // chunk-count matrix cells (blocks x n_loc)
struct AlignPlan {
  int blocks;   // 0: the one-workgroup kernel
  int chunk;
  size_t hist_ints;
};
AlignPlan align_plan(int N, int n_loc);
hipError_t launch_align(const int32_t* ids, int T, int k, int e_lo, int n_loc, int32_t* counts, int32_t* offsets,
                        int32_t* sorted_flat, int32_t* sorted_tok, int32_t* pos, int32_t* hist, hipStream_t s);
// The many-workgroup align's second pass alone: chunk b = flat ids [b*chunk, (b+1)*chunk)
// with its per-expert counts in hist[b][n_loc] (chunk a multiple of 4, blocks * n_loc cells
// at most kAlignMbMaxCells).
hipError_t launch_align_place(const int32_t* ids, int T, int k, int e_lo, int n_loc, int blocks, int chunk,
                              const int32_t* hist, int32_t* counts, int32_t* offsets, int32_t* sorted_flat,
                              int32_t* sorted_tok, int32_t* pos, hipStream_t s);
// Router then align; one workgroup runs both when route_align_fused() (small batches);
// otherwise, given hist, the router writes each workgroup's per-expert counts (the align's
// first pass, route_hist_ints(...) ints of hist) and align_place finishes, when that
// chunk-count matrix is small (router.hip); else the router and launch_align.
bool route_align_fused(int T, int E, int k, int n_loc);
size_t route_hist_ints(int T, int E, int k, int n_loc);
hipError_t launch_route_align(const float* logits, int T, int E, int k, int renorm, int e_lo, int n_loc,
                              int32_t* ids, float* w, int32_t* counts, int32_t* offsets, int32_t* sorted_flat,
                              int32_t* sorted_tok, int32_t* pos, int32_t* hist, hipStream_t s);
hipError_t launch_counts_to_offsets(const int32_t* counts, int S, int32_t* offsets, hipStream_t s);
// MoE prologue: residual add + RMSNorm (+ router logits).  Routers of at most
// kPrologueFusedMaxE experts and kPrologueFusedMaxGate bytes of gate weights are dotted in
// the same pass; others (E % 64 == 0) go through the grouped GEMM with the T rows as one
// dense segment, H split over up to kPrologueMaxSplit fp32 planes that a last kernel sums.
// The workspace holds the segment offsets (256 bytes) and the planes.
constexpr int kPrologueFusedMaxE = 32;
constexpr long long kPrologueFusedMaxGate = 128 * 1024;
constexpr int kPrologueMaxSplit = 8;
struct PrologueGemm {
  int tile;
  int k_split;
};
bool prologue_fused_router(int H, int E);
PrologueGemm prologue_router_gemm(int T, int H, int E);
size_t prologue_workspace_bytes(int T, int H, int E);
hipError_t launch_moe_prologue(const void* hidden, const void* residual, const void* norm_w, float eps,
                               const void* gate_w, int T, int H, int E, int logits_bf16, void* res_out, void* normed,
                               float* logits, void* workspace, hipStream_t s);

hipError_t launch_gather_rows(const void* x, int row_bytes, const int32_t* rows, const int32_t* num_rows,
                              int max_rows, void* xs, hipStream_t s);
// shared_n: planes of shared_y, T*H elements apart, summed (1 for a single plane).
hipError_t launch_combine(const void* y, int y_dtype, int n_split, long long split_stride, const int32_t* pos,
                          const float* w, int T, int k, int H, const void* shared_y, int shared_dtype, int shared_n,
                          void* out, int out_dtype, hipStream_t s);
// Decode: the down projection and the weighted combine in one kernel, per (token, 16 output
// columns), for bf16 weights [n_local][H][I] and bf16 h rows found through pos (h_lo optional).
bool down_combine_supported(int H, int I);
hipError_t launch_down_combine(const void* h, const void* h_lo, const void* w_down, int I, int H, const int32_t* ids,
                               const float* w, const int32_t* pos, int T, int k, int e_lo, const void* shared_y,
                               int shared_dtype, int shared_n, void* out, int out_dtype, hipStream_t s);
// epi: Epilogue; b_fp8: B is e4m3; max_rows bounds the grid; tile: TileCfg.
// a_fp8: A and B are both fp8-e4m3 (W8A8 on the fp8 MFMA); b_fp8 alone: W8A16.
hipError_t launch_grouped_gemm(const GemmArgs& p, int epi, bool b_fp8, bool a_fp8, int max_rows, int tile,
                               hipStream_t s);
// Tile for a launch: from the expected rows per segment, the output width and the bytes of
// one expert's weights (rows_hint/max_rows, p.S, p.N, p.K * p.k_split, nb_rows).
int gemm_pick_tile(const GemmArgs& p, int epi, bool b_fp8);
// The tile an automatic launch takes (kTileStream included): gemm_pick_tile's choice, the W8A16
// rule, and the switch to the weight-streaming kernel where it applies.
int gemm_choose_tile(const GemmArgs& p, int epi, bool b_fp8, bool a_fp8);
// Weight-streaming kernel (stream.hip) for segments of a few rows.  ops: 0 bf16 x bf16, 1 e4m3 x
// e4m3 (W8A8, with p.a_scale / p.b_scale), 2 e4m3 weights x bf16 activations (W8A16, p.b_scale).
bool stream_gemm_supported(const GemmArgs& p, int epi, int ops);
// widest output columns per streaming task (0: unsupported); fp8: e4m3 weights (128-wide k steps)
int stream_out_cols(int N, int epi, bool fp8);
hipError_t launch_stream_gemm(const GemmArgs& p, int epi, int ops, int max_rows, int mblk, hipStream_t s);
int gemm_out_cols_per_tile(int tile, int epi);
// fp32 operands on the fp32 MFMA (v_mfma_f32_16x16x4f32): A, B and the output in fp32 (epi
// kEpiSiluF32 or kEpiStoreF32); LDS-tiled kernels only (tiles 128x128, 32x128, 16x64).
hipError_t launch_grouped_gemm_f32(const GemmArgs& p, int epi, int max_rows, int tile, hipStream_t s);

// Base of expert e's weights: the pointer table when given, else b + e * b_estride elements.
__device__ __forceinline__ const uint8_t* expert_weights(const GemmArgs& p, int e, int elem_bytes) {
  return p.b_ptrs ? static_cast<const uint8_t*>(p.b_ptrs[e])
                  : static_cast<const uint8_t*>(p.b) + static_cast<long long>(e) * p.b_estride * elem_bytes;
}
hipError_t launch_quantize_rows_fp8(const void* x, int dtype, long long rows, int cols, uint8_t* q, float* scale,
                                    hipStream_t s);

}  // namespace eimoe
