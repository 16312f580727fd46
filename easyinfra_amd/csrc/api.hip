// C-ABI entry points (declared in include/eimoe.h): host-side validation, then
// stream-ordered launches.  No device allocation, no host synchronisation.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <mutex>

#include "../../include/eimoe.h"
#include "common.h"
#include "kernels.h"

using namespace eimoe;

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(EIMOE_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  g_err[0] = '\0';
  return EIMOE_OK;
}

#define REQUIRE_PTR(p)                                                      \
  do {                                                                      \
    if ((p) == nullptr) return fail(EIMOE_ERR_NULL, "%s is NULL", #p);      \
  } while (0)

inline hipStream_t S(void* s) { return static_cast<hipStream_t>(s); }

// A second stream per (host thread, device) with its fork/join events, created on first
// use and kept until eimoe_release_streams() on that thread (or the process's end): the fused
// layer runs the shared experts on it so
// their launches overlap the routed ones (each alone ends in a mostly idle CU round).
// Default priority, non-blocking; the fork/join through events also holds under graph
// capture of the caller's stream.
struct AuxStream {
  hipStream_t stream = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
};
constexpr int kMaxDevices = 64;

thread_local AuxStream g_aux[kMaxDevices];

// *out stays null when the stream does not exist yet and may not be created now (the
// caller's stream is capturing: creating a stream then would invalidate the capture).
hipError_t aux_stream(AuxStream** out, bool may_create) {
  AuxStream* aux = g_aux;
  *out = nullptr;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  AuxStream& a = aux[dev];
  if (!a.stream) {
    if (!may_create) return hipSuccess;
    if ((e = hipStreamCreateWithFlags(&a.stream, hipStreamNonBlocking)) != hipSuccess) return e;
    if ((e = hipEventCreateWithFlags(&a.fork, hipEventDisableTiming)) != hipSuccess) return e;
    if ((e = hipEventCreateWithFlags(&a.join, hipEventDisableTiming)) != hipSuccess) return e;
  }
  *out = &a;
  return hipSuccess;
}

inline size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

int elem_size(int dt) { return dt == EIMOE_F32 ? 4 : dt == EIMOE_BF16 ? 2 : dt == EIMOE_FP8 ? 1 : 0; }

int check_gemm_common(int max_rows, int n_seg, int e_mod) {
  if (max_rows < 0) return fail(EIMOE_ERR_SHAPE, "max_rows=%d < 0", max_rows);
  if (n_seg < 1 || n_seg > EIMOE_MAX_SEGMENTS)
    return fail(EIMOE_ERR_SHAPE, "n_seg=%d outside [1,%d]", n_seg, EIMOE_MAX_SEGMENTS);
  if (e_mod < 1) return fail(EIMOE_ERR_SHAPE, "e_mod=%d < 1", e_mod);
  return EIMOE_OK;
}

int check_tile(int tile, int epi, int N) {
  if (tile < EIMOE_TILE_AUTO || tile > EIMOE_TILE_64x128) return fail(EIMOE_ERR_SHAPE, "tile=%d unknown", tile);
  if (tile != EIMOE_TILE_AUTO) {
    const int oc = gemm_out_cols_per_tile(tile, epi);
    if (N % oc != 0) return fail(EIMOE_ERR_ALIGN, "N=%d not a multiple of the tile's %d output columns", N, oc);
  }
  return EIMOE_OK;
}

// Split of the down projection's K.  Work items (m-tiles x n-tiles x split) run in rounds
// of kNumCu workgroups, so a launch whose tile count sits just past a multiple of kNumCu
// wastes most of its last round (the Mixtral prefill layer: ~1104 tiles = 4.3 rounds).
// Each candidate split is charged its padded rounds, in units of one full-K tile, plus the
// HBM round trip of its extra partial planes (written here, read back by the combine);
// small launches also split until they fill the GPU twice over.
int pick_down_split(int max_rows, int rows_hint, int n_local, int H, int I, int y_elem, bool w8a8) {
  GemmArgs q{};
  q.max_rows = max_rows;
  q.rows_hint = rows_hint;
  q.S = n_local;
  q.N = H;
  q.K = I;
  q.k_split = 1;
  q.nb_rows = H;
  // the tile the launch will take (the W8A16 layer is costed as bf16: its workspace query does not
  // see the weight type; any split chosen here is valid for it, at worst on its LDS tiles)
  const int tile = gemm_choose_tile(q, kEpiStoreF32, w8a8, w8a8);
  if (tile == kTileStream) {
    // Few rows per segment: the weight-streaming kernel runs one workgroup per (segment,
    // column group, 32-row chunk, split).  Split until there are about 6 workgroups per CU
    // while the split divides the K steps (64 bf16 / 128 e4m3 bytes each) and leaves each
    // split >= 8 of them (Mixtral 64-token down, bf16: split 1/2/4/8 = 200/192/181/190 us).
    const int steps = w8a8 ? I / 128 : I / 64;
    const int cols = std::max(stream_out_cols(H, kEpiStoreF32, w8a8), 16);
    const long long tasks = (std::min<long long>(n_local, max_rows) + (max_rows + 31) / 32) * (H / cols);
    int split = 1;
    while (split < 8 && tasks * split < 6ll * kNumCu && steps % (split * 2) == 0 && steps / (split * 2) >= 8)
      split *= 2;
    return split;
  }
  // Experts too large for the caches, few rows each (decode batches on the LDS tiles): the
  // launch streams weights at the HBM rate whatever the tile count, and split 2 measured
  // best (Mixtral 64 tokens, 128x128 bf16: split 1/2/4/8 = 226/159/163/171 us; 32x128
  // e4m3: 109/84/99/94).
  const double expert_bytes = static_cast<double>(H) * I * (w8a8 ? 1 : 2);
  if (expert_bytes >= 32.0 * 1024 * 1024 && tile != kTileL)
    return (I / (w8a8 ? 128 : 64)) % 2 == 0 ? 2 : 1;
  if (w8a8) I /= 2;   // e4m3 tiles run at twice the bf16 rate: cost them as half the K
  const int bm = tile == kTileL ? 256 : tile == kTileM ? 128 : tile == kTileMS ? 64 : tile == kTileS ? 32 : 16;
  const int bn = gemm_out_cols_per_tile(tile, kEpiStoreF32);
  const int rows = rows_hint > 0 ? std::min(rows_hint, max_rows) : max_rows;
  // m-tiles in full-tile units from the expected rows per segment: whole tiles plus the remainder's
  // tile, which takes a quarter, half or full height (a short tile costs its share of a round)
  const int segs = std::max(1, std::min(n_local, rows));
  const double per = static_cast<double>(rows) / segs;
  double mt;
  if (tile == kTileL) {
    // The persistent 256x256 kernel: every m-tile of a segment costs about a full tile whatever its
    // height, and routed segments scatter around the mean, so an expected count just past a
    // multiple of 256 rows gives about half the segments one more m-tile.  Count
    // E[ceil(rows / 256)] with the rows ~ normal(mean, sqrt(mean)).
    const double sd = std::sqrt(std::max(per, 1.0));
    double e = 0.0;
    for (int j = 0; j * static_cast<double>(bm) < per + 6.0 * sd; ++j)
      e += 0.5 * std::erfc((j * static_cast<double>(bm) + 0.5 - per) / (sd * std::sqrt(2.0)));
    mt = segs * e;
  } else {
    // m-tiles in full-tile units from the expected rows per segment: whole tiles plus the
    // remainder's tile, which takes a quarter, half or full height (a short tile costs its share)
    const double rem = per - std::floor(per / bm) * bm;
    const double rem_tile = rem <= 0.0 ? 0.0 : rem <= bm / 4 ? 0.25 : rem <= bm / 2 ? 0.5 : 1.0;
    mt = segs * (std::floor(per / bm) + rem_tile);
  }
  const double work = mt * (H / bn);                                              // full-tile units
  const long long tiles = static_cast<long long>(segs * std::ceil(per / bm)) * (H / bn);   // workgroups
  constexpr double kTileFlops = 4.7e12;   // measured bf16 GEMM rate per CU, FLOP/s
  constexpr double kHbm = 5.0e12;         // achieved HBM rate for plane traffic, B/s
  const double t_tile = 2.0 * bm * bn * static_cast<double>(I) / kTileFlops;
  const double t_plane = 2.0 * static_cast<double>(max_rows) * H * y_elem / kHbm;
  // Four or more rounds of full-K 256x256 tiles: the partial last round costs little under the
  // power-limited clock, and each extra plane is a round trip of the whole output (the Mixtral-8x7B
  // 8192-token layer: one split)
  if (tile == kTileL && work >= 4.0 * kNumCu) return 1;
  int best = 1;
  double best_cost = 1e300;
  for (int split = 1; split <= 8; split *= 2) {
    if (I % (64 * split) != 0) break;
    const long long items = tiles * split;
    const double rounds = std::ceil(work * split / kNumCu);
    double cost = rounds / split * t_tile + (split - 1) * t_plane;
    // too few workgroups to fill the GPU: twice over for the one-tile-per-workgroup kernels, once
    // for the persistent 256x256 one (whose workgroups walk their tiles)
    const bool few = tile == kTileL ? work * split < kNumCu : items < 2 * kNumCu;
    if (few && split < 8 && I % (128 * split) == 0) cost = 1e300;
    if (cost < best_cost * 0.98) {
      best_cost = cost;
      best = split;
    }
  }
  return best;
}

struct FusedLayout {
  size_t ids, w, counts, offsets, sorted_flat, sorted_tok, pos, hist, h, h_lo, y, sh_off, sh_h, sh_h_lo, sh_y, xq, sx,
      hq, sh, total;
  int k_split;
  int h_terms;   // 2 with EIMOE_H_SPLIT: h stored as bf16 hi + lo, each projected into its own y planes
  int y_dtype;
  int rows_hint;
};

// Expected rows kept by an expert-parallel share of n_local of E experts (uniform routing):
// the tile choice's estimate; the launches stay bounded by all T*k rows.
int local_rows_hint(int T, int k, int E, int n_local) {
  const long long A = static_cast<long long>(T) * k;
  return n_local < E ? static_cast<int>(std::max<long long>(A * n_local / E, 1)) : static_cast<int>(A);
}

FusedLayout fused_layout(int T, int H, int I, int E, int k, int n_local, int Is, int out_dtype, int flags) {
  FusedLayout L{};
  const size_t A = static_cast<size_t>(T) * k;
  L.rows_hint = local_rows_hint(T, k, E, n_local);
  L.h_terms = (flags & EIMOE_H_SPLIT) ? 2 : 1;
  // The per-assignment outputs stay in fp32 whatever the output type: the combine sums a token's
  // slots (and split-K planes) in fp32 and rounds once.  With bf16 planes each partial sum was
  // rounded before the combine, which put the 8192-token Mixtral-8x7B layer's bf16 output 5.8e-2
  // from the fp32 oracle against 2.0e-2 + half an ulp for a single rounding.
  (void)out_dtype;
  L.y_dtype = EIMOE_F32;
  const size_t hb = (flags & EIMOE_FP32) ? 4 : 2;   // bytes per h element
  L.k_split = pick_down_split(static_cast<int>(A), L.rows_hint, n_local, H, I,
                              static_cast<int>(elem_size(L.y_dtype)), (flags & EIMOE_W8A8) != 0);
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o += align256(bytes);
    return at;
  };
  L.ids = take(A * 4);
  L.w = take(A * 4);
  L.counts = take(static_cast<size_t>(n_local) * 4);
  L.offsets = take(static_cast<size_t>(n_local + 1) * 4);
  L.sorted_flat = take(A * 4);
  L.sorted_tok = take(A * 4);
  L.pos = take(A * 4);
  L.hist = take(std::max(align_plan(static_cast<int>(A), n_local).hist_ints, route_hist_ints(T, E, k, n_local)) * 4);
  L.h = take(A * I * hb);
  if (L.h_terms == 2) L.h_lo = take(A * I * 2);
  L.y = take(static_cast<size_t>(L.h_terms) * L.k_split * A * H * elem_size(L.y_dtype));
  if (flags & EIMOE_W8A8) {
    L.xq = take(static_cast<size_t>(T) * H);
    L.sx = take(static_cast<size_t>(T) * 4);
    L.hq = take(A * I);
    L.sh = take(A * 4);
  }
  if (Is > 0) {
    L.sh_off = take(2 * 4);
    L.sh_h = take(static_cast<size_t>(T) * Is * hb);
    if (L.h_terms == 2) L.sh_h_lo = take(static_cast<size_t>(T) * Is * 2);
    L.sh_y = take(static_cast<size_t>(L.h_terms) * T * H * elem_size(L.y_dtype));
  }
  L.total = o;
  return L;
}

__global__ void dense_segment_kernel(int32_t* off, int T) {
  if (threadIdx.x == 0) {
    off[0] = 0;
    off[1] = T;
  }
}

int run_gate_up(const void* a, const int32_t* a_rows, long long a_nrows, int lda, const void* w, int w_dtype,
                const float* w_scale, int H, int I, const int32_t* seg, int n_seg, int e_mod, int max_rows, void* h,
                int tile, hipStream_t s, const float* a_scale = nullptr, int rows_hint = 0, void* h_lo = nullptr) {
  GemmArgs p{};
  p.c_lo = h_lo;
  p.rows_hint = rows_hint;
  p.a = a;
  p.a_rows = a_rows;
  p.lda = lda;
  p.b = w;
  p.b_estride = 2ll * I * H;
  p.ldb = H;
  p.b_scale = w_scale;
  p.nb_rows = 2 * I;
  p.N = I;
  p.K = H;
  p.up_off = I;
  p.seg_off = seg;
  p.S = n_seg;
  p.e_mod = e_mod;
  p.c = h;
  p.ldc = I;
  p.c_split_stride = 0;
  p.k_split = 1;
  p.max_rows = max_rows;
  p.a_rows_cap = a_rows ? a_nrows : max_rows;
  p.a_scale = a_scale;
  if (w_dtype == EIMOE_F32) return hip_check(launch_grouped_gemm_f32(p, kEpiSiluF32, max_rows, tile, s), "gate_up gemm");
  return hip_check(launch_grouped_gemm(p, kEpiSiluBF16, w_dtype == EIMOE_FP8, a_scale != nullptr, max_rows, tile, s),
                   "gate_up gemm");
}

int run_down(const void* h, int I, const void* w, int w_dtype, const float* w_scale, int H, const int32_t* seg,
             int n_seg, int e_mod, int max_rows, void* y, int y_dtype, int k_split, int tile, hipStream_t s,
             const float* h_scale = nullptr, int rows_hint = 0) {
  GemmArgs p{};
  p.rows_hint = rows_hint;
  p.a = h;
  p.a_rows = nullptr;
  p.lda = I;
  p.b = w;
  p.b_estride = static_cast<long long>(H) * I;
  p.ldb = I;
  p.b_scale = w_scale;
  p.nb_rows = H;
  p.N = H;
  p.K = I / k_split;
  p.up_off = 0;
  p.seg_off = seg;
  p.S = n_seg;
  p.e_mod = e_mod;
  p.c = y;
  p.ldc = H;
  p.c_split_stride = static_cast<long long>(max_rows) * H;
  p.k_split = k_split;
  p.max_rows = max_rows;
  p.a_rows_cap = max_rows;
  p.a_scale = h_scale;
  const int epi = y_dtype == EIMOE_F32 ? kEpiStoreF32 : kEpiStoreBF16;
  if (w_dtype == EIMOE_F32) return hip_check(launch_grouped_gemm_f32(p, epi, max_rows, tile, s), "down gemm");
  return hip_check(launch_grouped_gemm(p, epi, w_dtype == EIMOE_FP8, h_scale != nullptr, max_rows, tile, s),
                   "down gemm");
}

}  // namespace

extern "C" {

int eimoe_abi_version(void) { return EIMOE_ABI_VERSION; }

int eimoe_release_streams(void) {
  int prev = 0;
  int rc = hip_check(hipGetDevice(&prev), "current device");
  if (rc) return rc;
  for (int dev = 0; dev < kMaxDevices; ++dev) {
    AuxStream& a = g_aux[dev];
    if (!a.stream && !a.fork && !a.join) continue;
    int r = hip_check(hipSetDevice(dev), "set device");
    // the stream's work (shared experts of a layer still running) ends before it is destroyed;
    // each handle is cleared once destroyed, so a call after a failure here releases only the rest
    if (!r && a.stream) r = hip_check(hipStreamSynchronize(a.stream), "aux stream synchronize");
    if (!r && a.stream && !(r = hip_check(hipStreamDestroy(a.stream), "aux stream destroy"))) a.stream = nullptr;
    if (!r && a.fork && !(r = hip_check(hipEventDestroy(a.fork), "fork event destroy"))) a.fork = nullptr;
    if (!r && a.join && !(r = hip_check(hipEventDestroy(a.join), "join event destroy"))) a.join = nullptr;
    if (r) {
      hipSetDevice(prev);
      return r;
    }
    a = AuxStream{};
  }
  return hip_check(hipSetDevice(prev), "restore device");
}

const char* eimoe_last_error(void) { return g_err; }

int eimoe_router_topk(const float* logits, int T, int E, int k, int renormalize, int32_t* topk_ids,
                      float* topk_weights, void* stream) {
  if (T < 0) return fail(EIMOE_ERR_SHAPE, "T=%d < 0", T);
  if (E < 1 || E > EIMOE_MAX_EXPERTS) return fail(EIMOE_ERR_SHAPE, "E=%d outside [1,%d]", E, EIMOE_MAX_EXPERTS);
  if (k < 1 || k > E || k > EIMOE_MAX_TOPK)
    return fail(EIMOE_ERR_SHAPE, "k=%d outside [1,min(E=%d,%d)]", k, E, EIMOE_MAX_TOPK);
  if (T == 0) return EIMOE_OK;
  REQUIRE_PTR(logits);
  REQUIRE_PTR(topk_ids);
  REQUIRE_PTR(topk_weights);
  return hip_check(launch_router_topk(logits, T, E, k, renormalize ? 1 : 0, topk_ids, topk_weights, S(stream)),
                   "router_topk");
}

int eimoe_router_grouped_topk(const float* logits, int T, int E, int k, int n_group, int topk_group,
                              const float* bias, int renormalize, float scaling, int32_t* topk_ids,
                              float* topk_weights, void* stream) {
  if (T < 0) return fail(EIMOE_ERR_SHAPE, "T=%d < 0", T);
  if (E < 2 || E > EIMOE_MAX_EXPERTS) return fail(EIMOE_ERR_SHAPE, "E=%d outside [2,%d]", E, EIMOE_MAX_EXPERTS);
  if (k < 1 || k > E || k > EIMOE_MAX_TOPK)
    return fail(EIMOE_ERR_SHAPE, "k=%d outside [1,min(E=%d,%d)]", k, E, EIMOE_MAX_TOPK);
  if (n_group < 1 || E % n_group || E / n_group < 2)
    return fail(EIMOE_ERR_SHAPE, "n_group=%d must divide E=%d into groups of >= 2 experts", n_group, E);
  if (topk_group < 1 || topk_group > n_group)
    return fail(EIMOE_ERR_SHAPE, "topk_group=%d outside [1,n_group=%d]", topk_group, n_group);
  if (T == 0) return EIMOE_OK;
  REQUIRE_PTR(logits);
  REQUIRE_PTR(topk_ids);
  REQUIRE_PTR(topk_weights);
  return hip_check(launch_router_grouped(logits, T, E, k, n_group, topk_group, bias, renormalize ? 1 : 0, scaling,
                                         topk_ids, topk_weights, S(stream)),
                   "router_grouped_topk");
}

int eimoe_eplb_map(const int32_t* topk_ids, int T, int k, const int32_t* log2phy, int n_logical, int max_replicas,
                   const int32_t* replica_count, int32_t* physical_ids, void* stream) {
  if (T < 0 || k < 1) return fail(EIMOE_ERR_SHAPE, "T=%d, k=%d", T, k);
  if (static_cast<long long>(T) * k > 0x7fffffffll) return fail(EIMOE_ERR_SHAPE, "T*k overflows int32");
  if (n_logical < 1 || max_replicas < 1 || static_cast<long long>(n_logical) * max_replicas > 0x7fffffffll)
    return fail(EIMOE_ERR_SHAPE, "n_logical=%d, max_replicas=%d", n_logical, max_replicas);
  if (T == 0) return EIMOE_OK;
  REQUIRE_PTR(topk_ids);
  REQUIRE_PTR(log2phy);
  REQUIRE_PTR(replica_count);
  REQUIRE_PTR(physical_ids);
  return hip_check(launch_eplb_map(topk_ids, T * k, log2phy, n_logical, max_replicas, replica_count, physical_ids,
                                   S(stream)),
                   "eplb_map");
}

size_t eimoe_align_workspace_bytes(int T, int k, int n_local) {
  if (T < 0 || k < 1 || n_local < 1 || static_cast<long long>(T) * k > 0x7fffffffll) return 0;
  return align_plan(T * k, n_local).hist_ints * sizeof(int32_t);
}

int eimoe_align(const int32_t* topk_ids, int T, int k, int e_lo, int n_local, int32_t* counts, int32_t* offsets,
                int32_t* sorted_flat, int32_t* sorted_tok, int32_t* pos, void* workspace, size_t workspace_bytes,
                void* stream) {
  if (T < 0) return fail(EIMOE_ERR_SHAPE, "T=%d < 0", T);
  if (k < 1 || k > EIMOE_MAX_TOPK) return fail(EIMOE_ERR_SHAPE, "k=%d outside [1,%d]", k, EIMOE_MAX_TOPK);
  if (n_local < 1 || n_local > EIMOE_MAX_EXPERTS)
    return fail(EIMOE_ERR_SHAPE, "n_local=%d outside [1,%d]", n_local, EIMOE_MAX_EXPERTS);
  if (e_lo < 0) return fail(EIMOE_ERR_SHAPE, "e_lo=%d < 0", e_lo);
  if (static_cast<long long>(T) * k > 0x7fffffffll) return fail(EIMOE_ERR_SHAPE, "T*k overflows int32");
  REQUIRE_PTR(counts);
  REQUIRE_PTR(offsets);
  if (T > 0) {
    REQUIRE_PTR(topk_ids);
    REQUIRE_PTR(sorted_flat);
    REQUIRE_PTR(sorted_tok);
    REQUIRE_PTR(pos);
  }
  // the many-workgroup sort when the caller's workspace holds its chunk counts
  const size_t need = eimoe_align_workspace_bytes(T, k, n_local);
  int32_t* hist = (workspace != nullptr && need > 0 && workspace_bytes >= need) ? static_cast<int32_t*>(workspace)
                                                                                : nullptr;
  return hip_check(launch_align(topk_ids, T, k, e_lo, n_local, counts, offsets, sorted_flat, sorted_tok, pos, hist,
                                S(stream)),
                   "align");
}

int eimoe_route_align(const float* logits, int T, int E, int k, int renormalize, int e_lo, int n_local,
                      int32_t* topk_ids, float* topk_weights, int32_t* counts, int32_t* offsets,
                      int32_t* sorted_flat, int32_t* sorted_tok, int32_t* pos, void* stream) {
  if (T < 0) return fail(EIMOE_ERR_SHAPE, "T=%d < 0", T);
  if (E < 1 || E > EIMOE_MAX_EXPERTS) return fail(EIMOE_ERR_SHAPE, "E=%d outside [1,%d]", E, EIMOE_MAX_EXPERTS);
  if (k < 1 || k > E || k > EIMOE_MAX_TOPK)
    return fail(EIMOE_ERR_SHAPE, "k=%d outside [1,min(E=%d,%d)]", k, E, EIMOE_MAX_TOPK);
  if (n_local < 1 || n_local > EIMOE_MAX_EXPERTS)
    return fail(EIMOE_ERR_SHAPE, "n_local=%d outside [1,%d]", n_local, EIMOE_MAX_EXPERTS);
  if (e_lo < 0) return fail(EIMOE_ERR_SHAPE, "e_lo=%d < 0", e_lo);
  if (static_cast<long long>(T) * k > 0x7fffffffll) return fail(EIMOE_ERR_SHAPE, "T*k overflows int32");
  REQUIRE_PTR(counts);
  REQUIRE_PTR(offsets);
  if (T > 0) {
    REQUIRE_PTR(logits);
    REQUIRE_PTR(topk_ids);
    REQUIRE_PTR(topk_weights);
    REQUIRE_PTR(sorted_flat);
    REQUIRE_PTR(sorted_tok);
    REQUIRE_PTR(pos);
  }
  return hip_check(launch_route_align(logits, T, E, k, renormalize ? 1 : 0, e_lo, n_local, topk_ids, topk_weights,
                                      counts, offsets, sorted_flat, sorted_tok, pos, nullptr, S(stream)),
                   "route_align");
}

int eimoe_counts_to_offsets(const int32_t* counts, int n_seg, int32_t* offsets, void* stream) {
  if (n_seg < 1 || n_seg > EIMOE_MAX_SEGMENTS)
    return fail(EIMOE_ERR_SHAPE, "n_seg=%d outside [1,%d]", n_seg, EIMOE_MAX_SEGMENTS);
  REQUIRE_PTR(counts);
  REQUIRE_PTR(offsets);
  return hip_check(launch_counts_to_offsets(counts, n_seg, offsets, S(stream)), "counts_to_offsets");
}

int eimoe_gather(const void* x, int dtype, int H, const int32_t* rows, const int32_t* num_rows, int max_rows,
                 void* xs, void* stream) {
  if (dtype != EIMOE_F32 && dtype != EIMOE_BF16) return fail(EIMOE_ERR_DTYPE, "gather dtype=%d", dtype);
  if (H < 1) return fail(EIMOE_ERR_SHAPE, "H=%d < 1", H);
  const int row_bytes = H * elem_size(dtype);
  if (row_bytes % 16) return fail(EIMOE_ERR_ALIGN, "row bytes %d not a multiple of 16", row_bytes);
  if (max_rows < 0) return fail(EIMOE_ERR_SHAPE, "max_rows=%d < 0", max_rows);
  if (max_rows == 0) return EIMOE_OK;
  REQUIRE_PTR(x);
  REQUIRE_PTR(rows);
  REQUIRE_PTR(num_rows);
  REQUIRE_PTR(xs);
  return hip_check(launch_gather_rows(x, row_bytes, rows, num_rows, max_rows, xs, S(stream)), "gather");
}

int eimoe_gemm_gate_up_silu(const void* a, const int32_t* a_rows, int a_nrows, int lda, const void* w_gate_up, int w_dtype,
                            const float* w_scale, int H, int I, const int32_t* seg_offsets, int n_seg, int e_mod,
                            int max_rows, void* h, int tile, void* stream) {
  int rc = check_gemm_common(max_rows, n_seg, e_mod);
  if (rc) return rc;
  if (w_dtype != EIMOE_BF16 && w_dtype != EIMOE_FP8 && w_dtype != EIMOE_F32)
    return fail(EIMOE_ERR_DTYPE, "w_dtype=%d", w_dtype);
  if (H < 64 || H % 64) return fail(EIMOE_ERR_ALIGN, "H=%d must be a positive multiple of 64", H);
  if (I < 32 || I % 32) return fail(EIMOE_ERR_ALIGN, "I=%d must be a positive multiple of 32", I);
  if (lda < H) return fail(EIMOE_ERR_SHAPE, "lda=%d < H=%d", lda, H);
  if (a_rows && a_nrows < 1) return fail(EIMOE_ERR_SHAPE, "a_nrows=%d < 1 with a row map", a_nrows);
  if (!a_rows) a_nrows = max_rows;
  const long long ab = w_dtype == EIMOE_F32 ? 4 : 2;   // fp32 weights take fp32 activations
  if (static_cast<long long>(a_nrows) * lda * ab > 0x7fffffffll)
    return fail(EIMOE_ERR_SHAPE, "A buffer (%d rows x %d) exceeds 2 GiB", a_nrows, lda);
  if (2ll * I * H * elem_size(w_dtype) > 0x7fffffffll)
    return fail(EIMOE_ERR_SHAPE, "one expert's gate/up weights exceed 2 GiB");
  if (w_dtype == EIMOE_F32 && static_cast<long long>(max_rows) * I * 4 > 0x7fffffffll)
    return fail(EIMOE_ERR_SHAPE, "h (%d rows x %d, fp32) exceeds 2 GiB", max_rows, I);
  if (lda % 8) return fail(EIMOE_ERR_ALIGN, "lda=%d must be a multiple of 8", lda);
  if ((rc = check_tile(tile, kEpiSiluBF16, I))) return rc;
  if (max_rows == 0) return EIMOE_OK;
  REQUIRE_PTR(a);
  REQUIRE_PTR(w_gate_up);
  REQUIRE_PTR(seg_offsets);
  REQUIRE_PTR(h);
  if (w_dtype == EIMOE_FP8) REQUIRE_PTR(w_scale);
  return run_gate_up(a, a_rows, a_nrows, lda, w_gate_up, w_dtype, w_scale, H, I, seg_offsets, n_seg, e_mod, max_rows,
                     h, tile, S(stream));
}

int eimoe_gemm_down(const void* h, int I, const void* w_down, int w_dtype, const float* w_scale, int H,
                    const int32_t* seg_offsets, int n_seg, int e_mod, int max_rows, void* y, int y_dtype,
                    int k_split, int tile, void* stream) {
  int rc = check_gemm_common(max_rows, n_seg, e_mod);
  if (rc) return rc;
  if (w_dtype != EIMOE_BF16 && w_dtype != EIMOE_FP8 && w_dtype != EIMOE_F32)
    return fail(EIMOE_ERR_DTYPE, "w_dtype=%d", w_dtype);
  if (y_dtype != EIMOE_BF16 && y_dtype != EIMOE_F32) return fail(EIMOE_ERR_DTYPE, "y_dtype=%d", y_dtype);
  if (w_dtype == EIMOE_F32 && y_dtype != EIMOE_F32) return fail(EIMOE_ERR_DTYPE, "fp32 weights write fp32 y");
  if (H < 64 || H % 64) return fail(EIMOE_ERR_ALIGN, "H=%d must be a positive multiple of 64", H);
  if (k_split < 1 || k_split > 64) return fail(EIMOE_ERR_SHAPE, "k_split=%d outside [1,64]", k_split);
  if (I < 64 || I % (64 * k_split))
    return fail(EIMOE_ERR_ALIGN, "I=%d must be a positive multiple of 64*k_split=%d", I, 64 * k_split);
  if ((rc = check_tile(tile, kEpiStoreF32, H))) return rc;
  if (static_cast<long long>(max_rows) * I * (w_dtype == EIMOE_F32 ? 4 : 2) > 0x7fffffffll)
    return fail(EIMOE_ERR_SHAPE, "h (%d rows x %d) exceeds 2 GiB", max_rows, I);
  if (static_cast<long long>(H) * I * elem_size(w_dtype) > 0x7fffffffll)
    return fail(EIMOE_ERR_SHAPE, "one expert's down weights exceed 2 GiB");
  if (max_rows == 0) return EIMOE_OK;
  REQUIRE_PTR(h);
  REQUIRE_PTR(w_down);
  REQUIRE_PTR(seg_offsets);
  REQUIRE_PTR(y);
  if (w_dtype == EIMOE_FP8) REQUIRE_PTR(w_scale);
  return run_down(h, I, w_down, w_dtype, w_scale, H, seg_offsets, n_seg, e_mod, max_rows, y, y_dtype, k_split, tile,
                  S(stream));
}

int eimoe_gemm_gate_up_silu_w8a8(const void* a, const float* a_scale, const int32_t* a_rows, int a_nrows, int lda,
                                 const void* w_gate_up, const float* w_scale, int H, int I,
                                 const int32_t* seg_offsets, int n_seg, int e_mod, int max_rows, void* h, int tile,
                                 void* stream) {
  int rc = check_gemm_common(max_rows, n_seg, e_mod);
  if (rc) return rc;
  if (H < 128 || H % 128) return fail(EIMOE_ERR_ALIGN, "H=%d must be a positive multiple of 128", H);
  if (I < 32 || I % 32) return fail(EIMOE_ERR_ALIGN, "I=%d must be a positive multiple of 32", I);
  if (lda < H || lda % 16) return fail(EIMOE_ERR_SHAPE, "lda=%d must be >= H=%d and a multiple of 16", lda, H);
  if (a_rows && a_nrows < 1) return fail(EIMOE_ERR_SHAPE, "a_nrows=%d < 1 with a row map", a_nrows);
  if (!a_rows) a_nrows = max_rows;
  if (static_cast<long long>(a_nrows) * lda > 0x7fffffffll) return fail(EIMOE_ERR_SHAPE, "A buffer exceeds 2 GiB");
  if (2ll * I * H > 0x7fffffffll) return fail(EIMOE_ERR_SHAPE, "one expert's gate/up weights exceed 2 GiB");
  if ((rc = check_tile(tile, kEpiSiluBF16, I))) return rc;
  if (max_rows == 0) return EIMOE_OK;
  REQUIRE_PTR(a);
  REQUIRE_PTR(a_scale);
  REQUIRE_PTR(w_gate_up);
  REQUIRE_PTR(w_scale);
  REQUIRE_PTR(seg_offsets);
  REQUIRE_PTR(h);
  return run_gate_up(a, a_rows, a_nrows, lda, w_gate_up, EIMOE_FP8, w_scale, H, I, seg_offsets, n_seg, e_mod,
                     max_rows, h, tile, S(stream), a_scale);
}

int eimoe_gemm_down_w8a8(const void* hq, const float* h_scale, int I, const void* w_down, const float* w_scale, int H,
                         const int32_t* seg_offsets, int n_seg, int e_mod, int max_rows, void* y, int y_dtype,
                         int k_split, int tile, void* stream) {
  int rc = check_gemm_common(max_rows, n_seg, e_mod);
  if (rc) return rc;
  if (y_dtype != EIMOE_BF16 && y_dtype != EIMOE_F32) return fail(EIMOE_ERR_DTYPE, "y_dtype=%d", y_dtype);
  if (H < 64 || H % 64) return fail(EIMOE_ERR_ALIGN, "H=%d must be a positive multiple of 64", H);
  if (k_split < 1 || k_split > 64) return fail(EIMOE_ERR_SHAPE, "k_split=%d outside [1,64]", k_split);
  if (I < 128 || I % (128 * k_split))
    return fail(EIMOE_ERR_ALIGN, "I=%d must be a positive multiple of 128*k_split=%d", I, 128 * k_split);
  if ((rc = check_tile(tile, kEpiStoreF32, H))) return rc;
  if (static_cast<long long>(max_rows) * I > 0x7fffffffll) return fail(EIMOE_ERR_SHAPE, "hq exceeds 2 GiB");
  if (max_rows == 0) return EIMOE_OK;
  REQUIRE_PTR(hq);
  REQUIRE_PTR(h_scale);
  REQUIRE_PTR(w_down);
  REQUIRE_PTR(w_scale);
  REQUIRE_PTR(seg_offsets);
  REQUIRE_PTR(y);
  return run_down(hq, I, w_down, EIMOE_FP8, w_scale, H, seg_offsets, n_seg, e_mod, max_rows, y, y_dtype, k_split,
                  tile, S(stream), h_scale);
}

namespace {

// The grouped GEMM of the op point, expert weights either packed (b, b_expert_stride elements
// apart) or one [N, K] matrix per expert through a device table of b_ptrs.
int grouped_gemm_impl(const void* a, const int32_t* a_rows, int a_nrows, int lda, const void* b,
                      const void* const* b_ptrs, int b_dtype, const float* b_scale, long long b_expert_stride, int N,
                      int K, const int32_t* seg_offsets, int n_seg, int e_mod, int max_rows, void* c, int c_dtype,
                      int tile, void* stream) {
  int rc = check_gemm_common(max_rows, n_seg, e_mod);
  if (rc) return rc;
  if (b_dtype != EIMOE_BF16 && b_dtype != EIMOE_FP8 && b_dtype != EIMOE_F32)
    return fail(EIMOE_ERR_DTYPE, "b_dtype=%d", b_dtype);
  if (c_dtype != EIMOE_BF16 && c_dtype != EIMOE_F32) return fail(EIMOE_ERR_DTYPE, "c_dtype=%d", c_dtype);
  if (b_dtype == EIMOE_F32 && c_dtype != EIMOE_F32) return fail(EIMOE_ERR_DTYPE, "fp32 b writes fp32 c");
  if (K < 64 || K % 64) return fail(EIMOE_ERR_ALIGN, "K=%d must be a positive multiple of 64", K);
  if (N < 64 || N % 64) return fail(EIMOE_ERR_ALIGN, "N=%d must be a positive multiple of 64", N);
  if (lda < K || lda % 8) return fail(EIMOE_ERR_SHAPE, "lda=%d must be >= K=%d and a multiple of 8", lda, K);
  if (b_expert_stride < static_cast<long long>(N) * K)
    return fail(EIMOE_ERR_SHAPE, "b_expert_stride=%lld < N*K", b_expert_stride);
  if (b_expert_stride * elem_size(b_dtype) > 0x7fffffffll)
    return fail(EIMOE_ERR_SHAPE, "one expert's weights exceed 2 GiB");
  if (a_rows && a_nrows < 1) return fail(EIMOE_ERR_SHAPE, "a_nrows=%d < 1 with a row map", a_nrows);
  if (!a_rows) a_nrows = max_rows;
  if (static_cast<long long>(a_nrows) * lda * (b_dtype == EIMOE_F32 ? 4 : 2) > 0x7fffffffll)
    return fail(EIMOE_ERR_SHAPE, "A buffer (%d rows x %d) exceeds 2 GiB", a_nrows, lda);
  if ((rc = check_tile(tile, kEpiStoreF32, N))) return rc;
  if (max_rows == 0) return EIMOE_OK;
  REQUIRE_PTR(a);
  if (!b && !b_ptrs) return fail(EIMOE_ERR_NULL, "b is NULL");
  REQUIRE_PTR(seg_offsets);
  REQUIRE_PTR(c);
  if (b_dtype == EIMOE_FP8) REQUIRE_PTR(b_scale);
  GemmArgs p{};
  p.a = a;
  p.a_rows = a_rows;
  p.lda = lda;
  p.b = b;
  p.b_ptrs = b_ptrs;
  p.b_estride = b_expert_stride;
  p.ldb = K;
  p.b_scale = b_scale;
  p.nb_rows = N;
  p.N = N;
  p.K = K;
  p.seg_off = seg_offsets;
  p.S = n_seg;
  p.e_mod = e_mod;
  p.c = c;
  p.ldc = N;
  p.k_split = 1;
  p.max_rows = max_rows;
  p.a_rows_cap = a_nrows;
  const int epi = c_dtype == EIMOE_F32 ? kEpiStoreF32 : kEpiStoreBF16;
  if (b_dtype == EIMOE_F32) return hip_check(launch_grouped_gemm_f32(p, epi, max_rows, tile, S(stream)), "grouped_gemm");
  return hip_check(launch_grouped_gemm(p, epi, b_dtype == EIMOE_FP8, false, max_rows, tile, S(stream)),
                   "grouped_gemm");
}

}  // namespace

int eimoe_grouped_gemm(const void* a, const int32_t* a_rows, int a_nrows, int lda, const void* b, int b_dtype,
                       const float* b_scale, long long b_expert_stride, int N, int K, const int32_t* seg_offsets,
                       int n_seg, int e_mod, int max_rows, void* c, int c_dtype, int tile, void* stream) {
  return grouped_gemm_impl(a, a_rows, a_nrows, lda, b, nullptr, b_dtype, b_scale, b_expert_stride, N, K, seg_offsets,
                           n_seg, e_mod, max_rows, c, c_dtype, tile, stream);
}

int eimoe_grouped_gemm_ptrs(const void* a, const int32_t* a_rows, int a_nrows, int lda, const void* const* b_ptrs,
                            int n_b, int N, int K, const int32_t* seg_offsets, int n_seg, int e_mod, int max_rows,
                            void* c, int c_dtype, int tile, void* stream) {
  if (n_b < 1) return fail(EIMOE_ERR_SHAPE, "n_b=%d < 1", n_b);
  if (e_mod > n_b) return fail(EIMOE_ERR_SHAPE, "e_mod=%d > n_b=%d weight matrices", e_mod, n_b);
  if (max_rows > 0) REQUIRE_PTR(b_ptrs);
  return grouped_gemm_impl(a, a_rows, a_nrows, lda, nullptr, b_ptrs, EIMOE_BF16, nullptr,
                           static_cast<long long>(N) * K, N, K, seg_offsets, n_seg, e_mod, max_rows, c, c_dtype, tile,
                           stream);
}

int eimoe_combine(const void* y, int y_dtype, int n_split, long long split_stride, const int32_t* pos,
                  const float* topk_weights, int T, int k, int H, const void* shared_y, int shared_dtype, void* out,
                  int out_dtype, void* stream) {
  if (T < 0) return fail(EIMOE_ERR_SHAPE, "T=%d < 0", T);
  if (k < 1 || k > EIMOE_MAX_TOPK) return fail(EIMOE_ERR_SHAPE, "k=%d outside [1,%d]", k, EIMOE_MAX_TOPK);
  if (H < 8 || H % 8) return fail(EIMOE_ERR_ALIGN, "H=%d must be a positive multiple of 8", H);
  if (n_split < 1) return fail(EIMOE_ERR_SHAPE, "n_split=%d < 1", n_split);
  if (y_dtype != EIMOE_F32 && y_dtype != EIMOE_BF16) return fail(EIMOE_ERR_DTYPE, "y_dtype=%d", y_dtype);
  if (out_dtype != EIMOE_F32 && out_dtype != EIMOE_BF16) return fail(EIMOE_ERR_DTYPE, "out_dtype=%d", out_dtype);
  if (shared_y && shared_dtype != EIMOE_F32 && shared_dtype != EIMOE_BF16)
    return fail(EIMOE_ERR_DTYPE, "shared_dtype=%d", shared_dtype);
  if (T == 0) return EIMOE_OK;
  REQUIRE_PTR(y);
  REQUIRE_PTR(pos);
  REQUIRE_PTR(topk_weights);
  REQUIRE_PTR(out);
  return hip_check(launch_combine(y, y_dtype, n_split, split_stride, pos, topk_weights, T, k, H, shared_y,
                                  shared_dtype, 1, out, out_dtype, S(stream)),
                   "combine");
}

int eimoe_quantize_rows_fp8(const void* x, int dtype, long long rows, int cols, uint8_t* q, float* scale,
                            void* stream) {
  if (dtype != EIMOE_F32 && dtype != EIMOE_BF16) return fail(EIMOE_ERR_DTYPE, "dtype=%d", dtype);
  if (rows < 0 || cols < 1) return fail(EIMOE_ERR_SHAPE, "rows=%lld cols=%d", rows, cols);
  if (rows == 0) return EIMOE_OK;
  REQUIRE_PTR(x);
  REQUIRE_PTR(q);
  REQUIRE_PTR(scale);
  return hip_check(launch_quantize_rows_fp8(x, dtype, rows, cols, q, scale, S(stream)), "quantize_rows_fp8");
}

size_t eimoe_moe_prologue_workspace_bytes(int T, int H, int E) { return prologue_workspace_bytes(T, H, E); }

int eimoe_moe_prologue(const void* hidden, const void* residual, const void* norm_w, float eps, const void* gate_w,
                       int T, int H, int E, int flags, void* residual_out, void* normed, float* logits,
                       void* workspace, size_t workspace_bytes, void* stream) {
  if (T < 0) return fail(EIMOE_ERR_SHAPE, "T=%d < 0", T);
  if (H < 64 || H > 8192 || H % 64) return fail(EIMOE_ERR_ALIGN, "H=%d must be a multiple of 64 in [64, 8192]", H);
  if (E < 1 || E > EIMOE_MAX_EXPERTS) return fail(EIMOE_ERR_SHAPE, "E=%d outside [1,%d]", E, EIMOE_MAX_EXPERTS);
  const bool fused = prologue_fused_router(H, E);
  if (!fused && E % 64)
    return fail(EIMOE_ERR_SHAPE, "E=%d: up to %d experts with %lld bytes of gate weights, or a multiple of 64", E,
                kPrologueFusedMaxE, kPrologueFusedMaxGate);
  if (!(eps >= 0.f)) return fail(EIMOE_ERR_SHAPE, "eps must be >= 0");
  if (!fused && static_cast<long long>(T) * H * 2 > 0x7fffffffll)   // the router GEMM's 32-bit buffer offsets
    return fail(EIMOE_ERR_SHAPE, "normed (%d rows x %d) exceeds 2 GiB", T, H);
  if (T == 0) return EIMOE_OK;
  REQUIRE_PTR(hidden);
  REQUIRE_PTR(residual);
  REQUIRE_PTR(norm_w);
  REQUIRE_PTR(gate_w);
  REQUIRE_PTR(residual_out);
  REQUIRE_PTR(normed);
  REQUIRE_PTR(logits);
  if (normed == residual_out || normed == residual || normed == hidden)
    return fail(EIMOE_ERR_SHAPE, "normed must not alias the residual or hidden rows");
  if (!fused) {
    REQUIRE_PTR(workspace);
    const size_t need = prologue_workspace_bytes(T, H, E);
    if (workspace_bytes < need) return fail(EIMOE_ERR_WORKSPACE, "workspace %zu bytes < %zu", workspace_bytes, need);
  }
  return hip_check(launch_moe_prologue(hidden, residual, norm_w, eps, gate_w, T, H, E, (flags & EIMOE_LOGITS_BF16) ? 1 : 0,
                                       residual_out, normed, logits, workspace, S(stream)),
                   "moe_prologue");
}

size_t eimoe_fused_moe_workspace_bytes(int T, int H, int I, int E, int k, int n_local, int shared_inter,
                                       int out_dtype, int flags) {
  (void)E;
  if (T < 0 || H < 1 || I < 1 || k < 1 || n_local < 1 || shared_inter < 0) return 0;
  return fused_layout(T, H, I, E, k, n_local, shared_inter, out_dtype, flags).total;
}

int eimoe_fused_moe_down_split(int T, int H, int I, int E, int k, int n_local, int shared_inter, int out_dtype,
                               int flags) {
  if (T < 0 || H < 1 || I < 1 || k < 1 || n_local < 1 || shared_inter < 0) return 0;
  return fused_layout(T, H, I, E, k, n_local, shared_inter, out_dtype, flags).k_split;
}

}  // extern "C"

namespace {

// The fused layer over a workspace.  no_alloc: the workspace is the library's static scratch, so
// nothing may be created here (the shared experts then run on the caller's stream rather than on
// the second stream, which would be created on first use).
int fused_moe_impl(const void* x, const float* logits, int T, int H, int I, int E, int k, const void* w_gate_up,
                   const void* w_down, int w_dtype, const float* w_gate_up_scale, const float* w_down_scale, int e_lo,
                   int n_local, const void* shared_gate_up, const void* shared_down, int shared_inter, int flags,
                   void* out, int out_dtype, void* workspace, size_t workspace_bytes, int32_t* topk_ids_out,
                   float* topk_w_out, void* stream, bool no_alloc) {
  if (T < 0) return fail(EIMOE_ERR_SHAPE, "T=%d < 0", T);
  if (E < 1 || E > EIMOE_MAX_EXPERTS) return fail(EIMOE_ERR_SHAPE, "E=%d outside [1,%d]", E, EIMOE_MAX_EXPERTS);
  if (k < 1 || k > E || k > EIMOE_MAX_TOPK)
    return fail(EIMOE_ERR_SHAPE, "k=%d outside [1,min(E=%d,%d)]", k, E, EIMOE_MAX_TOPK);
  if (n_local < 1 || e_lo < 0 || e_lo + n_local > E)
    return fail(EIMOE_ERR_SHAPE, "expert window [%d,%d) not inside [0,%d)", e_lo, e_lo + n_local, E);
  if (H < 64 || H % 64) return fail(EIMOE_ERR_ALIGN, "H=%d must be a positive multiple of 64", H);
  if (I < 64 || I % 64) return fail(EIMOE_ERR_ALIGN, "I=%d must be a positive multiple of 64", I);
  if (shared_inter < 0 || (shared_inter > 0 && shared_inter % 64))
    return fail(EIMOE_ERR_ALIGN, "shared_inter=%d must be a multiple of 64", shared_inter);
  if (w_dtype != EIMOE_BF16 && w_dtype != EIMOE_FP8 && w_dtype != EIMOE_F32)
    return fail(EIMOE_ERR_DTYPE, "w_dtype=%d", w_dtype);
  if (out_dtype != EIMOE_BF16 && out_dtype != EIMOE_F32) return fail(EIMOE_ERR_DTYPE, "out_dtype=%d", out_dtype);
  if ((w_dtype == EIMOE_F32) != ((flags & EIMOE_FP32) != 0))
    return fail(EIMOE_ERR_DTYPE, "fp32 weights go with EIMOE_FP32 (fp32 x, h and y), and only they");
  if ((flags & EIMOE_FP32) && (flags & (EIMOE_W8A8 | EIMOE_H_SPLIT)))
    return fail(EIMOE_ERR_DTYPE, "EIMOE_FP32 keeps h in fp32: not with EIMOE_W8A8 or EIMOE_H_SPLIT");
  if (static_cast<long long>(T) * k > 0x7fffffffll) return fail(EIMOE_ERR_SHAPE, "T*k overflows int32");
  if ((flags & EIMOE_W8A8) && w_dtype != EIMOE_FP8) return fail(EIMOE_ERR_DTYPE, "EIMOE_W8A8 needs fp8 weights");
  if ((flags & EIMOE_W8A8) && (flags & EIMOE_H_SPLIT))
    return fail(EIMOE_ERR_DTYPE, "EIMOE_H_SPLIT keeps h in bf16 terms; W8A8 quantises it to fp8");
  if ((flags & EIMOE_W8A8) && (H % 128 || I % 128))
    return fail(EIMOE_ERR_ALIGN, "W8A8 needs H=%d and I=%d multiples of 128", H, I);
  {
    // The GEMMs address x, h and one expert's weights through 32-bit buffer offsets.
    const long long wb = elem_size(w_dtype);
    const long long ab = w_dtype == EIMOE_F32 ? 4 : 2;   // x, h and shared weights
    if (static_cast<long long>(T) * H * ab > 0x7fffffffll)
      return fail(EIMOE_ERR_SHAPE, "x (%d rows x %d) exceeds 2 GiB", T, H);
    if (static_cast<long long>(T) * k * I * ab > 0x7fffffffll)
      return fail(EIMOE_ERR_SHAPE, "h (%d x %d rows x %d) exceeds 2 GiB", T, k, I);
    if (2ll * I * H * wb > 0x7fffffffll) return fail(EIMOE_ERR_SHAPE, "one expert's gate/up weights exceed 2 GiB");
    if (static_cast<long long>(T) * shared_inter * ab > 0x7fffffffll || 2ll * shared_inter * H * ab > 0x7fffffffll)
      return fail(EIMOE_ERR_SHAPE, "shared experts (%d rows x %d) exceed 2 GiB", T, shared_inter);
  }
  if (T == 0) return EIMOE_OK;
  const bool routing_in = (flags & EIMOE_ROUTING_IN) != 0;
  REQUIRE_PTR(x);
  if (routing_in) {
    REQUIRE_PTR(topk_ids_out);
    REQUIRE_PTR(topk_w_out);
  } else {
    REQUIRE_PTR(logits);
  }
  REQUIRE_PTR(w_gate_up);
  REQUIRE_PTR(w_down);
  REQUIRE_PTR(out);
  REQUIRE_PTR(workspace);
  if (w_dtype == EIMOE_FP8) {
    REQUIRE_PTR(w_gate_up_scale);
    REQUIRE_PTR(w_down_scale);
  }
  if (shared_inter > 0) {
    REQUIRE_PTR(shared_gate_up);
    REQUIRE_PTR(shared_down);
  }
  const FusedLayout L = fused_layout(T, H, I, E, k, n_local, shared_inter, out_dtype, flags);
  if (workspace_bytes < L.total) {
    if (no_alloc)
      return fail(EIMOE_ERR_WORKSPACE, "this layer needs %zu bytes of scratch; eimoe_fused_moe_static holds %zu",
                  L.total, workspace_bytes);
    return fail(EIMOE_ERR_WORKSPACE, "workspace %zu bytes < required %zu", workspace_bytes, L.total);
  }
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  auto at = [&](size_t off) { return static_cast<void*>(ws + off); };
  int32_t* ids = topk_ids_out ? topk_ids_out : static_cast<int32_t*>(at(L.ids));
  float* w = topk_w_out ? topk_w_out : static_cast<float*>(at(L.w));
  int32_t* counts = static_cast<int32_t*>(at(L.counts));
  int32_t* offsets = static_cast<int32_t*>(at(L.offsets));
  int32_t* sorted_flat = static_cast<int32_t*>(at(L.sorted_flat));
  int32_t* sorted_tok = static_cast<int32_t*>(at(L.sorted_tok));
  int32_t* pos = static_cast<int32_t*>(at(L.pos));
  int32_t* hist = static_cast<int32_t*>(at(L.hist));   // the many-workgroup align's chunk counts
  const hipStream_t s = S(stream);
  const int A = T * k;
  int rc;
  // A decode step of a few routed pairs on small experts (T*k <= 16 and <= E/2, at most 4 MiB of
  // down weights per expert): the down projection and the combine as one kernel per (token,
  // column block).  Measured against the streaming down projection + combine (one box): the
  // Qwen3-30B-A3B 32-expert share (3 MiB experts) at 1 and 2 tokens 26.5 -> 22.1 and 22.0 ->
  // 17.6 us; slower at 8 tokens (47 -> 50 us) and on larger experts (DeepSeek-V2-Lite, 5.8 MiB,
  // 1 token: 74 -> 83 us; Mixtral-8x7B): a plain-FMA GEMV streams them below the MFMA streaming
  // kernel's rate.
  const bool down_combine = !(flags & (EIMOE_W8A8 | EIMOE_FP32)) && w_dtype == EIMOE_BF16 &&
                            down_combine_supported(H, I) && A <= 16 && 2ll * A <= E &&
                            static_cast<long long>(H) * I * 2 <= 4ll * 1024 * 1024;
  // Routing first: the shared experts forked below would otherwise fill the GPU ahead of the small
  // routing kernels on the critical path.
  if (routing_in) {
    if ((rc = hip_check(launch_align(ids, T, k, e_lo, n_local, counts, offsets, sorted_flat, sorted_tok, pos, hist,
                                     s),
                        "align")))
      return rc;
  } else if ((rc = hip_check(launch_route_align(logits, T, E, k, (flags & EIMOE_RENORMALIZE) ? 1 : 0, e_lo, n_local,
                                                ids, w, counts, offsets, sorted_flat, sorted_tok, pos, hist, s),
                             "route_align"))) {
    return rc;
  }
  // Shared experts (every token, weight 1) depend only on x: fork them onto the second
  // stream once the routing is enqueued, so they run beside the routed GEMMs; joined before
  // the combine.
  const void* sh_y = nullptr;
  AuxStream* aux = nullptr;
  if (shared_inter > 0) {
    if (!no_alloc) {
      hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
      if ((rc = hip_check(hipStreamIsCapturing(s, &cap), "capture status"))) return rc;
      if ((rc = hip_check(aux_stream(&aux, cap == hipStreamCaptureStatusNone), "aux stream"))) return rc;
    }
    const hipStream_t s2 = aux ? aux->stream : s;   // no second stream yet under capture: serial
    if (aux) {
      if ((rc = hip_check(hipEventRecord(aux->fork, s), "fork"))) return rc;
      if ((rc = hip_check(hipStreamWaitEvent(s2, aux->fork, 0), "fork wait"))) return rc;
    }
    auto shared = [&]() -> int {
      int rc;
      int32_t* sh_off = static_cast<int32_t*>(at(L.sh_off));
      hipLaunchKernelGGL(dense_segment_kernel, dim3(1), dim3(64), 0, s2, sh_off, T);
      if ((rc = hip_check(hipGetLastError(), "shared offsets"))) return rc;
      void* sh_lo = L.h_terms == 2 ? at(L.sh_h_lo) : nullptr;
      const int sh_dtype = w_dtype == EIMOE_F32 ? EIMOE_F32 : EIMOE_BF16;   // shared weights: bf16 or fp32
      if ((rc = run_gate_up(x, nullptr, T, H, shared_gate_up, sh_dtype, nullptr, H, shared_inter, sh_off, 1, 1, T,
                            at(L.sh_h), EIMOE_TILE_AUTO, s2, nullptr, 0, sh_lo)))
        return rc;
      if ((rc = run_down(at(L.sh_h), shared_inter, shared_down, sh_dtype, nullptr, H, sh_off, 1, 1, T, at(L.sh_y),
                         L.y_dtype, 1, EIMOE_TILE_AUTO, s2)))
        return rc;
      if (!sh_lo) return EIMOE_OK;
      return run_down(sh_lo, shared_inter, shared_down, EIMOE_BF16, nullptr, H, sh_off, 1, 1, T,
                      at(L.sh_y + static_cast<size_t>(T) * H * elem_size(L.y_dtype)), L.y_dtype, 1, EIMOE_TILE_AUTO,
                      s2);
    };
    rc = shared();
    if (aux) {
      const int rj = hip_check(hipEventRecord(aux->join, s2), "join");
      if (rc || rj) {   // still make the caller's stream wait for whatever was launched
        hipStreamWaitEvent(s, aux->join, 0);
        return rc ? rc : rj;
      }
    }
    if (rc) return rc;
    sh_y = at(L.sh_y);
  }
  // Routed part; whatever it returns, the caller's stream then waits for the shared work
  // (an early error return must not leave the second stream using the workspace unjoined).
  auto routed = [&]() -> int {
    int rc;
    if (flags & EIMOE_W8A8) {
      // activations quantised per token (x) and per row (h); both GEMMs on the fp8 MFMA
      uint8_t* xq = static_cast<uint8_t*>(at(L.xq));
      float* sx = static_cast<float*>(at(L.sx));
      uint8_t* hq = static_cast<uint8_t*>(at(L.hq));
      float* sh = static_cast<float*>(at(L.sh));
      if ((rc = hip_check(launch_quantize_rows_fp8(x, kBF16, T, H, xq, sx, s), "quantize x"))) return rc;
      if ((rc = run_gate_up(xq, sorted_tok, T, H, w_gate_up, w_dtype, w_gate_up_scale, H, I, offsets, n_local, n_local,
                            A, at(L.h), EIMOE_TILE_AUTO, s, sx, L.rows_hint)))
        return rc;
      if ((rc = hip_check(launch_quantize_rows_fp8(at(L.h), kBF16, A, I, hq, sh, s), "quantize h"))) return rc;
      if ((rc = run_down(hq, I, w_down, w_dtype, w_down_scale, H, offsets, n_local, n_local, A, at(L.y), L.y_dtype,
                         L.k_split, EIMOE_TILE_AUTO, s, sh, L.rows_hint)))
        return rc;
    } else {
      void* h_lo = L.h_terms == 2 ? at(L.h_lo) : nullptr;
      if ((rc = run_gate_up(x, sorted_tok, T, H, w_gate_up, w_dtype, w_gate_up_scale, H, I, offsets, n_local, n_local,
                            A, at(L.h), EIMOE_TILE_AUTO, s, nullptr, L.rows_hint, h_lo)))
        return rc;
      if (down_combine) return EIMOE_OK;   // projected inside the combine below
      if ((rc = run_down(at(L.h), I, w_down, w_dtype, w_down_scale, H, offsets, n_local, n_local, A, at(L.y),
                         L.y_dtype, L.k_split, EIMOE_TILE_AUTO, s, nullptr, L.rows_hint)))
        return rc;
      // the lo term into the planes after the hi term's (the combine sums them all)
      if (h_lo && (rc = run_down(h_lo, I, w_down, w_dtype, w_down_scale, H, offsets, n_local, n_local, A,
                                 at(L.y + static_cast<size_t>(L.k_split) * A * H * elem_size(L.y_dtype)), L.y_dtype,
                                 L.k_split, EIMOE_TILE_AUTO, s, nullptr, L.rows_hint)))
        return rc;
    }
    return EIMOE_OK;
  };
  rc = routed();
  if (aux) {
    const int rj = hip_check(hipStreamWaitEvent(s, aux->join, 0), "join wait");
    if (!rc) rc = rj;
  }
  if (rc) return rc;
  if (down_combine)
    return hip_check(launch_down_combine(at(L.h), L.h_terms == 2 ? at(L.h_lo) : nullptr, w_down, I, H, ids, w, pos, T,
                                         k, e_lo, sh_y, L.y_dtype, L.h_terms, out, out_dtype, s),
                     "down + combine");
  return hip_check(launch_combine(at(L.y), L.y_dtype, L.h_terms * L.k_split, static_cast<long long>(A) * H, pos, w, T,
                                  k, H, sh_y, L.y_dtype, L.h_terms, out, out_dtype, s),
                   "combine");
}

// Static scratch of eimoe_fused_moe_static: every GPU the library runs on holds one copy for the
// life of the process.  Host code never uses the array's name as an address (on the host it is a
// stand-in, not device memory); it uses the per-device address from hipGetSymbolAddress.
constexpr size_t kStaticScratchBytes = 64ull << 20;
static __device__ __align__(256) uint8_t scratch[kStaticScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Looked up once per device, on the entry point's first call with that device current.
int static_scratch(void** out) {
  int dev = 0;
  int rc = hip_check(hipGetDevice(&dev), "current device");
  if (rc) return rc;
  if (dev < 0 || dev >= kMaxDevices) return fail(EIMOE_ERR_HIP, "device %d outside [0,%d)", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    if ((rc = hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "static scratch address"))) return rc;
    if (!p) return fail(EIMOE_ERR_HIP, "static scratch address is NULL");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return EIMOE_OK;
}

}  // namespace

extern "C" {

int eimoe_fused_moe(const void* x, const float* logits, int T, int H, int I, int E, int k, const void* w_gate_up,
                    const void* w_down, int w_dtype, const float* w_gate_up_scale, const float* w_down_scale, int e_lo,
                    int n_local, const void* shared_gate_up, const void* shared_down, int shared_inter, int flags,
                    void* out, int out_dtype, void* workspace, size_t workspace_bytes, int32_t* topk_ids_out,
                    float* topk_w_out, void* stream) {
  return fused_moe_impl(x, logits, T, H, I, E, k, w_gate_up, w_down, w_dtype, w_gate_up_scale, w_down_scale, e_lo,
                        n_local, shared_gate_up, shared_down, shared_inter, flags, out, out_dtype, workspace,
                        workspace_bytes, topk_ids_out, topk_w_out, stream, false);
}

size_t eimoe_fused_moe_static_bytes(void) { return kStaticScratchBytes; }

int eimoe_fused_moe_static(const void* x, const float* logits, int T, int H, int I, int E, int k,
                           const void* w_gate_up, const void* w_down, int w_dtype, const float* w_gate_up_scale,
                           const float* w_down_scale, int e_lo, int n_local, const void* shared_gate_up,
                           const void* shared_down, int shared_inter, int flags, void* out, int out_dtype,
                           int32_t* topk_ids_out, float* topk_w_out, void* stream) {
  void* ws = nullptr;
  const int rc = static_scratch(&ws);
  if (rc) return rc;
  return fused_moe_impl(x, logits, T, H, I, E, k, w_gate_up, w_down, w_dtype, w_gate_up_scale, w_down_scale, e_lo,
                        n_local, shared_gate_up, shared_down, shared_inter, flags, out, out_dtype, ws,
                        kStaticScratchBytes, topk_ids_out, topk_w_out, stream, true);
}

}  // extern "C"
