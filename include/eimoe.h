/* eimoe — MI355X (gfx950) fused-MoE expert path, C ABI.
 *
 * Drop-in boundary for EasyInfra's MoE expert plugin point
 * (easyinfra/generation/modules/moe/config.py:4-15 get_moe_impl, the FusedMoE
 * class of fused_moe.py:15-156) and its native grouped-GEMM op point
 * (easyinfra/__init__.py:7-20, single_group_gemm_moe.py:53-91).
 *
 * Conventions
 *  - Every pointer argument except the stream is a DEVICE pointer unless noted.
 *  - `stream` is a hipStream_t passed as void* (NULL = the default stream).  All work is
 *    enqueued on it; no entry point synchronises the device or allocates memory.  The caller
 *    owns every buffer, including the workspace.
 *  - Return value: EIMOE_OK (0) or a negative EIMOE_ERR_* code; eimoe_last_error() then
 *    returns a message (thread-local).  Arguments are validated on the host before any launch.
 *  - dtype codes: EIMOE_F32, EIMOE_BF16, EIMOE_FP8 (OCP e4m3fn, one byte).
 *  - Row/column-major: all matrices are row-major with the given leading dimension; expert
 *    weights use nn.Linear layout [out_features, in_features] (K contiguous).
 *  - Integer outputs (ids, counts, offsets, permutations) are deterministic and bit-exact.
 */
#ifndef EIMOE_H_
#define EIMOE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define EIMOE_ABI_VERSION 1

enum {
  EIMOE_OK = 0,
  EIMOE_ERR_NULL = -1,      /* a required pointer is NULL */
  EIMOE_ERR_SHAPE = -2,     /* a size is out of the supported range */
  EIMOE_ERR_ALIGN = -3,     /* a dimension is not a multiple of the required granule */
  EIMOE_ERR_DTYPE = -4,     /* unsupported dtype code / combination */
  EIMOE_ERR_WORKSPACE = -5, /* workspace smaller than eimoe_fused_moe_workspace_bytes() */
  EIMOE_ERR_HIP = -6        /* the HIP runtime reported an error at launch */
};

enum { EIMOE_F32 = 0, EIMOE_BF16 = 1, EIMOE_FP8 = 2 };

/* flags for eimoe_fused_moe */
enum {
  EIMOE_RENORMALIZE = 1, /* renormalise the top-k weights (norm_topk_prob) */
  EIMOE_Y_F32 = 2,       /* accepted for compatibility, no effect: the per-assignment expert outputs
                            are always kept in fp32 and the combine rounds once to the output type */
  EIMOE_W8A8 = 4,        /* fp8 weights: also quantise activations per token and run the fp8 MFMA */
  EIMOE_ROUTING_IN = 8,  /* topk_ids / topk_w are inputs (routing done by the caller, e.g. with
                            eimoe_router_grouped_topk); logits are not read and may be NULL */
  EIMOE_H_SPLIT = 16,    /* precise mode: the SiLU*mul intermediate h is kept as two bf16 terms
                            (h = hi + lo, ~16 significant bits instead of 8) and the down projection
                            runs once per term (twice its time); y is kept in fp32.  Not with W8A8. */
  EIMOE_FP32 = 32        /* fp32 layer: x, the weights (w_dtype EIMOE_F32, shared weights too), h
                            and y in fp32 on the fp32 MFMA (the reference's fp32 F.linear path,
                            native_moe.py:56-103).  Required with, and only with, fp32 weights;
                            size the workspace with it.  Not with W8A8 or H_SPLIT. */
};

/* tile selector for the GEMM entry points (0 = automatic).  EIMOE_TILE_STREAM is the
 * weight-streaming kernel for a few rows per segment (bf16 weights with K % 64 == 0, or e4m3
 * weights with K % 128 == 0 and bf16 or, in the W8A8 entry points, e4m3 activations; the output
 * columns a multiple of 16 for gate/up, 32 otherwise); automatic selection uses it when the
 * average rows per segment are small.  The fp32 layer has no 256x256, 64x128 or streaming
 * kernel: those requests take the 128x128 tile there. */
enum { EIMOE_TILE_AUTO = 0, EIMOE_TILE_256x256 = 1, EIMOE_TILE_128x128 = 2, EIMOE_TILE_32x128 = 3,
       EIMOE_TILE_16x64 = 4, EIMOE_TILE_STREAM = 5, EIMOE_TILE_64x128 = 6 };

#define EIMOE_MAX_TOPK 32
#define EIMOE_MAX_EXPERTS 512
#define EIMOE_MAX_SEGMENTS 1024

int eimoe_abi_version(void);
const char* eimoe_last_error(void);

/* Releases the calling thread's second stream and its two events (one set per device, created by
 * the first eimoe_fused_moe call with shared experts on that thread and device), after waiting for
 * the work queued on them.  No counterpart in the reference (its shared experts run on the caller's
 * stream, moe_all2all.py:535-537); for callers that end worker threads or want the stream back
 * before the process ends.  A later eimoe_fused_moe call creates them again.  Restores the current
 * device. */
int eimoe_release_streams(void);

/* Router: softmax -> top-k -> optional renormalisation.
 * Replaces Qwen3MoeSparseMoeBlock._routing (models/qwen3_moe/modeling_qwen3_moe.py:255-266).
 * logits [T,E] fp32 -> topk_ids [T,k] int32 (descending logit, ties to the lower id),
 * topk_weights [T,k] fp32.  1 <= k <= min(E, EIMOE_MAX_TOPK), E <= EIMOE_MAX_EXPERTS. */
int eimoe_router_topk(const float* logits, int T, int E, int k, int renormalize, int32_t* topk_ids,
                      float* topk_weights, void* stream);

/* DeepSeek-V3 router, "noaux_tc" grouped top-k: DeepseekV3MoEGate.forward
 * (models/deepseek_v3/modeling_deepseek_v3.py:151-203) from its logits on.
 *   s = sigmoid(logits) (correctly rounded fp32); c = s + bias (bias [E] or NULL for zeros);
 *   group score = sum of the 2 largest c in each of n_group equal groups of experts;
 *   the topk_group best groups are kept and c is set to 0 elsewhere;
 *   topk_ids = top-k of c (descending c, ties to the lower id);
 *   topk_weights = s[ids], divided by their sum + 1e-20 when renormalize and k > 1, times scaling.
 * logits [T,E] fp32 -> topk_ids [T,k] int32, topk_weights [T,k] fp32 (the reference casts the
 * weights to the activation dtype; they stay fp32 here).  E <= EIMOE_MAX_EXPERTS, E % n_group == 0,
 * E / n_group >= 2, 1 <= topk_group <= n_group, 1 <= k <= min(E, EIMOE_MAX_TOPK). */
int eimoe_router_grouped_topk(const float* logits, int T, int E, int k, int n_group, int topk_group,
                              const float* bias, int renormalize, float scaling, int32_t* topk_ids,
                              float* topk_weights, void* stream);

/* EPLB logical -> physical expert ids: eplb_map_to_physical_and_record
 * (generation/blocks/moe/base.py:40-64), with the maps built at base.py:162-185.
 * physical_ids[i] = log2phy[topk_ids[i]][i % replica_count[topk_ids[i]]] over the flattened
 * [T,k] ids (i = t*k + slot), so repeated picks of one logical expert spread over its replicas.
 * log2phy [n_logical, max_replicas] int32, replica_count [n_logical] int32.  Ids outside
 * [0, n_logical) map to -1.  physical_ids may alias topk_ids. */
int eimoe_eplb_map(const int32_t* topk_ids, int T, int k, const int32_t* log2phy, int n_logical, int max_replicas,
                   const int32_t* replica_count, int32_t* physical_ids, void* stream);

/* Align: per-expert counts, offsets and the stable expert-major permutation.
 * Replaces _MoeBlock._all_expert_count_compute (generation/blocks/moe/base.py:343-364) and the
 * sort/index steps of MoeAll2AllBlock.all2all_chunk_routing_compute (blocks/moe/moe_all2all.py:346-348).
 * Only ids in [e_lo, e_lo+n_local) are kept (one GPU's EP share, blocks/moe/base.py:162-169, 187).
 * Outputs: counts[n_local], offsets[n_local+1] (offsets[n_local] = rows kept),
 * sorted_flat[T*k] (flat index t*k+slot per row), sorted_tok[T*k] (t per row),
 * pos[T*k] (row of each flat index, -1 if not local).  Rows beyond offsets[n_local] are untouched.
 * 1 <= n_local <= EIMOE_MAX_EXPERTS.  workspace (eimoe_align_workspace_bytes(T, k, n_local) bytes;
 * may be NULL) lets large batches (from 4096 routed pairs) spread the sort over many workgroups
 * in two launches; without it one workgroup sorts.  Same result either way. */
size_t eimoe_align_workspace_bytes(int T, int k, int n_local);
int eimoe_align(const int32_t* topk_ids, int T, int k, int e_lo, int n_local, int32_t* counts, int32_t* offsets,
                int32_t* sorted_flat, int32_t* sorted_tok, int32_t* pos, void* workspace, size_t workspace_bytes,
                void* stream);

/* Router then align in one call: the outputs of eimoe_router_topk followed by eimoe_align on
 * its ids, same arguments, same results bit for bit.  Small batches run both phases in one
 * workgroup (one launch; the ids stay on chip between them).  Replaces the same reference code
 * as the two calls: models/qwen3_moe/modeling_qwen3_moe.py:255-266, then
 * generation/blocks/moe/base.py:343-364 and blocks/moe/moe_all2all.py:346-348. */
int eimoe_route_align(const float* logits, int T, int E, int k, int renormalize, int e_lo, int n_local,
                      int32_t* topk_ids, float* topk_weights, int32_t* counts, int32_t* offsets,
                      int32_t* sorted_flat, int32_t* sorted_tok, int32_t* pos, void* stream);

/* Segment offsets from per-segment row counts (exclusive prefix sum, offsets[n_seg] = total).
 * Replaces the block schedule of TritonExperts.forward_ep (fused_moe.py:413-439) for callers that
 * pass pre-grouped rows (FusedMoE.forward_ep(hidden_states, expert_count), fused_moe.py:106-156). */
int eimoe_counts_to_offsets(const int32_t* counts, int n_seg, int32_t* offsets, void* stream);

/* Gather: xs[r,:] = x[rows[r],:] for r < min(*num_rows, max_rows).
 * Replaces send_hidden_states = h[send_indices] (blocks/moe/moe_all2all.py:351).
 * dtype EIMOE_F32 or EIMOE_BF16; H*elem_size must be a multiple of 16 bytes. */
int eimoe_gather(const void* x, int dtype, int H, const int32_t* rows, const int32_t* num_rows, int max_rows,
                 void* xs, void* stream);

/* Grouped gate/up GEMM with SiLU*mul fused:  h[r,:] = silu(g) * u, [g|u] = a[row(r)] . W_gu[e]^T
 * for r in segment s (rows [seg_offsets[s], seg_offsets[s+1])), e = s % e_mod.
 * Replaces fused_moe.py:445-459 (first fused_moe_kernel launch + silu(g)*u).
 * a: bf16 [a_nrows, lda], row r reads a[(a_rows ? a_rows[r] : r) * lda + :H] (a_rows gathers tokens
 * directly; every a_rows entry must be < a_nrows, reads beyond the buffer return 0).
 * w_gate_up: [E_w, 2I, H] bf16 or fp8 (rows [0,I) gate, [I,2I) up, fused_moe.py:91-101);
 * w_scale: fp8 only, [E_w, 2I] fp32 per-output-channel scales.  h: bf16 [max_rows, I].
 * w_dtype EIMOE_F32: a and w_gate_up fp32 on the fp32 MFMA, h fp32 [max_rows, I].
 * H % 64 == 0, I % 32 == 0.  max_rows bounds seg_offsets[n_seg]. */
int eimoe_gemm_gate_up_silu(const void* a, const int32_t* a_rows, int a_nrows, int lda, const void* w_gate_up, int w_dtype,
                            const float* w_scale, int H, int I, const int32_t* seg_offsets, int n_seg, int e_mod,
                            int max_rows, void* h, int tile, void* stream);

/* Grouped down GEMM: y[r,:] = h[r,:] . W_d[e]^T (fused_moe.py:463-476).
 * h: bf16 [max_rows, I]; w_down: [E_w, H, I] bf16 or fp8 (+ w_scale [E_w, H]); or h and w_down
 * fp32 with w_dtype EIMOE_F32 (the fp32 MFMA; y_dtype EIMOE_F32).
 * y: y_dtype (EIMOE_F32 / EIMOE_BF16) [k_split][max_rows, H]; with k_split > 1 each K-slice
 * writes its own partial plane (summed by eimoe_combine), I/k_split % 64 == 0. */
int eimoe_gemm_down(const void* h, int I, const void* w_down, int w_dtype, const float* w_scale, int H,
                    const int32_t* seg_offsets, int n_seg, int e_mod, int max_rows, void* y, int y_dtype,
                    int k_split, int tile, void* stream);

/* W8A8 twins of the two expert GEMMs: fp8-e4m3 activations with per-row scales and fp8-e4m3
 * weights with per-output-channel scales, on the gfx950 fp8 MFMA; result = acc * a_scale[row] *
 * w_scale[col] (the gate/up pair scaled before SiLU*mul).  No reference counterpart
 * (fused_moe.py:331-335 maps fp8 inputs to a bf16 compute type and takes no scales).
 * gate/up: a [a_nrows, lda] fp8, a_scale[a_nrows] (row r uses a_scale[a_rows ? a_rows[r] : r]);
 *          H % 128 == 0, I % 32 == 0; h bf16 [max_rows, I].
 * down:    hq [max_rows, I] fp8, h_scale[max_rows]; I/k_split % 128 == 0. */
int eimoe_gemm_gate_up_silu_w8a8(const void* a, const float* a_scale, const int32_t* a_rows, int a_nrows, int lda,
                                 const void* w_gate_up, const float* w_scale, int H, int I,
                                 const int32_t* seg_offsets, int n_seg, int e_mod, int max_rows, void* h, int tile,
                                 void* stream);
int eimoe_gemm_down_w8a8(const void* hq, const float* h_scale, int I, const void* w_down, const float* w_scale, int H,
                         const int32_t* seg_offsets, int n_seg, int e_mod, int max_rows, void* y, int y_dtype,
                         int k_split, int tile, void* stream);

/* Plain grouped GEMM, the X_grouped_gemm_single(A, B_list, block_sizes) contract
 * (single_group_gemm_moe.py:76-91): c[rows_s] = a[rows_s] . B[s % e_mod]^T with B packed as
 * [E_w, N, K] (b_expert_stride elements apart).  a bf16 [a_nrows, lda] (rows gathered through a_rows
 * when given); b bf16/fp8 (+b_scale [E_w,N]), or a and b fp32 with b_dtype EIMOE_F32 (c fp32);
 * c f32 or bf16 [max_rows, N].  K % 64 == 0, N % 64 == 0. */
int eimoe_grouped_gemm(const void* a, const int32_t* a_rows, int a_nrows, int lda, const void* b, int b_dtype,
                       const float* b_scale, long long b_expert_stride, int N, int K, const int32_t* seg_offsets,
                       int n_seg, int e_mod, int max_rows, void* c, int c_dtype, int tile, void* stream);

/* The same grouped GEMM over separate per-expert weight tensors, read where they lie: b_ptrs is a
 * DEVICE array of n_b pointers, b_ptrs[e] a bf16 [N, K] row-major matrix (nn.Linear layout).
 * The reference hands the op a Python list of per-expert Parameters, repeated ep_size times
 * (single_group_gemm_moe.py:73-76, 89); pass the n_b distinct ones with e_mod = n_b instead of
 * stacking them (a copy of every expert's weights per call). */
int eimoe_grouped_gemm_ptrs(const void* a, const int32_t* a_rows, int a_nrows, int lda, const void* const* b_ptrs,
                            int n_b, int N, int K, const int32_t* seg_offsets, int n_seg, int e_mod, int max_rows,
                            void* c, int c_dtype, int tile, void* stream);

/* Weighted top-k combine: out[t,:] = sum_j w[t,j] * sum_s y[s][pos[t*k+j],:]  (+ shared_y[t,:]).
 * Replaces _all2all_chunk_output_compute (blocks/moe/moe_all2all.py:291-307) and the shared-expert
 * residual add (moe_all2all.py:535-537).  Slots with pos < 0 contribute nothing; a token with no
 * local slot gets a zero row (or just shared_y).  fp32 accumulation, deterministic.
 * y: y_dtype [n_split][*, H] planes split_stride elements apart; shared_y optional [T,H]. */
int eimoe_combine(const void* y, int y_dtype, int n_split, long long split_stride, const int32_t* pos,
                  const float* topk_weights, int T, int k, int H, const void* shared_y, int shared_dtype, void* out,
                  int out_dtype, void* stream);

/* fp8 quantisation per row: scale[r] = max|x[r,:]|/448 (1 for a zero row), q = rne_e4m3fn(x/scale).
 * Used for per-output-channel weight scales and per-token activation scales.  No reference
 * counterpart (fused_moe.py:331-335 takes no scales). */
int eimoe_quantize_rows_fp8(const void* x, int dtype, long long rows, int cols, uint8_t* q, float* scale,
                            void* stream);

/* MoE block prologue, one pass over a chunk of hidden states:
 *   residual_out = residual + hidden                        (bf16; _add_to_residual,
 *                                                            generation/utils/compute_utils.py:14)
 *   normed = norm_w * bf16(r * rsqrt(mean(r^2) + eps))       (bf16, r = residual_out in fp32;
 *                                                            _rmsnorm, generation/modules/rmsnorm/base_rmsnorm.py:6-12)
 *   logits = normed . gate_w^T                               (fp32 accumulation; the router gate)
 * in the order of MoeAll2AllBlock.all2all_chunk_routing_compute (blocks/moe/moe_all2all.py:329-336).
 * EIMOE_LOGITS_BF16 rounds the logits to bf16 values (the Qwen3 / Mixtral gate is an F.linear
 * in bf16, generation/modules/linear/base_linear.py:28-36); without it they stay fp32 (DeepseekV3MoEGate,
 * models/deepseek_v3/modeling_deepseek_v3.py:155-157).
 *   hidden, residual, residual_out, normed [T,H] bf16; norm_w [H] bf16; gate_w [E,H] bf16;
 *   logits [T,E] fp32.  64 <= H <= 8192, H % 64 == 0; E <= 32 with E*H*2 <= 128 KiB (one pass),
 *   or E % 64 == 0 up to EIMOE_MAX_EXPERTS (router GEMM on the MFMA, needs the workspace:
 *   eimoe_moe_prologue_workspace_bytes(T, H, E) bytes, 0 for the one-pass routers).
 *   residual_out may alias residual; normed may not alias residual_out. */
enum { EIMOE_LOGITS_BF16 = 1 };
size_t eimoe_moe_prologue_workspace_bytes(int T, int H, int E);
int eimoe_moe_prologue(const void* hidden, const void* residual, const void* norm_w, float eps, const void* gate_w,
                       int T, int H, int E, int flags, void* residual_out, void* normed, float* logits,
                       void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes for eimoe_fused_moe with these sizes and flags. */
size_t eimoe_fused_moe_workspace_bytes(int T, int H, int I, int E, int k, int n_local, int shared_inter,
                                       int out_dtype, int flags);

/* The K split of the down projection that eimoe_fused_moe picks for these arguments: its
 * per-assignment outputs are that many fp32 planes [T*k, H], summed by the combine.  No counterpart
 * in the reference (its down projection is one unsplit launch, fused_moe.py:463-476); for callers
 * that time the layer's stages through the op-level entry points and want the same launches.
 * Returns 0 for arguments eimoe_fused_moe_workspace_bytes refuses. */
int eimoe_fused_moe_down_split(int T, int H, int I, int E, int k, int n_local, int shared_inter, int out_dtype,
                               int flags);

/* The whole layer: hidden_states, router logits and top_k in, combined output out.
 * Composes router -> align -> gate/up+SiLU (gathering x rows directly) -> down -> combine
 * (+ shared experts), i.e. MoeAll2AllBlock's stages at ep=1 (blocks/moe/moe_all2all.py:85-95)
 * with FusedMoE.forward_ep (fused_moe.py:106-156) as the expert step.
 *   x [T,H] bf16; logits [T,E] fp32; w_gate_up [n_local,2I,H], w_down [n_local,H,I] in w_dtype
 *   (bf16 or fp8 with per-channel scales [n_local,2I] / [n_local,H]); experts e_lo..e_lo+n_local-1
 *   of the router's E are resident (pass 0, E for a whole layer); shared experts optional
 *   (shared_gate_up [2*Is,H], shared_down [H,Is] bf16, weight 1.0); out [T,H] in out_dtype.
 *   With EIMOE_FP32: x, the weights (w_dtype EIMOE_F32) and the shared weights are fp32.
 * Optional outputs (may be NULL): topk_ids_out [T,k] int32, topk_w_out [T,k] fp32; with
 * EIMOE_ROUTING_IN both are required inputs instead and the router is skipped. */
int eimoe_fused_moe(const void* x, const float* logits, int T, int H, int I, int E, int k, const void* w_gate_up,
                    const void* w_down, int w_dtype, const float* w_gate_up_scale, const float* w_down_scale, int e_lo,
                    int n_local, const void* shared_gate_up, const void* shared_down, int shared_inter, int flags,
                    void* out, int out_dtype, void* workspace, size_t workspace_bytes, int32_t* topk_ids_out,
                    float* topk_w_out, void* stream);

/* eimoe_fused_moe without a workspace argument, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  No
 * counterpart in the reference.  Same arguments and results as eimoe_fused_moe; its scratch is a
 * static device array of eimoe_fused_moe_static_bytes() (64 MiB) that each GPU holds from the
 * first call until the process ends, so it fits decode-sized layers (a Mixtral-8x7B layer up to
 * 545 tokens with either output type; eimoe_fused_moe_workspace_bytes gives the need) and returns
 * EIMOE_ERR_WORKSPACE,
 * launching nothing, when a layer needs more.  It calls no hipMalloc/hipFree and creates no
 * stream or event (shared experts run on `stream` after the routed ones).  Every call on a GPU
 * uses that GPU's one scratch array: calls that overlap on one GPU (other streams, other host
 * threads) race and must be serialised by the caller. */
size_t eimoe_fused_moe_static_bytes(void);
int eimoe_fused_moe_static(const void* x, const float* logits, int T, int H, int I, int E, int k,
                           const void* w_gate_up, const void* w_down, int w_dtype, const float* w_gate_up_scale,
                           const float* w_down_scale, int e_lo, int n_local, const void* shared_gate_up,
                           const void* shared_down, int shared_inter, int flags, void* out, int out_dtype,
                           int32_t* topk_ids_out, float* topk_w_out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* EIMOE_H_ */
