/* C-ABI of libglm52_hip.so: the GLM-5.2 MoE FFN block on MI355X (gfx950).
 *
 * Every entry point takes raw device pointers, sizes and element strides plus the HIP
 * stream to launch on; none allocates, none synchronises the host, and all return 0 on
 * success, a negative GLM52_E* code for an invalid argument, or a positive hipError_t
 * from the launch.  bf16 tensors are passed as pointers to 16-bit words; base pointers
 * and row strides of bf16 tensors must be 16-byte aligned (strides multiples of 8).
 *
 * Each function replaces one launcher of the reference's Python package
 * (HansonZhang-cuhksz/fusion, glm52/kernels/*.py), whose Python signatures the package
 * fusion_amd.kernels keeps; the citation is given per function.
 */
#ifndef GLM52_HIP_H
#define GLM52_HIP_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GLM52_OK 0
#define GLM52_EINVAL (-1)
#define GLM52_EUNSUPPORTED (-2)

/* ResAdd + RMSNorm.  Replaces add_rmsnorm.fused_add_rmsnorm / add_only / norm_only
 * (glm52/kernels/add_rmsnorm.py:234-246; kernel :50-190).
 *   do_add:  h1 = bf16(x + res);  do_norm: out = bf16(bf16(h * rstd) * w), h = h1 or x.
 *   N % 8 == 0, N <= 8192.  rows_per_wave_mode: 1 wave/row, 0 workgroup/row, -1 by T. */
int glm52_add_rmsnorm(const void* x, const void* res, const void* w, void* h1, void* out,
                      int64_t stride_x, int64_t stride_r, int64_t stride_h, int64_t stride_o,
                      int T, int N, float eps, int do_add, int do_norm, int rows_per_wave_mode,
                      hipStream_t stream);

/* Router logits [T, E] fp32 = y [T, H] bf16 . wgt (bf16, or fp32 if wg_is_f32), the
 * products summed in fp64 and rounded once.  Replaces norm_router.router_gemm
 * (glm52/kernels/norm_router.py:347-349).  wgt is addressed wgt[k * stride_wk + e * stride_we]:
 *   stride_we == 1: the reference's [H, E] layout, read by the fp64 MFMA mapping; small T
 *     splits K and needs a workspace of glm52_router_workspace_bytes(T, H, E) bytes;
 *   stride_wk == 1: gate rows [E, H], one wave per expert row; no workspace.
 * E <= 256, E % 16 == 0, H % 64 == 0, H <= 8192; wgt 16-byte aligned. */
int glm52_router_logits(const void* y, int64_t stride_y, const void* wgt, int64_t stride_wk,
                        int64_t stride_we, int wg_is_f32, float* logits, int64_t stride_l,
                        void* workspace, int64_t workspace_bytes, int T, int H, int E,
                        hipStream_t stream);

/* Split-K scratch the router needs at T tokens (bytes).  No counterpart in the reference,
 * whose Triton router sizes its grid on the host. */
int64_t glm52_router_workspace_bytes(int T, int H, int E);

/* glm52_router_logits followed by glm52_router_topk in two launches, the split-K
 * reduction folded into the top-k pass.  Replaces the router_gemm + topk_only pair the
 * reference chain launches (glm52/bench/bench_layer.py:426-428).
 * On the gate's rows (stride_wk == 1, bf16) and T > 16 the logits run on bf16 MFMA with a
 * proven error bound, and only each token's candidates -- the experts the bound cannot
 * exclude from the top k -- get the exact logit: ids and weights equal the exact rule's
 * bit for bit; logits are exact for the candidates and within the bound elsewhere.  That
 * path needs glm52_router_select_workspace_bytes(T, H, E) bytes of workspace (16-byte
 * aligned), H of 4096, 6144 or 8192 and E % 4 == 0; with a smaller workspace (the size
 * glm52_router_workspace_bytes gives) or a y that is not 16-byte aligned the exact
 * mappings run instead, with every logit exact. */
int64_t glm52_router_select_workspace_bytes(int T, int H, int E);
int glm52_router(const void* y, int64_t stride_y, const void* wgt, int64_t stride_wk,
                 int64_t stride_we, int wg_is_f32, float* logits, int64_t stride_l,
                 void* workspace, int64_t workspace_bytes, const float* bias, float* topw,
                 int64_t stride_w, int32_t* topi, int64_t stride_i, int T, int H, int E,
                 int topk, float scale, int norm_prob, hipStream_t stream);

/* Sigmoid + noaux_tc top-k with optional correction bias (nullable), renormalisation and
 * scaling.  Replaces norm_router.topk_only (glm52/kernels/norm_router.py:352-354) with
 * the semantics of glm52/reference.py:46-79.  E <= 256, topk <= 8. */
int glm52_router_topk(const float* logits, int64_t stride_l, const float* bias, float* topw,
                      int64_t stride_w, int32_t* topi, int64_t stride_i, int T, int E, int topk,
                      float scale, int norm_prob, hipStream_t stream);

/* Dispatch layout.  Replaces reference.moe_align_block_size (glm52/reference.py:85-128)
 * without its host sync: capacity >= numel + E * (block_m - 1), capacity % block_m == 0;
 * the tail past *num_tokens_post_padded holds the sentinel numel / expert id -1. */
int glm52_moe_align(const int32_t* topk_ids, int numel, int block_m, int num_experts,
                    int capacity, int32_t* sorted_token_ids, int32_t* expert_ids,
                    int32_t* num_tokens_post_padded, hipStream_t stream);

/* The same layout for large inputs, by one workgroup per chunk of 2048 ids in two
 * launches (chunk histograms, then prefix and stable scatter), with a caller-owned
 * workspace of ceil(numel / 2048) * num_experts int32 histograms.  Same outputs, bit for
 * bit, as glm52_moe_align, which it calls when the workspace is null or too small (or
 * numel <= 2048).  glm52_moe_align_workspace_bytes(numel, num_experts) gives that size
 * where the chunked build is the faster one (numel >= 16384), else 0.  No counterpart interface in
 * the reference: a faster route to reference.moe_align_block_size
 * (glm52/reference.py:85-128) for prefill sizes. */
int64_t glm52_moe_align_workspace_bytes(int numel, int num_experts);
int glm52_moe_align_ws(const int32_t* topk_ids, int numel, int block_m, int num_experts,
                       int capacity, int32_t* sorted_token_ids, int32_t* expert_ids,
                       int32_t* num_tokens_post_padded, void* workspace,
                       int64_t workspace_bytes, hipStream_t stream);

/* glm52_moe_align_ws with no workspace argument and no allocation: the chunk histograms
 * live in a scratch array of the library's own (512 KB per GPU, held until the process
 * ends), whose device address the first call on each device looks up with that device
 * current.  Same outputs, bit for bit.  numel <= 1048576 and num_experts <= 256, else
 * GLM52_EINVAL with nothing launched.  Calls that overlap on one GPU share the scratch and
 * race; the stream must belong to the current device.  No counterpart in the reference:
 * it is for callers that cannot allocate (code under graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). */
int glm52_moe_align_noalloc(const int32_t* topk_ids, int numel, int block_m, int num_experts,
                            int capacity, int32_t* sorted_token_ids, int32_t* expert_ids,
                            int32_t* num_tokens_post_padded, hipStream_t stream);

/* glm52_router_topk followed by glm52_moe_align in one single-workgroup launch, for
 * decode (T * topk <= 256).  Replaces the topk_only + moe_align_block_size pair
 * (glm52/kernels/norm_router.py:352-354, glm52/reference.py:85-128). */
int glm52_router_topk_align(const float* logits, int64_t stride_l, const float* bias, float* topw,
                            int64_t stride_w, int32_t* topi, int64_t stride_i, int T, int E,
                            int topk, float scale, int norm_prob, int block_m, int capacity,
                            int32_t* sorted_token_ids, int32_t* expert_ids,
                            int32_t* num_tokens_post_padded, hipStream_t stream);

/* Decode front end in one launch (T <= 4): ResAdd + RMSNorm (h1, y), router logits from
 * the gate rows ([E, H], K contiguous), sigmoid + biased top-k, renormalisation and
 * scaling, and the dispatch layout; outputs bit-identical to glm52_add_rmsnorm +
 * glm52_router_logits + glm52_router_topk_align.  Replaces the chain
 * add_rmsnorm.fused_add_rmsnorm (glm52/kernels/add_rmsnorm.py:234-236) ->
 * norm_router.router_gemm -> topk_only (glm52/kernels/norm_router.py:347-354) ->
 * reference.moe_align_block_size (glm52/reference.py:85-128).  `counter` is one int32
 * that must be zero before the first launch; the kernel leaves it zero.  Launches that
 * overlap on one counter race. */
int glm52_decode_front(const void* x, int64_t stride_x, const void* res, int64_t stride_r,
                       const void* w_norm, void* h1, int64_t stride_h, void* y, int64_t stride_y,
                       const void* gate, int64_t stride_g, const float* bias, float* logits,
                       int64_t stride_l, float* topw, int64_t stride_w, int32_t* topi,
                       int64_t stride_i, int T, int H, int E, int topk, float eps, float scale,
                       int norm_prob, int block_m, int capacity, int32_t* sorted_token_ids,
                       int32_t* expert_ids, int32_t* num_tokens_post_padded, int32_t* counter,
                       hipStream_t stream);

/* The norm and router-logits part of glm52_decode_front (T <= 4), without the top-k and
 * the layout: h1, y and logits, bit-identical to glm52_add_rmsnorm + glm52_router_logits.
 * Replaces add_rmsnorm.fused_add_rmsnorm (glm52/kernels/add_rmsnorm.py:234-236) followed
 * by norm_router.router_gemm (glm52/kernels/norm_router.py:347-349). */
int glm52_decode_norm_logits(const void* x, int64_t stride_x, const void* res, int64_t stride_r,
                             const void* w_norm, void* h1, int64_t stride_h, void* y,
                             int64_t stride_y, const void* gate, int64_t stride_g, float* logits,
                             int64_t stride_l, int T, int H, int E, float eps,
                             hipStream_t stream);

/* Decode (T <= 4): glm52_router_topk_align (block_m 16) followed by glm52_moe_gemm_shared
 * (gated, unweighted) in one launch -- the routing is derived from the logits inside the
 * GEMM.  Writes topw / topi and the layout (sorted_token_ids, expert_ids,
 * num_tokens_post_padded; `capacity` slots) exactly as glm52_router_topk_align, and
 * c[f] = bf16(silu(a[f / topk] . w[e, n]) * (a[f / topk] . w[e, gate_up_offset + n])) for
 * the routed slots, c_shared[t] likewise with w_shared for tokens t < T.  Replaces
 * norm_router.topk_only (glm52/kernels/norm_router.py:352-354) ->
 * reference.moe_align_block_size (glm52/reference.py:85-128) ->
 * moe_gateup.launch_gateup(fused=True) (glm52/kernels/moe_gateup.py:199-248) for the routed
 * and the shared expert (glm52/bench/bench_layer.py:470-480). */
int glm52_moe_gemm_route_shared(const float* logits, int64_t stride_l, const float* bias, int T,
                                int E, int topk, float scale, int norm_prob, float* topw,
                                int64_t stride_w, int32_t* topi, int64_t stride_i,
                                int32_t* sorted_token_ids, int32_t* expert_ids,
                                int32_t* num_tokens_post_padded, int capacity, const void* a,
                                int64_t stride_am, const void* w, int64_t stride_we,
                                int64_t stride_wn, int gate_up_offset, void* c, int64_t stride_cm,
                                const void* a_shared, int64_t stride_as, const void* w_shared,
                                void* c_shared, int64_t stride_cs, int n_out, int k,
                                hipStream_t stream);

/* glm52_moe_gemm_route_shared on packed weights: w_packed = glm52_pack_w512 of w13 (gated,
 * n_out outputs, gate_up_offset n_out), w_shared_packed the same of the [1, 2 n_out, k]
 * shared w13; n_out % 256 == 0, k % 512 == 0.  The same routing, layout and bits as the
 * row-major entry.  Replaces the same reference chain: norm_router.topk_only
 * (glm52/kernels/norm_router.py:352-354) -> reference.moe_align_block_size
 * (glm52/reference.py:85-128) -> moe_gateup.launch_gateup(fused=True)
 * (glm52/kernels/moe_gateup.py:199-248), routed and shared (glm52/bench/bench_layer.py:470-480),
 * on the one resident weight layout this build keeps. */
int glm52_moe_gemm_route_shared_packed(const float* logits, int64_t stride_l, const float* bias,
                                       int T, int E, int topk, float scale, int norm_prob,
                                       float* topw, int64_t stride_w, int32_t* topi,
                                       int64_t stride_i, int32_t* sorted_token_ids,
                                       int32_t* expert_ids, int32_t* num_tokens_post_padded,
                                       int capacity, const void* a, int64_t stride_am,
                                       const void* w_packed, void* c, int64_t stride_cm,
                                       const void* a_shared, int64_t stride_as,
                                       const void* w_shared_packed, void* c_shared,
                                       int64_t stride_cs, int n_out, int k, hipStream_t stream);

/* Grouped expert GEMM on bf16 MFMA.  Replaces moe_gateup.launch_gateup
 * (glm52/kernels/moe_gateup.py:199-248; gated = fused SwiGLU, gate_up_offset = I) and
 * moe_down_merge.launch_down with fuse_merge=False (glm52/kernels/moe_down_merge.py:427-476;
 * topk_weights non-null = MUL_ROUTED_WEIGHT).  A rows are a[sorted_id / a_row_div],
 * W is [E, N, K] with K contiguous, C rows are indexed by the flat token id.
 * variant: 0 auto, 1 weight-streaming, 2 register-staged LDS tiles (block_m in {32, 64,
 * 128}), 3 / 4 wide 256-row W tiles fed by direct global -> LDS loads through 64-k / 32-k
 * stages (block_m in {64, 128}), 5 512-row W tiles on the 32x32x16 MFMA (block_m in
 * {64, 128}), 6 contiguous-run weight stream (block_m 16); auto runs 6 at block_m 16 and
 * 5 at 64 and 128, falling back to 1 and 3 for shapes those have no instance for. */
int glm52_moe_gemm(const void* a, int64_t stride_am, int a_row_div, const void* w,
                   int64_t stride_we, int64_t stride_wn, int gate_up_offset, void* c,
                   int64_t stride_cm, const float* topk_weights, const int32_t* sorted_token_ids,
                   const int32_t* expert_ids, const int32_t* num_tokens_post_padded,
                   int capacity, int block_m, int num_valid_tokens, int n_out, int k, int gated,
                   int variant, hipStream_t stream);

/* glm52_moe_gemm (weight-streaming mapping, block_m = 16) with the shared expert in the
 * same launch: an extra expert with weights w_shared ([N, K], K contiguous, rows strided
 * like w) applied to rows 0 .. shared_rows - 1 of a_shared, without routing weight,
 * written to c_shared.  Replaces the routed + shared launch pairs of the reference chain
 * (launch_gateup twice, launch_down twice: glm52/bench/bench_layer.py:430-480). */
int glm52_moe_gemm_shared(const void* a, int64_t stride_am, int a_row_div, const void* w,
                          int64_t stride_we, int64_t stride_wn, int gate_up_offset, void* c,
                          int64_t stride_cm, const float* topk_weights,
                          const int32_t* sorted_token_ids, const int32_t* expert_ids,
                          const int32_t* num_tokens_post_padded, int capacity, int block_m,
                          int num_valid_tokens, const void* a_shared, int64_t stride_as,
                          const void* w_shared, void* c_shared, int64_t stride_cs,
                          int shared_rows, int n_out, int k, int gated, hipStream_t stream);

/* Packed weights, the one resident layout of this build's block: no counterpart in the
 * reference, whose kernels read W in place.  The prefill mapping reads each 32-k stage of a
 * 512-row W tile as 512 runs of 64 bytes; the packed copy holds every stage as 32 KB of
 * contiguous memory in the order the tile's loads fill LDS, and each 1 KB load slot of a
 * stage (16 rows x 32 k) is also what the decode weight stream reads.  Packing is done once
 * per weight tensor; the GEMMs on the packed copy compute the same bits as glm52_moe_gemm
 * (variants 5 and 6) on the original.
 *   glm52_packed_w512_bytes: bytes of the packed copy of num_experts experts' W for n_out
 *     outputs (gated: `gate` rows n and `up` rows gate_up_offset + n) and K = k; negative
 *     if the mapping has no instance for the shape (n_out % 256 gated / 512 plain, k % 64).
 *   glm52_pack_w512: writes that copy (w, strides, gate_up_offset as for glm52_moe_gemm).
 *   glm52_moe_gemm_packed: glm52_moe_gemm with block_m 64, 128 or 256 on the packed copy,
 *     or with block_m 16 (the decode weight stream, k % 512 == 0), which reads each packed
 *     load slot -- 16 rows x 32 k, 1 KB of contiguous memory -- as it streams the rows. */
int64_t glm52_packed_w512_bytes(int num_experts, int n_out, int k, int gated);
int glm52_pack_w512(const void* w, int64_t stride_we, int64_t stride_wn, int num_experts,
                    int n_out, int k, int gate_up_offset, int gated, void* packed,
                    hipStream_t stream);
int glm52_moe_gemm_packed(const void* a, int64_t stride_am, int a_row_div, const void* w_packed,
                          void* c, int64_t stride_cm, const float* topk_weights,
                          const int32_t* sorted_token_ids, const int32_t* expert_ids,
                          const int32_t* num_tokens_post_padded, int capacity, int block_m,
                          int num_valid_tokens, int n_out, int k, int gated, hipStream_t stream);

/* glm52_moe_gemm_packed with the shared expert in the same launch (prefill, block_m 64,
 * 128 or 256): an extra expert whose packed weights w_shared_packed (glm52_pack_w512 of
 * the [1, N, K] shared weight, same n_out / k / gated) apply to rows 0 .. shared_rows - 1
 * of a_shared, without routing weight, written to c_shared.  Replaces the routed + shared
 * launch pairs of the reference chain (launch_gateup twice, launch_down twice:
 * glm52/bench/bench_layer.py:430-480) for block sizes 64 and up. */
int glm52_moe_gemm_packed_shared(const void* a, int64_t stride_am, int a_row_div,
                                 const void* w_packed, void* c, int64_t stride_cm,
                                 const float* topk_weights, const int32_t* sorted_token_ids,
                                 const int32_t* expert_ids,
                                 const int32_t* num_tokens_post_padded, int capacity,
                                 int block_m, int num_valid_tokens, const void* a_shared,
                                 int64_t stride_as, const void* w_shared_packed, void* c_shared,
                                 int64_t stride_cs, int shared_rows, int n_out, int k, int gated,
                                 hipStream_t stream);

/* o_proj + ResAdd1, the dense GEMM upstream of the block (`glm52/kernels/oproj_resadd.py`).
 * A [M, K] bf16 (K contiguous), B [K, N] bf16 (strides in elements), r [M, N] bf16.
 *   glm52_oproj_gemm: c = A @ B with the epilogue of oproj_gemm_kernel: r non-null adds
 *     the residual (FUSE_RESADD); c_f32 != 0 accumulates into an fp32 c, c += result
 *     (ATOMIC_OUT, without atomics: one writer per element); else c = bf16(result).
 *     Replaces oproj_resadd.gemm_launch (glm52/kernels/oproj_resadd.py:144-178).  M <= 16
 *     with B N-contiguous streams B (split K, fixed-order reduction); otherwise b_packed
 *     from glm52_oproj_pack is required (N % 512 == 0, K % 64 == 0).  The workspace holds
 *     glm52_oproj_workspace_bytes(M, N, K) bytes.
 *   glm52_oproj_pack / glm52_oproj_packed_bytes: B packed once as the 512-row tile
 *     mapping's W = B^T, cut into `splits` K slices (no counterpart in the reference);
 *     glm52_oproj_splits(M, N, K) is the count glm52_oproj_gemm wants for that shape
 *     (more slices when M gives too few 512-row tiles to fill the GPU).
 *   glm52_cast_add: o = bf16(c (+ r)), c bf16 or fp32 -- oproj_resadd.epilogue_launch
 *     (glm52/kernels/oproj_resadd.py:181-196). */
int64_t glm52_oproj_workspace_bytes(int M, int N, int K);
int glm52_oproj_splits(int M, int N, int K);
int64_t glm52_oproj_packed_bytes(int K, int N);
int glm52_oproj_pack(const void* b, int64_t stride_bk, int64_t stride_bn, int K, int N,
                     int splits, void* packed, hipStream_t stream);
int glm52_oproj_gemm(const void* a, int64_t stride_am, const void* b, int64_t stride_bk,
                     int64_t stride_bn, const void* b_packed, int splits, const void* r,
                     int64_t stride_rm, void* c, int64_t stride_cm, int c_f32, int M, int N,
                     int K, void* workspace, int64_t workspace_bytes, hipStream_t stream);
int glm52_cast_add(const void* c, int c_f32, int64_t stride_c, const void* r, int64_t stride_r,
                   void* o, int64_t stride_o, int M, int N, hipStream_t stream);

/* Half-fused pre-norm (`glm52/kernels/lazy_prenorm.py`, fusion #11b').
 *   glm52_rstd: rstd[t] = fp32(1 / sqrt(sum_k x[t, k]^2 / N + eps)) for x [T, N] bf16, the
 *     squares summed in fp64 (the statistic of glm52_add_rmsnorm); rstd_flat, if
 *     non-null, receives each value `repeat` times.  Replaces rstd_kernel / launch_rstd
 *     (glm52/kernels/lazy_prenorm.py:346-390).
 *   glm52_router_logits_rstd: glm52_router_logits with the USE_RSTD epilogue of the
 *     reference's router GEMM (glm52/kernels/lazy_prenorm.py:229-330, launch_router :457):
 *     each logit, rounded to fp32, times rstd[t] (one fp32 product) before its store. */
int glm52_rstd(const void* x, int64_t stride_x, int T, int N, float eps, float* rstd,
               float* rstd_flat, int repeat, hipStream_t stream);
/* glm52_prenorm_router_rows: the same router for T <= 4 tokens on a gate read as rows
 *     ([E, H], the transposed view of the [H, E] operand): one workgroup per gate row; when
 *     rstd_in is null the statistic is computed in the same pass over h (the reference's
 *     FUSE_NORM, lazy_prenorm.py:300-322) and written to rstd_out if that is non-null. */
int glm52_prenorm_router_rows(const void* h, int64_t stride_h, const void* gate, int64_t stride_g,
                              const float* rstd_in, float eps, float* logits, int64_t stride_l,
                              float* rstd_out, int T, int H, int E, hipStream_t stream);
int glm52_router_logits_rstd(const void* y, int64_t stride_y, const void* wgt, int64_t stride_wk,
                             int64_t stride_we, int wg_is_f32, const float* rstd, float* logits,
                             int64_t stride_l, void* workspace, int64_t workspace_bytes, int T,
                             int H, int E, hipStream_t stream);
/* glm52_router_rstd: glm52_router with the same epilogue -- the router GEMM with USE_RSTD
 *     (glm52/kernels/lazy_prenorm.py:229-330, launch_router :457-489) followed by the
 *     top-k the block's router takes on its logits (topk_only, glm52/kernels/
 *     norm_router.py:352-354): each logit is its fp32 value times rstd[t], and ids and
 *     weights are the exact rule's on those logits.  On the gate's rows from 17 tokens the
 *     bounded path of glm52_router runs (its workspace query, its logits semantics: exact
 *     times rstd for the candidates, within the bound times rstd elsewhere). */
int glm52_router_rstd(const void* y, int64_t stride_y, const void* wgt, int64_t stride_wk,
                      int64_t stride_we, int wg_is_f32, const float* rstd, float* logits,
                      int64_t stride_l, void* workspace, int64_t workspace_bytes,
                      const float* bias, float* topw, int64_t stride_w, int32_t* topi,
                      int64_t stride_i, int T, int H, int E, int topk, float scale,
                      int norm_prob, hipStream_t stream);

/* The down GEMM with the atomic expert merge: fusion #8(a) / #9(a), replaces
 * moe_down_merge.launch_down(fuse_merge=True) (glm52/kernels/moe_down_merge.py:427-476,
 * FUSE_MERGE epilogue :160-169).  For every valid flat token f of the layout,
 * out[f / top_k, :] += bf16(topk_weights[f] * (a[f] . w[e]^T)), each add a packed bf16
 * atomic, so the rounding order depends on timing.  out [T, n_out] is seeded by the
 * caller (zeros or the residual; launch_seed).  block_m 16, 64 or 128; w_packed
 * (glm52_pack_w512, may be null; not with block_m 16) is read by the 64/128 mapping. */
int glm52_moe_down_merge(const void* a, int64_t stride_am, const void* w, int64_t stride_we,
                         int64_t stride_wn, const void* w_packed, void* out, int64_t stride_om,
                         const float* topk_weights, const int32_t* sorted_token_ids,
                         const int32_t* expert_ids, const int32_t* num_tokens_post_padded,
                         int capacity, int block_m, int num_valid_tokens, int top_k, int n_out,
                         int k, hipStream_t stream);

/* Token-major down GEMV + expert merge (+ residual): fusion #8(b) / #9(b), replaces
 * moe_down_merge.launch_down_token_major (glm52/kernels/moe_down_merge.py:479-516,
 * moe_down_token_major_kernel :165-293).
 *   out[t, n] = bf16(sum_k w[t, k] * (a[t * top_k + k] . w2[ids[t, k], n]) (+ r[t, n])),
 * fp32 accumulation over all of a token's experts, one rounding, no atomics.  ids outside
 * [0, num_experts) contribute nothing.  With w2_shared non-null a shared expert (activation
 * a_shared[t], weight 1) joins the sum.  K (= I) must be 1024 or 2048. */
int glm52_down_token_major(const void* a, int64_t stride_am, const void* w2, int64_t stride_we,
                           int64_t stride_wn, const float* topk_weights, const int32_t* topk_ids,
                           int64_t stride_tk, int top_k, int num_experts, const void* a_shared,
                           int64_t stride_as, const void* w2_shared, int64_t stride_ws,
                           const void* residual, int64_t stride_rm, void* out, int64_t stride_om,
                           int T, int N, int K, hipStream_t stream);

/* glm52_down_token_major on packed weights: w2_packed = glm52_pack_w512 of w2 ([E, N, K],
 * plain, n_out = N), w2_shared_packed (may be null) the same of the [1, N, K] shared w2;
 * N % 512 == 0, K 1024 or 2048, a / a_shared row strides as for glm52_down_token_major.
 * The same sum with one fp32 accumulation and one rounding, its adds in another order.
 * Replaces moe_down_merge.launch_down_token_major (glm52/kernels/moe_down_merge.py:479-516)
 * on the one resident weight layout this build keeps. */
int glm52_down_token_major_packed(const void* a, int64_t stride_am, const void* w2_packed,
                                  const float* topk_weights, const int32_t* topk_ids,
                                  int64_t stride_tk, int top_k, int num_experts,
                                  const void* a_shared, int64_t stride_as,
                                  const void* w2_shared_packed, const void* residual,
                                  int64_t stride_rm, void* out, int64_t stride_om, int T, int N,
                                  int K, hipStream_t stream);

/* y[M, I] = bf16(silu(x[:, :I]) * x[:, I:]).  Replaces moe_gateup.launch_silu_and_mul
 * (glm52/kernels/moe_gateup.py:251-266). */
int glm52_silu_and_mul(const void* x, int64_t stride_x, void* y, int64_t stride_y, int M, int I,
                       hipStream_t stream);

/* out[T, N] = bf16(sum_k y[t, k] (+ residual)).  Replaces moe_down_merge.launch_moe_sum
 * (glm52/kernels/moe_down_merge.py:519-540). */
int glm52_moe_sum(const void* y, int64_t stride_t, int64_t stride_k, void* out, int64_t stride_o,
                  const void* residual, int64_t stride_r, int T, int N, int topk, int add_residual,
                  hipStream_t stream);

/* o = bf16(x + r).  Replaces moe_down_merge.launch_resadd (glm52/kernels/moe_down_merge.py:543-559). */
int glm52_resadd(const void* x, int64_t stride_x, const void* r, int64_t stride_r, void* o,
                 int64_t stride_o, int M, int N, hipStream_t stream);

/* Weighted merge + ResAdd.  Replaces merge_resadd.fused_merge_resadd / merge_only /
 * resadd_only (glm52/kernels/merge_resadd.py:243-255). */
int glm52_merge_resadd(const void* y, int64_t stride_yt, int64_t stride_yk, const float* wt,
                       int64_t stride_wt, const void* res, int64_t stride_r, void* m,
                       int64_t stride_m, void* out, int64_t stride_o, int T, int N, int topk,
                       int do_merge, int do_resadd, int round_mid, hipStream_t stream);

/* Block tail: out = bf16(sum_{k<8} y[t, k] + h + shared_out) (shared_out nullable).
 * Replaces the pair launch_moe_sum(add_residual=True) + launch_resadd(shared) of
 * glm52/bench/bench_layer.py:462-480 with one pass and one rounding. */
int glm52_block_merge(const void* y, int64_t stride_yt, int64_t stride_yk, const void* h,
                      int64_t stride_h, const void* shared_out, int64_t stride_s, void* out,
                      int64_t stride_o, int T, int N, hipStream_t stream);

/* Read-bandwidth probe: streams `bytes` (a multiple of 16) of `buf` with 16-byte loads
 * (non-temporal if `nontemporal`) on `grid` workgroups of 256.  It calibrates the HBM
 * ceiling, following the reference's rule of measured ceilings (glm52/traffic.py:70-81).
 * It replaces no launcher of the reference's kernel API. */
int glm52_stream_read(const void* buf, int64_t bytes, int nontemporal, int grid, uint32_t* sink,
                      hipStream_t stream);

/* Self-test of the MFMA result layouts the kernels assume (bf16 16x16x32, fp64 16x16x4 and
 * bf16 32x32x16): writes 1536 floats -- two 16 x 16 fp32 matrices whose row r is all (r + 1),
 * then the 64 x 16 raw 32x32x16 results (lane-major) of C[r][c] = 32 r + c.
 * No counterpart in the reference. */
int glm52_selftest_mfma_layout(float* out, hipStream_t stream);

/* Measurement hook of the prefill tile (the 512-row and 256 x 256 tile launches of
 * glm52_moe_gemm, glm52_moe_gemm_packed(_shared), glm52_oproj_gemm): with `buf` set (at least
 * 256 x 4 words of device memory), every later launch writes, per workgroup w, words
 * 4w .. 4w+3 = its start and end on the 100 MHz wall clock, the items it ran and its XCD;
 * with `buf` null (the default) nothing is recorded.  Process-wide; not for overlapping
 * launches.  No counterpart in the reference: it shows how the items are dealt. */
int glm52_debug_item_trace(void* buf, int64_t bytes);

#ifdef __cplusplus
}
#endif

#endif /* GLM52_HIP_H */
