/*
 * mrsa.h - C ABI of the MI355X (gfx950) mask-routed sparse attention library.
 *
 * Every entry point takes raw device pointers, element counts and scalars,
 * enqueues its kernels on `stream` (a hipStream_t; NULL = the default stream)
 * and returns immediately.  Nothing here allocates device memory: callers pass
 * every output and workspace buffer.  Inputs are never written.
 *
 * Tensor conventions: "bf16" buffers hold raw bfloat16 bit patterns, "bool"
 * buffers hold one byte per element (0 = false, anything else = true), all
 * tensors are dense row-major with the shapes given in brackets, batch first.
 *
 * Return value: MRSA_OK, or a status naming the first problem found.  Shape /
 * argument problems are detected on the host before anything is launched.
 *
 * Reference citations are relative to the root of
 * NRHLYM/Mask-Routed-Sparse-Attention-for-Long-Context-Diffusion-Language-Models.
 */
#ifndef MRSA_H
#define MRSA_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MRSA_OK 0
#define MRSA_ERR_INVALID_ARGUMENT 1 /* bad shape, size or pointer */
#define MRSA_ERR_UNSUPPORTED 2      /* valid call outside what the kernels implement */
#define MRSA_ERR_LAUNCH 3           /* the HIP runtime rejected a launch */
#define MRSA_ERR_SCRATCH 4          /* exceeds a no-allocation entry point's static buffer */

/* Human-readable text for a status code (static storage). */
const char* mrsa_status_string(int status);

/* Increments whenever an entry point's signature or semantics change. */
int mrsa_abi_version(void);

/*
 * Output fusion: out = bf16(float(remote) + float(local_weight) * float(local)).
 * Replaces fuse_hils_outputs (ops/hils_bidir_output_fusion_tilelang.py:138-148,
 * kernel :15-37).
 *   remote_output, local_output, output: bf16 [rows, head_dim]
 *   local_weight:                        bf16 [rows]
 * (rows = B * L * H for the reference's [B, L, H, D] tensors.)
 */
int mrsa_fuse_hils_outputs_fwd(const void* remote_output, const void* local_output,
                               const void* local_weight, void* output, int64_t rows,
                               int64_t head_dim, void* stream);

/*
 * Backward of the output fusion.  Replaces _FuseHiLSOutputs.backward
 * (ops/hils_bidir_output_fusion_tilelang.py:90-99, kernel _fusion_bwd :40-77).
 *   local_output, grad_output:  bf16 [rows, head_dim]
 *   local_weight:               bf16 [rows]
 *   d_remote (out) = grad_output; d_local (out) = bf16(local_weight * grad);
 *   d_weight (out): bf16 [rows] = bf16(sum_d grad * local) (fp32 sum)
 */
int mrsa_fuse_hils_outputs_bwd(const void* local_output, const void* local_weight,
                               const void* grad_output, void* d_remote, void* d_local,
                               void* d_weight, int64_t rows, int64_t head_dim, void* stream);

/*
 * Landmark (mask-token) chunk-summary attention pool.
 * Replaces chunk_attn_pool_gqa (ops/chunk_attn_pool_gqa_tilelang.py:425-448):
 * the fused kernel _pool_gqa_fwd (:47-180) when groups > 1, and the compiled
 * torch twin _compact_pool_torch (:17-37) when dense_torch_semantics != 0
 * (the reference takes that branch for groups == 1).
 *   mu_q:      bf16 [batch_chunks, kv_heads, groups, head_dim]
 *   k_chunked: bf16 [batch_chunks, chunk_size, kv_heads, head_dim]
 *   key_valid: bool [batch_chunks, chunk_size]
 *   landmark_keys (out): bf16 [batch_chunks, kv_heads, groups, head_dim]
 *   entropy (out):       fp32 [batch_chunks, kv_heads, groups]
 *   bias_scale:  optional fp32 [kv_heads * groups]; when given together with
 *   prior_bias (out, fp32 [batch_chunks, kv_heads, groups]) the kernel also
 *   writes prior_bias = entropy * bias_scale[head] (attention.py:1425-1430).
 * Limits: 2 <= chunk_size <= 128, groups <= 16, head_dim <= 256, head_dim % 8 == 0.
 */
int mrsa_chunk_attn_pool_gqa_fwd(const void* mu_q, const void* k_chunked,
                                 const uint8_t* key_valid, int64_t batch_chunks,
                                 int64_t chunk_size, int64_t kv_heads, int64_t groups,
                                 int64_t head_dim, float sm_scale, int dense_torch_semantics,
                                 const float* bias_scale, void* landmark_keys, float* entropy,
                                 float* prior_bias, void* stream);

/*
 * The same pool reading the landmark queries in place: query row of
 * batch-chunk bc at mu_q + bc * mu_row_stride elements (each row holds
 * [kv_heads][groups][head_dim] contiguous), so the mask-token rows of the
 * route queries [B, L, Hq, D] (mu_q = route_q + (chunk_size - 1) * Hq * D,
 * mu_row_stride = chunk_size * Hq * D) need no gather.  No reference
 * counterpart (the reference gathers the rows with a strided slice first).
 * mu_row_stride >= kv_heads * groups * head_dim.
 */
int mrsa_chunk_attn_pool_gqa_strided_fwd(const void* mu_q, int64_t mu_row_stride,
                                         const void* k_chunked, const uint8_t* key_valid,
                                         int64_t batch_chunks, int64_t chunk_size,
                                         int64_t kv_heads, int64_t groups, int64_t head_dim,
                                         float sm_scale, int dense_torch_semantics,
                                         const float* bias_scale, void* landmark_keys,
                                         float* entropy, float* prior_bias, void* stream);

/*
 * Landmark refresh of the affected chunks of a K/V cache, in place: replaces
 * the gather-pool-scatter of the cached block step
 * (dream_dllm_hils/fastdllm_attention.py:236-292: the landmark rows of
 * route_q located among the query positions, the chunks' key rows and valid
 * bytes gathered from the cache, chunk_attn_pool_gqa, prior = entropy x
 * entropy_bias_scale, index_copy_ into landmark_keys / prior_bias) with one
 * launch that reads everything in place.  Fused pool semantics, the same
 * bits as mrsa_chunk_attn_pool_gqa_fwd on the gathered rows.
 *   route_q: bf16 [batch, query_len, kv_heads * groups, head_dim]
 *   query_positions: int64 [query_len], sorted ascending
 *   key: bf16 [batch, cache_len, kv_heads, head_dim]; key_valid: u8 [batch, cache_len]
 *   chunks: int64 [count]; bias_scale: fp32 [kv_heads * groups]
 *   landmark_keys (in/out): bf16 [batch, cache_len / 64, kv_heads, groups, head_dim]
 *   prior_bias (in/out): fp32 [batch, cache_len / 64, kv_heads, groups]
 * A chunk outside [0, cache_len / 64), or whose landmark position
 * (64 c + 63) is not a query position, is left as it is (the argument checks
 * of mrsa_cached_step_checks report both).
 * Limits: chunk_size == 64, head_dim == 128, groups <= 16, cache_len % 64 == 0.
 */
int mrsa_pool_cached_chunks_fwd(const void* route_q, const int64_t* query_positions,
                                int64_t query_len, const void* key, const uint8_t* key_valid,
                                int64_t batch, int64_t cache_len, const int64_t* chunks,
                                int64_t count, int64_t kv_heads, int64_t groups,
                                int64_t head_dim, int64_t chunk_size, float sm_scale,
                                const float* bias_scale, void* landmark_keys, float* prior_bias,
                                void* stream);

/*
 * Backward of the landmark pool; the probabilities are recomputed from mu_q
 * and K.  Replaces _ChunkAttnPoolGQA.backward
 * (ops/chunk_attn_pool_gqa_tilelang.py:355-394, kernel _pool_gqa_bwd :183-325)
 * and, with dense_torch_semantics != 0, the autograd of _compact_pool_torch
 * (:17-37) that the reference runs for groups == 1.
 *   mu_q, k_chunked, key_valid: as mrsa_chunk_attn_pool_gqa_fwd
 *   grad_landmark: bf16 [batch_chunks, kv_heads, groups, head_dim] or NULL (zeros)
 *   grad_entropy:  fp32 [batch_chunks, kv_heads, groups] or NULL (zeros)
 *   d_mu_q (out):      bf16 [batch_chunks, kv_heads, groups, head_dim]
 *   d_k_chunked (out): bf16 [batch_chunks, chunk_size, kv_heads, head_dim]
 * Limits: as the forward.
 */
int mrsa_chunk_attn_pool_gqa_bwd(const void* mu_q, const void* k_chunked,
                                 const uint8_t* key_valid, const void* grad_landmark,
                                 const float* grad_entropy, int64_t batch_chunks,
                                 int64_t chunk_size, int64_t kv_heads, int64_t groups,
                                 int64_t head_dim, float sm_scale, int dense_torch_semantics,
                                 void* d_mu_q, void* d_k_chunked, void* stream);

/*
 * Remote-route drop mask (1 = the chunk may not be routed to).
 * Replaces remote_drop_mask (dream_dllm_hils/kernel_utils.py:102-161) with the
 * chunk-aligned local bounds of chunk_aligned_local_bounds (:75-99).
 *   valid_mask:   bool [batch, seq_len]
 *   allowed_mask: optional bool [batch, seq_len, seq_len]
 *   drop_mask (out): int32 [batch, seq_len, seq_len / chunk_size]
 */
int mrsa_remote_drop_mask(const uint8_t* valid_mask, const uint8_t* allowed_mask,
                          int64_t batch, int64_t seq_len, int64_t window, int64_t chunk_size,
                          int32_t* drop_mask, void* stream);

/*
 * Rows of the remote drop mask for queries at given cache positions: row i is
 * row query_positions[i] of mrsa_remote_drop_mask(valid_mask, NULL, ...).
 * Replaces remote_drop_mask(cache.key_valid, window, chunk_size)
 * .index_select(1, query_positions) in the cached decode path
 * (dream_dllm_hils/fastdllm_attention.py:295-299), without materialising the
 * full [batch, seq_len, chunks] mask.
 *   valid_mask: bool [batch, seq_len]; query_positions: int64 [rows], each in
 *   [0, seq_len) (not checked on the device)
 *   drop_mask (out): int32 [batch, rows, seq_len / chunk_size]
 */
int mrsa_remote_drop_mask_rows(const uint8_t* valid_mask, const int64_t* query_positions,
                               int64_t batch, int64_t seq_len, int64_t rows, int64_t window,
                               int64_t chunk_size, int32_t* drop_mask, void* stream);

/*
 * The device-side argument checks of the cached block step in one launch
 * (one workgroup), for callers that validate before launching, as
 * cached_route_attention's checks do (dream_dllm_hils/fastdllm_attention.py:
 * 54-66, 84-118: positions sorted, unique and in range, affected chunks in
 * range, each affected chunk's landmark position among the query positions).
 *   query_positions: int64 [count]; affected_chunks: int64 [affected_count]
 *   flags (out): int32 [4] -- [0] positions not strictly ascending, [1] a
 *   position outside [0, cache_len), [2] an affected chunk outside
 *   [0, cache_len / chunk_size), [3] an affected chunk whose landmark position
 *   (c chunk_size + chunk_size - 1) is not a query position (meaningful once
 *   [0] is clear)
 * No reference counterpart as an entry point: the reference runs these
 * checks as separate torch expressions with host synchronisations.
 */
int mrsa_cached_step_checks(const int64_t* query_positions, int64_t count,
                            const int64_t* affected_chunks, int64_t affected_count,
                            int64_t cache_len, int64_t chunk_size, int32_t* flags, void* stream);

/*
 * Route scoring with per-KV-group top-k ("softmax then max pooling").
 * Replaces ref_softmax_topk_max_pooling (ops/topk_head_softmax.py:15-156),
 * which route_topk_g7 (dream_dllm_hils/routing.py:52-171) and
 * online_softmax_topk_head (ops/topk_head_softmax.py:1242-1415) dispatch to.
 *   q:   bf16 [batch, seq_len, kv_heads, groups, head_dim] (routing query)
 *   lmk: bf16 [batch, chunks, kv_heads * groups, head_dim] when per_head_lmk,
 *        else [batch, chunks, kv_heads, head_dim]
 *   lse_local: fp32 [batch, seq_len, kv_heads, groups] (unused for pre-softmax)
 *   bias:      optional fp32 [batch, chunks, kv_heads, groups]
 *   drop_mask: optional int32 [batch, seq_len, chunks] (nonzero = drop)
 *   derive_window >= 0 replaces drop_mask by the in-kernel equivalent of
 *     remote_drop_mask(key_valid, derive_window, block_size) (requires
 *     chunks * block_size == seq_len); key_valid (bool [batch, seq_len]) may
 *     then be NULL for all-valid.
 *   is_causal / window_size / q_offset: the reference's causal chunk mask.
 *   selection_mode: 0 = "post_softmax", 1 = "pre_softmax".
 *   indices (out): int32 [batch, seq_len, kv_heads, topk], ascending, -1 last.
 *   scores (out):  [batch, seq_len, kv_heads, groups, topk] raw scaled q.k at
 *     the picked chunks (-inf at -1 slots); bf16, or fp32 if scores_fp32.
 * Ties in the selection score are broken toward the lower chunk index.
 */
int mrsa_route_topk_fwd(const void* q, const void* lmk, const float* lse_local,
                        const float* bias, const int32_t* drop_mask, const uint8_t* key_valid,
                        int64_t derive_window, int64_t batch, int64_t seq_len, int64_t chunks,
                        int64_t kv_heads, int64_t groups, int64_t head_dim, int64_t topk,
                        int64_t block_size, int per_head_lmk, int is_causal, int64_t window_size,
                        int64_t q_offset, int selection_mode, float sm_scale, int32_t* indices,
                        void* scores, int scores_fp32, void* stream);

/*
 * mrsa_route_topk_fwd with a caller-provided workspace (16-byte aligned).
 * The same reference call sites; the decode caller is route_topk_g7 at
 * dream_dllm_hils/fastdllm_attention.py:299-314 (32 query rows against the
 * whole cache).
 *   - Shapes of the matrix-core kernel (head_dim 128, groups 7 or 8,
 *     chunks <= 256, topk <= 64, bf16 scores, not causal): a workspace of
 *     at least batch * seq_len * kv_heads * groups * chunks * 2 bytes holds
 *     the bf16 raw scores of every chunk, so the kernel runs one pass and
 *     gathers the picks' scores from it instead of recomputing them.
 *   - Otherwise, with mrsa_route_topk_workspace_bytes() bytes and
 *     head_dim == 128, groups <= 8, chunks <= 4096, the logits of all rows are
 *     computed on the matrix cores into the fp32 workspace and selected by a
 *     second kernel, one workgroup per (row, KV head).
 * Other shapes (and a smaller workspace) take mrsa_route_topk_fwd's paths.
 * Same results either way.
 */
int64_t mrsa_route_topk_workspace_bytes(int64_t batch, int64_t seq_len, int64_t chunks,
                                        int64_t kv_heads, int64_t groups);
int mrsa_route_topk_ws_fwd(const void* q, const void* lmk, const float* lse_local,
                           const float* bias, const int32_t* drop_mask, const uint8_t* key_valid,
                           int64_t derive_window, int64_t batch, int64_t seq_len, int64_t chunks,
                           int64_t kv_heads, int64_t groups, int64_t head_dim, int64_t topk,
                           int64_t block_size, int per_head_lmk, int is_causal,
                           int64_t window_size, int64_t q_offset, int selection_mode,
                           float sm_scale, int32_t* indices, void* scores, int scores_fp32,
                           void* workspace, int64_t workspace_bytes, void* stream);

/*
 * mrsa_route_topk_ws_fwd without a caller workspace and without allocating:
 * the workspace is a static device buffer of MRSA_ROUTE_TOPK_SCRATCH_BYTES
 * per GPU inside the library.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc), e.g. the cached
 * block step's routing over up to 4096 landmarks.
 *   Arguments as mrsa_route_topk_ws_fwd minus the workspace; same results.
 *   Returns MRSA_ERR_SCRATCH when the short-block path (more than 256
 *   chunks) needs more than MRSA_ROUTE_TOPK_SCRATCH_BYTES of fp32 logits
 *   (batch * seq_len * kv_heads * groups * chunks * 4 bytes); shapes of the
 *   matrix-core path (up to 256 chunks) need none.
 *   Every call on a GPU shares that GPU's buffer: calls that overlap on one
 *   GPU (other streams, other threads) race.
 */
#define MRSA_ROUTE_TOPK_SCRATCH_BYTES (16u << 20)
int mrsa_route_topk_noalloc_fwd(const void* q, const void* lmk, const float* lse_local,
                                const float* bias, const int32_t* drop_mask,
                                const uint8_t* key_valid, int64_t derive_window, int64_t batch,
                                int64_t seq_len, int64_t chunks, int64_t kv_heads,
                                int64_t groups, int64_t head_dim, int64_t topk,
                                int64_t block_size, int per_head_lmk, int is_causal,
                                int64_t window_size, int64_t q_offset, int selection_mode,
                                float sm_scale, int32_t* indices, void* scores, int scores_fp32,
                                void* stream);

/*
 * Backward of the route scores score[l, h, g, k] = sm_scale * q[l, h, g] .
 * lmk[idx[l, h, k], hl] (hl = h * groups + g per-head, h shared): replaces
 * SoftmaxTopKMaxPoolingFusedFn.backward (ops/topk_head_softmax.py:1074-1122),
 * without its dense [batch * kv_heads * groups, seq_len, chunks] scatter
 * buffer.  The gradient is multiplied by sm_scale and rounded to bf16 (the
 * reference's mul_ in the gradient's bf16 dtype); slots whose index lies
 * outside [0, chunks) contribute nothing.
 *   q:           bf16 [batch, seq_len, kv_heads, groups, 128]
 *   landmarks:   bf16 [batch, chunks, kv_heads * groups or kv_heads, 128]
 *   indices:     int32 [batch, seq_len, kv_heads, topk]
 *   grad_scores: [batch, seq_len, kv_heads, groups, topk], bf16 or fp32
 *                (grad_scores_fp32 = 1)
 *   grad_q (out):         bf16, the shape of q
 *   grad_landmarks (out): bf16, the shape of landmarks (summed over the
 *                         group for shared landmarks)
 *   workspace: 16-byte aligned, mrsa_route_score_bwd_workspace_bytes(...)
 *              bytes (fp32 parts of grad_landmarks; grad_q in fp32 when
 *              chunks > 256).  The result does not depend on timing.
 * Requirements: head_dim 128, topk <= 4096.
 */
int64_t mrsa_route_score_bwd_workspace_bytes(int64_t batch, int64_t seq_len, int64_t chunks,
                                             int64_t kv_heads, int64_t groups,
                                             int per_head_lmk);
int mrsa_route_score_bwd(const void* q, const void* landmarks, const int32_t* indices,
                         const void* grad_scores, int grad_scores_fp32, int64_t batch,
                         int64_t seq_len, int64_t chunks, int64_t kv_heads, int64_t groups,
                         int64_t head_dim, int64_t topk, int per_head_lmk, float sm_scale,
                         void* grad_q, void* grad_landmarks, void* workspace,
                         int64_t workspace_bytes, void* stream);

/*
 * Route weights: softmax over [score_k + bias[idx_k] (k < topk), local_lse].
 * Replaces _route_weights_torch (dream_dllm_hils/attention.py:126-235; the
 * topk >= 32 path, selected at :1571-1621) and route_weights
 * (ops/hils_bidir_route_weights_tilelang.py:276-290, topk <= 31).
 *   scores: bf16 [batch, seq_len, kv_heads * groups, topk]
 *   indices: int32 [batch, seq_len, kv_heads, topk]
 *   prior_bias: fp32 [batch, chunks, kv_heads, groups]
 *   local_lse: fp32 [batch, seq_len, kv_heads * groups]
 *   gate_offset, gate_scale: fp32 device scalars (the layer's
 *   fusion_gate_offset / fusion_gate_scale parameters, read in place), or
 *   NULL when not given.  A gate_scale selects the affine-sigmoid form
 *   (sigmoid(gate_scale * (remote_lse - local) + gate_offset)); otherwise the
 *   plain softmax with local_lse - gate_offset when gate_offset is given.
 *   remote_weights (out): bf16 [batch, seq_len, kv_heads * groups, topk]
 *   local_weight (out):   bf16 [batch, seq_len, kv_heads * groups]
 *   gate_logit (out, or NULL): fp32 [batch, seq_len, kv_heads * groups], the
 *   return_gate_logit=True output (attention.py:196-235): remote_lse - local
 *   logit, affine-transformed in the affine form, 0 where every logit is
 *   masked.
 */
int mrsa_route_weights_fwd(const void* scores, const int32_t* indices, const float* prior_bias,
                           const float* local_lse, int64_t batch, int64_t seq_len,
                           int64_t chunks, int64_t kv_heads, int64_t groups, int64_t topk,
                           float temperature, const float* gate_offset, const float* gate_scale,
                           void* remote_weights, void* local_weight, float* gate_logit,
                           void* stream);

/*
 * mrsa_route_weights_fwd with _route_weights_torch's two additive inputs
 * (dream_dllm_hils/attention.py:172-181): value_bonus and selected_gumbel,
 * fp32 [batch, seq_len, kv_heads * groups, topk] (either may be null), are
 * added to each valid slot's logit after its bias, in that order, before the
 * temperature.
 */
int mrsa_route_weights_extra_fwd(const void* scores, const int32_t* indices,
                                 const float* prior_bias, const float* local_lse, int64_t batch,
                                 int64_t seq_len, int64_t chunks, int64_t kv_heads,
                                 int64_t groups, int64_t topk, float temperature,
                                 const float* gate_offset, const float* gate_scale,
                                 const float* value_bonus, const float* selected_gumbel,
                                 void* remote_weights, void* local_weight, float* gate_logit,
                                 void* stream);

/*
 * Backward of the route weights; the row logits are recomputed from the
 * forward inputs.  Replaces _RouteWeights.backward
 * (ops/hils_bidir_route_weights_tilelang.py:185-242, kernel _route_weights_bwd
 * :97-166; plain form, there at temperature 1) and the autograd of
 * _route_weights_torch (dream_dllm_hils/attention.py:126-235) in both forms.
 *   forward inputs and options: as mrsa_route_weights_fwd
 *   grad_remote: bf16 [batch, seq_len, kv_heads * groups, topk]
 *   grad_local:  bf16 [batch, seq_len, kv_heads * groups], or NULL for zeros
 *   grad_gate_logit: fp32 [batch, seq_len, kv_heads * groups], or NULL for
 *                zeros (upstream gradient of the gate_logit output)
 *   d_scores (out):    fp32 [batch, seq_len, kv_heads * groups, topk]
 *                      (0 at invalid chunk indices)
 *   d_bias (in/out):   fp32 [batch, chunks, kv_heads, groups], caller-zeroed;
 *                      each valid selected entry's gradient is added atomically
 *   d_local_lse (out): fp32 [batch, seq_len, kv_heads * groups]
 *   d_gate (in/out):   fp32 [2] = {d gate_scale, d gate_offset}, caller-zeroed;
 *                      may be NULL when neither gate option is set
 * Rows whose outputs are constant (every logit masked; the affine form with
 * no valid chunk) get zero gradients.
 */
int mrsa_route_weights_bwd(const void* scores, const int32_t* indices, const float* prior_bias,
                           const float* local_lse, const void* grad_remote,
                           const void* grad_local, const float* grad_gate_logit, int64_t batch,
                           int64_t seq_len, int64_t chunks, int64_t kv_heads, int64_t groups,
                           int64_t topk, float temperature, const float* gate_offset,
                           const float* gate_scale, float* d_scores, float* d_bias,
                           float* d_local_lse, float* d_gate, void* stream);

/*
 * mrsa_route_weights_bwd for a forward with value_bonus / selected_gumbel
 * (mrsa_route_weights_extra_fwd; the same two fp32 inputs, either null).
 * Their gradients equal d_scores (each is added to the logit as it is).
 */
int mrsa_route_weights_extra_bwd(const void* scores, const int32_t* indices,
                                 const float* prior_bias, const float* local_lse,
                                 const void* grad_remote, const void* grad_local,
                                 const float* grad_gate_logit, int64_t batch, int64_t seq_len,
                                 int64_t chunks, int64_t kv_heads, int64_t groups, int64_t topk,
                                 float temperature, const float* gate_offset,
                                 const float* gate_scale, const float* value_bonus,
                                 const float* selected_gumbel, float* d_scores, float* d_bias,
                                 float* d_local_lse, float* d_gate, void* stream);

/*
 * Re-lays K and V out as per-chunk fragments: for each 64-key chunk, the
 * register images of the 32 matrix-core operand loads of the routed
 * attention (16x16x32 bf16 products; lane l = 16 grp + j, elements e = 0..7):
 *   f[512 i + 8 l + e]        = K[key 16 mt + j][dim 32 ks + 8 grp + e],  i = 4 mt + ks
 *   f[8192 + 512 i + 8 l + e] = V[key 32 ks + 16 (e >> 2) + 4 grp + (e & 3)][dim 16 nt + j],
 *                               i = 2 nt + ks
 * so every operand load is one contiguous 1 KB read.  Keys past seq_len are zero.
 *   k, v: bf16 [batch, seq_len, kv_heads, head_dim], 16-byte aligned; v may be
 *         NULL (the V part is then zero: enough for the candidate token scores)
 *   kv_frags (out): bf16 [batch, kv_heads, ceil(seq_len / 64), 16384], 16-byte aligned
 * Limits: head_dim == 128.
 * No reference counterpart: internal layout step of the two attention ops.
 */
int64_t mrsa_kv_fragments_bytes(int64_t batch, int64_t seq_len, int64_t kv_heads,
                                int64_t head_dim);
int mrsa_kv_fragments(const void* k, const void* v, int64_t batch, int64_t seq_len,
                      int64_t kv_heads, int64_t head_dim, void* kv_frags, void* stream);

/*
 * Rewrites the fragments of the given rows of k and v after the rows were
 * replaced (LayerKVCache.replace, dream_dllm_hils/fastdllm_cache.py:94-125).
 * positions: int64 [count]; entries outside [0, seq_len) are ignored.
 */
int mrsa_kv_fragments_rows(const void* k, const void* v, int64_t batch, int64_t seq_len,
                           int64_t kv_heads, int64_t head_dim, const int64_t* positions,
                           int64_t count, void* kv_frags, void* stream);

/*
 * The row writes of LayerKVCache.replace (dream_dllm_hils/fastdllm_cache.py:
 * 126-127, key.index_copy_(1, positions, k_rows) and the same for value) and
 * the fragment rewrite of those rows (mrsa_kv_fragments_rows) in one launch.
 *   k_rows, v_rows: bf16 [batch, count, kv_heads, head_dim]
 *   positions: int64 [count]; entries outside [0, seq_len) are ignored
 *   key, value (in/out): bf16 [batch, seq_len, kv_heads, head_dim]
 *   kv_frags (in/out, optional): as in mrsa_kv_fragments
 * Limits: head_dim == 128.  Positions must be unique (a duplicate leaves
 * either row, as index_copy_ does).
 */
/*
 * Up to 8 device-to-device buffer copies in one launch (src[i] -> dst[i],
 * bytes[i] bytes; host arrays of count entries).  Every pointer and size
 * must be a multiple of 8 bytes (MRSA_ERR_UNSUPPORTED otherwise).  For
 * callers that refill the input buffers of a captured step (the cached block
 * step's query, routing query, K/V rows and positions) each call.  No
 * reference counterpart: the reference runs its cached step eagerly.
 */
int mrsa_copy_buffers(int32_t count, const void* const* src, void* const* dst,
                      const int64_t* bytes, void* stream);

int mrsa_kv_replace_rows(const void* k_rows, const void* v_rows, const int64_t* positions,
                         int64_t count, int64_t batch, int64_t seq_len, int64_t kv_heads,
                         int64_t head_dim, void* key, void* value, void* kv_frags, void* stream);

/*
 * Q fragments: per (batch, KV head, query) the 2 KB register image of the
 * routed attention's Q^T operand for the query's q_heads / kv_heads head
 * columns,
 *   q_frags[((b * kv_heads + h) * seq_len + i) * 1024 + 256 ks + 64 grp + 8 g + e]
 *     = q[b, i, h * G + g, 32 ks + 8 grp + e]   (g < G; zeros for G <= g < 8),
 * so that the routed kernel reads the 8 head columns of a query's lane group
 * as one 128-byte line instead of eight 64-byte pieces.
 *   q: bf16 [batch, seq_len, q_heads, head_dim], 16-byte aligned
 *   q_frags (out): bf16 [batch, kv_heads, seq_len, 1024], 16-byte aligned
 * Limits: head_dim == 128, q_heads / kv_heads <= 8.
 * No reference counterpart: internal layout step of the routed attention
 * (mrsa_local_attention_qf_fwd writes the same images as a by-product).
 */
int64_t mrsa_q_fragments_bytes(int64_t batch, int64_t seq_len, int64_t kv_heads,
                               int64_t head_dim);
int mrsa_q_fragments(const void* q, int64_t batch, int64_t seq_len, int64_t q_heads,
                     int64_t kv_heads, int64_t head_dim, void* q_frags, void* stream);

/*
 * mrsa_kv_fragments and mrsa_chunk_attn_pool_gqa_strided_fwd (fused
 * semantics) in one pass over the keys: each chunk's K and V rows are read
 * once, laid out as fragments and K pooled against the chunk's landmark
 * query rows.  Same outputs as the two calls, bit for bit.
 *   k, v, kv_frags as in mrsa_kv_fragments (v required)
 *   mu_q, mu_row_stride, key_valid, sm_scale, bias_scale, landmark_keys,
 *   entropy, prior_bias as in mrsa_chunk_attn_pool_gqa_strided_fwd with
 *   batch_chunks = batch * seq_len / 64 and chunk_size 64
 * Limits: head_dim == 128, 2 <= groups <= 16 (groups == 1 pools with the
 * dense torch semantics: use the two calls), seq_len % 64 == 0.
 * No reference counterpart beyond the two it combines (the pool replaces
 * chunk_attn_pool_gqa, ops/chunk_attn_pool_gqa_tilelang.py:425-448).
 */
int mrsa_kv_fragments_pool_fwd(const void* k, const void* v, const void* mu_q,
                               int64_t mu_row_stride, const uint8_t* key_valid, int64_t batch,
                               int64_t seq_len, int64_t kv_heads, int64_t groups,
                               int64_t head_dim, float sm_scale, const float* bias_scale,
                               void* kv_frags, void* landmark_keys, float* entropy,
                               float* prior_bias, void* stream);

/*
 * Bidirectional sliding-window GQA attention with natural-log LSE.
 * Replaces the flash-attn window call behind bidir_local_attention and
 * cached_local_attention (dream_dllm_hils/local_attention.py:67-200):
 * key j is visible to the query at position p iff |p - j| <= window.
 * Keys that fail key_valid, and when inert_chunk > 0 the slots with
 * (j + 1) % inert_chunk == 0, take zero K and zero V (local_attention.py:35-54):
 * they stay in the softmax denominator with logit 0 and add nothing to the
 * output.
 *   q: bf16 [batch, q_len, q_heads, head_dim]
 *   kv_frags: output of mrsa_kv_fragments for the keys and values (kv_len rows)
 *   key_valid: optional bool [batch, kv_len];  query_positions: optional int64 [q_len]
 *   (NULL = query row i sits at position i)
 *   out: bf16 [batch, q_len, q_heads, head_dim];  lse: fp32 [batch, q_len, q_heads]
 *   sm_scale: finite and > 0 (MRSA_ERR_INVALID_ARGUMENT otherwise)
 * Limits: head_dim == 128, q_heads / kv_heads <= 8, kv_len < 8388608.
 */
int mrsa_local_attention_fwd(const void* q, const void* kv_frags,
                             const uint8_t* key_valid, const int64_t* query_positions,
                             int64_t batch, int64_t q_len, int64_t kv_len, int64_t q_heads,
                             int64_t kv_heads, int64_t head_dim, int64_t window,
                             int64_t inert_chunk, float sm_scale, void* out, float* lse,
                             void* stream);

/*
 * mrsa_local_attention_fwd that also writes q_frags (bf16 [batch, kv_heads,
 * q_len, 1024], 16-byte aligned), exactly what mrsa_q_fragments writes for
 * q, from the Q operands its waves load anyway.  No reference counterpart: it
 * serves the route-layer composition (the routed attention then reads Q as
 * whole cache lines).  Limits as mrsa_local_attention_fwd.
 */
int mrsa_local_attention_qf_fwd(const void* q, const void* kv_frags,
                                const uint8_t* key_valid, const int64_t* query_positions,
                                int64_t batch, int64_t q_len, int64_t kv_len, int64_t q_heads,
                                int64_t kv_heads, int64_t head_dim, int64_t window,
                                int64_t inert_chunk, float sm_scale, void* q_frags, void* out,
                                float* lse, void* stream);

/*
 * Backward of mrsa_local_attention_fwd for full sequences (q_len == kv_len,
 * no query positions): the gradient flash-attn's flash_attn_func gives
 * bidir_local_attention (dream_dllm_hils/local_attention.py:67-107), with
 * _apply_key_valid's masking (:50-54): keys that fail key_valid and, when
 * inert_chunk > 0, the landmark slots carry k' = v' = 0 (in the softmax with
 * logit 0), so their grad_k / grad_v are 0.
 *   q, grad_out, out: bf16 [batch, seq_len, q_heads, 128] (out and lse as the
 *                     forward returned them); k, v: bf16 [batch, seq_len,
 *                     kv_heads, 128]; lse: fp32 [batch, seq_len, q_heads]
 *   window, inert_chunk, sm_scale, key_valid: as the forward's
 *   grad_q: fp32 [batch, seq_len, q_heads, 128]; grad_k, grad_v: fp32
 *           [batch, seq_len, kv_heads, 128] (every element written)
 *   workspace: 256-byte aligned, mrsa_local_attention_bwd_workspace_bytes
 *           bytes (the operand images of K, V, Q and dO, and per-row lse / D)
 * The LSE output carries no gradient (flash-attn's autograd drops it).
 * Rounding points as flash-attn's: P and dS are bf16 matrix operands, every
 * sum is fp32.  Requirements: head_dim 128, 16-byte aligned tensors.
 */
int64_t mrsa_local_attention_bwd_workspace_bytes(int64_t batch, int64_t seq_len,
                                                 int64_t q_heads, int64_t kv_heads);
int mrsa_local_attention_bwd(const void* q, const void* k, const void* v,
                             const uint8_t* key_valid, const void* out, const float* lse,
                             const void* grad_out, int64_t batch, int64_t seq_len,
                             int64_t q_heads, int64_t kv_heads, int64_t head_dim, int64_t window,
                             int64_t inert_chunk, float sm_scale, float* grad_q, float* grad_k,
                             float* grad_v, void* workspace, int64_t workspace_bytes,
                             void* stream);

/*
 * The same window attention for short query blocks (cached_local_attention,
 * dream_dllm_hils/local_attention.py:147-200, at the cached block step):
 * each 32-query block's key tiles are split over `parts` workgroups (1..64)
 * whose unnormalised partial outputs and (max, sum) pairs, kept in the
 * caller's fp32 workspace of mrsa_local_attention_workspace_bytes() bytes
 * (16-byte aligned), a second kernel merges.  parts == 1 is
 * mrsa_local_attention_fwd (workspace unused).  batch * parts <= 65535.
 */
int64_t mrsa_local_attention_workspace_bytes(int64_t batch, int64_t q_len, int64_t q_heads,
                                             int64_t parts);
int mrsa_local_attention_split_fwd(const void* q, const void* kv_frags,
                                   const uint8_t* key_valid, const int64_t* query_positions,
                                   int64_t batch, int64_t q_len, int64_t kv_len, int64_t q_heads,
                                   int64_t kv_heads, int64_t head_dim, int64_t window,
                                   int64_t inert_chunk, float sm_scale, int64_t parts,
                                   void* workspace, int64_t workspace_bytes, void* out,
                                   float* lse, void* stream);

/*
 * Routed chunk attention: for each query head, the sum over its routed chunks
 * of weight * softmax over that chunk's keys (each chunk normalised on its
 * own), times V.  Replaces HiLS_block_M_head
 * (ops/hils_fwd_bwd_head.py:1113-1150, forward kernel :190-570) as called by
 * selected_attention_g7 / selected_attention_g7_cached
 * (dream_dllm_hils/routing.py:305-472); the formula is the reference's
 * test_hils_non_power_two_topk.py:122-138.
 *   q: bf16 [batch, q_len, q_heads, head_dim]
 *   kv_frags: output of mrsa_kv_fragments for the cache's k and v (kv_len rows)
 *   weights: bf16 [batch, q_len, q_heads, topk]
 *   indices: int32 [batch, q_len, kv_heads, topk] (chunk ids; entries < 0 or
 *            >= kv_len / chunk_size are skipped)
 *   key_valid: optional bool [batch, kv_len]
 *   out: bf16 [batch, q_len, q_heads, head_dim]
 *   sm_scale: finite and > 0 (MRSA_ERR_INVALID_ARGUMENT otherwise)
 * Limits: chunk_size == 64, head_dim == 128, q_heads / kv_heads <= 8, topk <= 64,
 * kv_len < 8388608.
 */
int mrsa_selected_attention_fwd(const void* q, const void* kv_frags,
                                const void* weights, const int32_t* indices,
                                const uint8_t* key_valid, int64_t batch, int64_t q_len,
                                int64_t kv_len, int64_t q_heads, int64_t kv_heads,
                                int64_t head_dim, int64_t topk, int64_t chunk_size,
                                int mask_last_token, float sm_scale, void* out, void* stream);

/*
 * The same routed chunk attention for short query blocks, the shape of the
 * Fast-dLLM cached block step (selected_attention_g7_cached called at
 * dream_dllm_hils/fastdllm_attention.py:363): each (query tile, KV head)
 * walk is split over `parts` workgroups, which write fp32 partial outputs
 * that a second kernel sums into `out`.  Arguments as
 * mrsa_selected_attention_fwd, plus:
 *   parts: 1..64 (1: exactly mrsa_selected_attention_fwd; partial unused)
 *   partial: fp32 workspace of parts * batch * q_len * q_heads * 128 floats,
 *            16-byte aligned, provided by the caller (no allocation here)
 * batch * parts must not exceed 65535.
 */
int mrsa_selected_attention_split_fwd(const void* q, const void* kv_frags,
                                      const void* weights, const int32_t* indices,
                                      const uint8_t* key_valid, int64_t batch, int64_t q_len,
                                      int64_t kv_len, int64_t q_heads, int64_t kv_heads,
                                      int64_t head_dim, int64_t topk, int64_t chunk_size,
                                      int mask_last_token, float sm_scale, int64_t parts,
                                      float* partial, void* out, void* stream);

/*
 * Routed chunk attention with the token keep mask of the remote-token
 * refinement: HiLS_block_M_head / selected_attention_g7[_cached] called with
 * token_keep (ops/hils_fwd_bwd_head.py:457-507, the TokenKeep[b, q, h, slot,
 * key] == 0 exclusion; dream_dllm_hils/attention.py:1729-1769).  Arguments as
 * mrsa_selected_attention_split_fwd (parts == 1: partial unused), plus
 *   token_keep: int8 [batch, q_len, kv_heads, topk, chunk_size], nonzero = keep
 * A chunk listed twice for one query counts once with the summed weights and
 * the keep row of its first slot.
 */
int mrsa_selected_attention_keep_fwd(const void* q, const void* kv_frags,
                                     const void* weights, const int32_t* indices,
                                     const uint8_t* key_valid, const int8_t* token_keep,
                                     int64_t batch, int64_t q_len, int64_t kv_len,
                                     int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                                     int64_t topk, int64_t chunk_size, int mask_last_token,
                                     float sm_scale, int64_t parts, float* partial, void* out,
                                     void* stream);

/*
 * Backward of the routed chunk attention: replaces the backward kernel of
 * HiLS_block_M_head (ops/hils_fwd_bwd_head.py:573-910, called from
 * _hils_block_M_attention_inverse.backward, :1050-1098).  Each listed
 * (query, chunk) recomputes its chunk softmax; with the reference's rounding
 * points P = bf16(2^(s c - lse)), di = sum P dP, dS = bf16(scale w P (dP - di)):
 *   grad_q += sum dS K              fp32 [batch, q_len, q_heads, head_dim] (added:
 *                                   zero it first); the chunk-major pass stores
 *                                   each (query, head, slot)'s bf16 dS and the
 *                                   forward kernel's walk adds dS K into the rows
 *                                   of the queries it owns (a slot that repeats
 *                                   an earlier chunk of its list adds with atomics)
 *   grad_k += dS^T Q, grad_v += P^T bf16(w dO)
 *                                   fp32 [batch, kv_len, kv_heads, head_dim]
 *                                   (zero them first: a chunk no query routes to
 *                                   is not written)
 *   grad_weights = di               bf16 [batch, q_len, q_heads, topk] (slots past
 *                                   the list's end or out of range are not
 *                                   written: zero it first)
 * Arguments as mrsa_selected_attention_keep_fwd (token_keep may be null), plus
 *   grad_out:     bf16 [batch, q_len, q_heads, head_dim] upstream gradient
 *   kv_frags_bwd: mrsa_kv_fragments(v, k) (the roles of k and v swapped: V as
 *                 keys x dims, K^T as dims x keys)
 *   workspace:    256-byte aligned, mrsa_selected_attention_bwd_workspace_bytes
 *                 bytes: the per-chunk lists of (query, slot) pairs from which
 *                 grad_k / grad_v are computed chunk by chunk (one write per
 *                 chunk; chunks with more than 1024 pairs add their segments'
 *                 sums with atomics, so their last bits depend on timing), and
 *                 the dS records (128 bytes per (query, head, slot)).
 * Requirements: head_dim 128, chunk_size 64, q_heads / kv_heads <= 8, topk <= 64,
 * kv_len / 64 <= 8192, q_len < 2^24.
 */
int64_t mrsa_selected_attention_bwd_workspace_bytes(int64_t batch, int64_t q_len,
                                                    int64_t kv_len, int64_t q_heads,
                                                    int64_t kv_heads, int64_t topk);
int mrsa_selected_attention_bwd(const void* q, const void* grad_out, const void* kv_frags,
                                const void* kv_frags_bwd, const void* weights,
                                const int32_t* indices, const uint8_t* key_valid,
                                const int8_t* token_keep, int64_t batch, int64_t q_len,
                                int64_t kv_len, int64_t q_heads, int64_t kv_heads,
                                int64_t head_dim, int64_t topk, int64_t chunk_size,
                                int mask_last_token, float sm_scale, float* grad_q,
                                float* grad_k, float* grad_v, void* grad_weights,
                                void* workspace, int64_t workspace_bytes, void* stream);

/*
 * mrsa_selected_attention_bwd with ALiBi slopes: the backward of
 * mrsa_selected_attention_alibi_fwd (ops/hils_fwd_bwd_head.py:755-760, the
 * bias term of the reference's backward kernel).  slope: fp32 [q_heads],
 * required.  No gradient flows to the slopes (the reference's backward
 * returns none for them).
 */
int mrsa_selected_attention_alibi_bwd(const void* q, const void* grad_out, const void* kv_frags,
                                      const void* kv_frags_bwd, const void* weights,
                                      const int32_t* indices, const uint8_t* key_valid,
                                      const int8_t* token_keep, const float* slope,
                                      int64_t batch, int64_t q_len, int64_t kv_len,
                                      int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                                      int64_t topk, int64_t chunk_size, int mask_last_token,
                                      float sm_scale, float* grad_q, float* grad_k,
                                      float* grad_v, void* grad_weights, void* workspace,
                                      int64_t workspace_bytes, void* stream);

/*
 * Routed chunk attention with the output fusion folded in: the result is
 * fuse_hils_outputs(remote, local_output, local_weight)
 * (ops/hils_bidir_output_fusion_tilelang.py:138-148) of the routed output
 * `remote` that mrsa_selected_attention_keep_fwd would write, bit for bit,
 * without writing or re-reading `remote`.  It has no counterpart in the
 * reference, which runs the two ops in sequence (dream_dllm_hils/
 * attention.py:1770-1774); it serves the route-layer composition.
 * Arguments as mrsa_selected_attention_keep_fwd (token_keep may be null),
 * plus
 *   local_output: bf16 [batch, q_len, q_heads, head_dim], 8-byte aligned
 *   local_weight: bf16 [batch, q_len, q_heads]
 */
int mrsa_selected_attention_fused_fwd(const void* q, const void* kv_frags,
                                      const void* weights, const int32_t* indices,
                                      const uint8_t* key_valid, const int8_t* token_keep,
                                      const void* local_output, const void* local_weight,
                                      int64_t batch, int64_t q_len, int64_t kv_len,
                                      int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                                      int64_t topk, int64_t chunk_size, int mask_last_token,
                                      float sm_scale, int64_t parts, float* partial, void* out,
                                      void* stream);

/*
 * mrsa_selected_attention_fused_fwd reading the queries from q_frags
 * (mrsa_q_fragments(q) or the by-product of mrsa_local_attention_qf_fwd)
 * instead of q: same result.  No reference counterpart; it serves the
 * route-layer composition.  q is still passed (shape checks only).
 */
int mrsa_selected_attention_fused_qf_fwd(const void* q, const void* q_frags,
                                         const void* kv_frags, const void* weights,
                                         const int32_t* indices, const uint8_t* key_valid,
                                         const int8_t* token_keep, const void* local_output,
                                         const void* local_weight, int64_t batch, int64_t q_len,
                                         int64_t kv_len, int64_t q_heads, int64_t kv_heads,
                                         int64_t head_dim, int64_t topk, int64_t chunk_size,
                                         int mask_last_token, float sm_scale, int64_t parts,
                                         float* partial, void* out, void* stream);

/*
 * Routed chunk attention with every option of the entry points above in one
 * call, plus `flags`:
 *   MRSA_ROUTED_FIXED_ORDER  each output row adds its chunk terms in
 *                            ascending chunk order (per-query tickets instead
 *                            of the row lock), so two launches -- and a
 *                            captured graph and the eager call -- give the
 *                            same bits.  The reference's forward accumulates
 *                            each query block in a fixed order too, and it
 *                            replaced a kernel for being nondeterministic
 *                            (dream_dllm_hils/routing.py:133-134).
 * q_frags may be null (q is read); with q_frags the fusion operands are
 * required.  token_keep, local_output / local_weight and partial as in
 * mrsa_selected_attention_fused_fwd.  Unknown flag bits:
 * MRSA_ERR_INVALID_ARGUMENT.  No reference counterpart beyond the ones of
 * the options it combines.
 */
#define MRSA_ROUTED_FIXED_ORDER 1
int mrsa_selected_attention_ex_fwd(const void* q, const void* q_frags, const void* kv_frags,
                                   const void* weights, const int32_t* indices,
                                   const uint8_t* key_valid, const int8_t* token_keep,
                                   const void* local_output, const void* local_weight,
                                   int64_t batch, int64_t q_len, int64_t kv_len, int64_t q_heads,
                                   int64_t kv_heads, int64_t head_dim, int64_t topk,
                                   int64_t chunk_size, int mask_last_token, float sm_scale,
                                   int64_t parts, float* partial, int flags, void* out,
                                   void* stream);

/*
 * mrsa_selected_attention_ex_fwd with ALiBi slopes: HiLS_block_M_head's
 * `slope` argument (ops/hils_fwd_bwd_head.py:1113-1150; hils_torch_ref
 * :68-76 and the forward kernel :445-451).  Before the scale, the raw logit
 * of key s of a chunk (s = 0..63) gets -slope[head] * max(0, 62 - s):
 *   softmax_s((q . k_s - slope[head] max(0, 62 - s)) * sm_scale)
 * slope: fp32 [q_heads] on the device, required; every other argument as in
 * mrsa_selected_attention_ex_fwd.
 */
int mrsa_selected_attention_alibi_fwd(const void* q, const void* q_frags, const void* kv_frags,
                                      const void* weights, const int32_t* indices,
                                      const uint8_t* key_valid, const int8_t* token_keep,
                                      const void* local_output, const void* local_weight,
                                      const float* slope, int64_t batch, int64_t q_len,
                                      int64_t kv_len, int64_t q_heads, int64_t kv_heads,
                                      int64_t head_dim, int64_t topk, int64_t chunk_size,
                                      int mask_last_token, float sm_scale, int64_t parts,
                                      float* partial, int flags, void* out, void* stream);

/*
 * Routed-attention lock status.  It has no counterpart in the reference
 * (whose kernels take no lock); it makes the bounded lock wait of the routed
 * attention kernels (mrsa_selected_attention_*) observable.  A tile whose
 * wait for its owners' rows runs out (mrsa_set_routed_lock_spin_limit tries,
 * 65536 by default) is deferred: the workgroup replays it onto the rows after
 * its walk, when no wave holds them, so the output stays exact.  The count
 * only reports that slow path.  It is one word per device, shared by every
 * stream and caller: reading it waits for all of the device's queued work
 * (hipDeviceSynchronize, so never under graph capture), stores the count
 * since the last reset in *count and clears it when `reset` is nonzero.
 */
int mrsa_routed_lock_giveups(uint64_t* count, int reset);

/*
 * Test hook: the lock tries of the routed-attention kernels before a tile is
 * deferred (process-wide; read at each launch, so a captured graph keeps the
 * value of its capture).  limit <= 0 defers every tile.  Default 65536.
 * No reference counterpart.
 */
int mrsa_set_routed_lock_spin_limit(int limit);

/*
 * Global token keep: select_global_token_keep
 * (dream_dllm_hils/token_refinement.py:112-148) without training noise.  In
 * each of `rows` rows of n fp32 scores the min(token_budget, n) largest are
 * kept (1) when finite, others 0; ties at the threshold go to the lower index
 * (the reference's torch.topk(sorted=False) leaves their order to the device).
 *   scores: fp32 [rows, n] (the [B, L, Hkv, K, S] candidate scores, n = K * S)
 *   keep (out): uint8 [rows, n]
 * Limits: n <= 4096, token_budget > 0.
 */
int mrsa_token_keep_fwd(const float* scores, int64_t rows, int64_t n, int64_t token_budget,
                        uint8_t* keep, void* stream);

/*
 * Entropy-adaptive token keep: replaces the selection of
 * refine_remote_tokens_entropy_g7 (dream_dllm_hils/token_refinement.py:396-438)
 * -- gather_selected_chunk_entropy (:244-284), allocate_entropy_token_budget
 * (:150-241) and select_entropy_adaptive_token_keep (:287-333) -- without
 * training noise.  Per (batch, query, KV head) row of topk slots:
 *   capacity[k]   finite scores of slot k (or given)
 *   entropy_k     the group mean of entropy at the slot's chunk (clamped to
 *                 [0, chunks - 1]; 0 for a negative index), or given
 *   allocation    min(sum capacity, token_budget) slots apportioned by
 *                 support exp(clamp(entropy, 0, ln token_budget)): baseline
 *                 min(capacity, min_tokens_per_chunk), then topk + 1 rounds
 *                 of capped largest remainder (ties to the lower slot)
 *   keep          per slot, its allocation's largest finite scores (ties to
 *                 the lower key)
 *   scores:           fp32 [batch, seq_len, kv_heads, topk, chunk_size] or NULL
 *   capacity:         int64 [batch, seq_len, kv_heads, topk] or NULL (count
 *                     finite scores; one of the two must be given)
 *   selected_entropy: fp32 [batch, seq_len, kv_heads, topk] or NULL, then
 *   entropy:          fp32 [batch, chunks, kv_heads, groups] and
 *   indices:          int32 [batch, seq_len, kv_heads, topk]
 *   keep (out):       bytes [batch, seq_len, kv_heads, topk, chunk_size] 0/1,
 *                     or NULL (allocation only)
 *   allocation (out): int64 [batch, seq_len, kv_heads, topk]
 * Requirements: topk <= 64, chunk_size <= 64, token_budget >= topk *
 * min_tokens_per_chunk.  The support sum is exact before its rounding to
 * fp32 (order-independent).
 */
int mrsa_token_keep_entropy_fwd(const float* scores, const int64_t* capacity,
                                const float* selected_entropy, const float* entropy,
                                const int32_t* indices, int64_t batch, int64_t seq_len,
                                int64_t kv_heads, int64_t groups, int64_t chunks, int64_t topk,
                                int64_t chunk_size, int64_t token_budget,
                                int64_t min_tokens_per_chunk, uint8_t* keep,
                                int64_t* allocation, void* stream);

/*
 * gather_selected_chunk_entropy (dream_dllm_hils/token_refinement.py:244-284):
 * out[b, l, h, k] = mean over g of entropy[b, clamp(idx, 0, chunks - 1), h, g],
 * 0 where idx < 0.
 *   entropy: fp32 [batch, chunks, kv_heads, groups]
 *   indices: int32 [batch, seq_len, kv_heads, topk]
 *   out:     fp32 [batch, seq_len, kv_heads, topk]
 */
int mrsa_gather_selected_chunk_entropy(const float* entropy, const int32_t* indices,
                                       int64_t batch, int64_t seq_len, int64_t chunks,
                                       int64_t kv_heads, int64_t groups, int64_t topk, float* out,
                                       void* stream);

/*
 * Per-token candidate scores inside routed chunks: max over the query group of
 * q.k * sm_scale; -inf for the landmark slot, invalid keys and -1 chunks.
 * Replaces candidate_token_scores_gqa (ops/hils_token_score_gqa_tilelang.py:174-208).
 *   kv_frags: output of mrsa_kv_fragments (the V part is not read)
 *   scores (out): fp32 [batch, q_len, kv_heads, topk, chunk_size]
 * Limits: as mrsa_selected_attention_fwd.
 */
int mrsa_candidate_token_scores_fwd(const void* q, const void* kv_frags, const int32_t* indices,
                                    const uint8_t* key_valid, int64_t batch, int64_t q_len,
                                    int64_t kv_len, int64_t q_heads, int64_t kv_heads,
                                    int64_t head_dim, int64_t topk, int64_t chunk_size,
                                    float sm_scale, float* scores, void* stream);

/*
 * Self-test of the matrix-core lane layout every kernel above relies on:
 * c = a @ b for a = bf16 [16, 32], b = bf16 [32, 16], c = fp32 [16, 16],
 * computed with one v_mfma_f32_16x16x32_bf16.  No reference counterpart.
 */
int mrsa_selftest_mfma_layout(const void* a, const void* b, float* c, void* stream);

/*
 * Decoder-layer glue of the Dream-7B-shaped forward (the layers around the
 * attention path: dream_dllm_hils/fastdllm_v1.py:375-403).
 *
 * Residual add + RMSNorm (Qwen2RMSNorm as the decoder layer applies it):
 *   sum = bf16(x + residual) (when residual != NULL; written to sum_out when given)
 *   out = bf16(weight * bf16(sum * rsqrt(mean(sum^2) + eps)))
 *   x, residual, sum_out, out: bf16 [rows, hidden]; weight: bf16 [hidden]
 * Limits: hidden % 8 == 0, hidden <= 8192, 16-byte aligned rows.
 */
int mrsa_add_rms_norm_fwd(const void* x, const void* residual, const void* weight, int64_t rows,
                          int64_t hidden, float eps, void* sum_out, void* out, void* stream);

/*
 * Rotary embedding of the fused QKV projection, plus the Q-Cal routing query.
 * Replaces apply_rotary_pos_emb (dream_dllm_hils/attention.py:41-52) in the
 * fp32 form of ops/rope_tilelang_fp32.py:19-94, and _finish_calibrated_query
 * (attention.py:477-502; qcal.py:22-26) when qcal_delta != NULL.
 *   qkv: bf16 [tokens, (q_heads + 2 kv_heads) * 128] (q heads, k heads, v heads)
 *   cos_table, sin_table: fp32 [tokens, 64] (attention factor folded in)
 *   qcal_delta: bf16 [tokens, q_heads, 128] or NULL; qcal_norm_weight: fp32 [128]
 *   q (out): bf16 [tokens, q_heads, 128]; k, v (out): bf16 [tokens, kv_heads, 128]
 *   route_q (out, with qcal_delta): rope(rms_norm(q_unrotated + delta) * weight)
 */
int mrsa_rope_qkv_fwd(const void* qkv, const float* cos_table, const float* sin_table,
                      const void* qcal_delta, const float* qcal_norm_weight, float qcal_eps,
                      int64_t tokens, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                      void* q, void* k, void* v, void* route_q, void* stream);

/*
 * SwiGLU of the fused gate/up projection (Qwen2 MLP act_fn(gate) * up):
 *   gate_up: bf16 [rows, 2 * intermediate] (gate columns first)
 *   out:     bf16 [rows, intermediate] = bf16(bf16(silu(gate)) * up)
 */
int mrsa_swiglu_fwd(const void* gate_up, int64_t rows, int64_t intermediate, void* out,
                    void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MRSA_H */
