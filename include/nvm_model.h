/*
 * C ABI of the fused element-wise steps of the Qwen3 layer (the model port's
 * glue around the matrix products), in the same library and with the same
 * conventions as nvm_moe.h: device pointers, work on `stream`, no device
 * allocation, NVM_OK or a negative NVM_ERR_* status (message in
 * nvm_last_error()).  Activations are f16/bf16 (`dtype` as in nvm_moe.h);
 * arithmetic is float32, rounded to the activation dtype where the reference
 * model materialises an activation tensor.
 */
#ifndef NVM_MODEL_H
#define NVM_MODEL_H

#include "nvm_moe.h"

#ifdef __cplusplus
extern "C" {
#endif

/*
 * Residual add and RMSNorm: h_out = rnd(h + r) (skipped when r is NULL, then
 * h_out may be NULL), x_out = rnd(rms_norm(h_out) * w) with rms_norm(v) =
 * v / sqrt(mean(v^2) + eps) in float32.  Replaces `h = x + r` and
 * `RMSNorm.__call__` (mx.fast.rms_norm) of models/qwen3.py:244-252 and
 * layers/layernorm.py:4-14.  h, r, h_out, x_out [T, H]; w [H].  h_out may
 * alias h.  H at most 8192, a multiple of 2.
 */
int nvm_residual_rms_norm(const void *h, const void *r, const void *w, int64_t T, int64_t H,
                          float eps, int dtype, void *h_out, void *x_out, nvm_stream_t stream);

/*
 * The attention block between the q/k/v projections and the attention
 * (models/qwen3.py:103-133): per head, RMSNorm of q and k with q_norm/k_norm
 * (float32, rounded), RoPE of both (non-traditional halves, rotation by the
 * float32 tables cos/sin[position][D/2], rounded; layers/rotary_embedding.py),
 * then k and v stored in the layer's pages and q handed to the attention in
 * float32.
 *   qkv          [T, (Hq + 2 Hkv) * D] act: q heads, then k heads, then v heads
 *   positions    [T] int32; cos, sin [max_pos, D/2] float32
 *   page_ids, slots [T] int32: where token t's k/v go
 *   key_pages, value_pages [P, Hkv, page_size, D] act
 *   q_out        [T, Hq, D] float32
 *   k_out, v_out [T, Hkv, D] float32, or NULL (the rounded k and v, for a
 *                dense prefill attention)
 * D a multiple of 4, at most 128.  Page ids outside [0, P) and slots outside
 * [0, page_size) are not stored.
 */
int nvm_qk_norm_rope_store(const void *qkv, int64_t T, int Hq, int Hkv, int64_t D,
                           const void *q_norm_w, const void *k_norm_w, float eps,
                           const int32_t *positions, const float *cos, const float *sin,
                           int64_t max_pos, const int32_t *page_ids, const int32_t *slots,
                           void *key_pages, void *value_pages, int64_t P, int64_t page_size,
                           int dtype, float *q_out, float *k_out, float *v_out,
                           nvm_stream_t stream);

/*
 * The MoE block with its combine fused into the residual add and RMSNorm
 * that follow it in the model (models/qwen3.py:249-252 around
 * layers/moe.py:69-86): the stages of nvm_moe_forward, then per token
 * y = rnd(sum_j rnd(down_j * score_j)) in slot order (bit-identical to
 * nvm_moe_forward's y), h_out = rnd(h + y), x_out = rnd(rms_norm(h_out) * w).
 * Arguments as nvm_moe_forward, with h [T, H], norm_w [H], eps, h_out and
 * x_out [T, H] in place of y / ids_out / scores_out (16-byte aligned).  H a
 * multiple of 8, at most 8192.  Workspace: nvm_moe_workspace_size.
 */
int nvm_moe_forward_residual_norm(const void *x, int64_t T, int64_t H, int64_t I, int64_t E,
                                  int top_k, int norm_topk_prob, int group_size, int bits,
                                  int dtype, const uint32_t *wr, const void *sr, const void *br,
                                  const uint32_t *wg, const void *sg, const void *bg,
                                  const uint32_t *wu, const void *su, const void *bu,
                                  const uint32_t *wd, const void *sd, const void *bd,
                                  const void *h, const void *norm_w, float eps, void *h_out,
                                  void *x_out, int regime, void *workspace,
                                  size_t workspace_bytes, nvm_stream_t stream);

/*
 * Embedding lookup of a 4-bit affine-quantised table (MLX layout, as the
 * expert weights): out[t] = rnd(q * s + b) over row tokens[t], the value
 * computed in float32 and rounded once to the activation dtype.  Replaces
 * `QuantizedEmbedding.__call__` (layers/embed_head.py:21-36: mx.dequantize of
 * the gathered rows).  tokens [T] int32; wq [V, D/8] uint32; scales, biases
 * [V, D/group] act; out [T, D] act (16-byte aligned).  Ids outside [0, V)
 * give zero rows (the reference reads out of bounds there).
 */
int nvm_embedding(const int32_t *tokens, int64_t T, const uint32_t *wq, const void *scales,
                  const void *biases, int64_t V, int64_t D, int group_size, int bits, int dtype,
                  void *out, nvm_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* NVM_MODEL_H */
