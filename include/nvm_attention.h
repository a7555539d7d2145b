/*
 * C ABI of paged attention over a paged KV cache (the step before each MoE
 * block in decode), in the same library and with the same conventions as
 * nvm_moe.h: device pointers, work enqueued on `stream`, no host
 * synchronisation, no device allocation (callers pass outputs and the
 * workspace), NVM_OK or a negative NVM_ERR_* status with the message in
 * nvm_last_error().
 */
#ifndef NVM_ATTENTION_H
#define NVM_ATTENTION_H

#include "nvm_moe.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Storage type of the key and value pages.  Int8 pages carry one float32
 * scale per (page, kv head, slot): the value is code * scale. */
enum nvm_kv_dtype { NVM_KV_F16 = 0, NVM_KV_BF16 = 1, NVM_KV_F32 = 2, NVM_KV_I8 = 3 };

/*
 * out = softmax(q . paged_key^T * scale) . paged_value, per query row.
 * Replaces `metal.paged_attention(query, key_pages, value_pages, block_table,
 * context_lens, scale, is_causal, num_kv_heads, num_heads)`
 * (metal/bindings.cpp:50-66; op metal/src/paged_attention.cpp:17-68, CPU loop
 * :122-296, GPU dispatch :413-574) and `metal.paged_attention_int8_decode`
 * (bindings.cpp:68-80; op :70-120, CPU loop :298-410), which
 * `paged_attention` calls (layers/attention.py:154-230).
 *
 *   q            [N = B * num_heads, L, D] float32 (row n: batch n / num_heads,
 *                query head n % num_heads, kv head (n % num_heads) /
 *                (num_heads / num_kv_heads))
 *   key_pages,
 *   value_pages  [P, num_kv_heads, page_size, D] of kv_dtype
 *   key_scales,
 *   value_scales [P, num_kv_heads, page_size] float32 (NVM_KV_I8), else NULL
 *   block_table  [B, max_pages] int32: page of each logical page of a request
 *   context_lens [B] int32
 *   out          [N, L, D] of out_dtype: NVM_KV_F32 (the reference op's
 *                output), or NVM_KV_BF16 / NVM_KV_F16, the float32 result
 *                rounded once (the model's cast back to its activations)
 *
 * Key position j of request b (j < min(context_lens[b], max_pages *
 * page_size)) lives in page block_table[b, j / page_size], slot j % page_size.
 * Positions whose page id is negative are skipped, as in the reference; so are
 * page ids >= P (the reference reads past its pool there).  With is_causal,
 * query row i (of L) sees positions j <= i + context_len - L.  Rows with no
 * visible position are zero.  Sums are float32, like the reference.
 *
 * L = 1 with f16/bf16 pages and D of 64 or 128 runs the split-context decode
 * kernel (the query heads of a kv head share every page read); other shapes
 * run a one-wavefront-per-row kernel.  Each page tensor must be below 2 GiB.
 * Workspace: nvm_paged_attention_workspace_size (zero bytes when no split is
 * needed; workspace may then be NULL).
 */
int nvm_paged_attention_workspace_size(int64_t N, int64_t L, int64_t D, int64_t max_pages,
                                       int64_t page_size, int kv_dtype, int num_kv_heads,
                                       int num_heads, size_t *bytes);
int nvm_paged_attention(const float *q, int64_t N, int64_t L, int64_t D, const void *key_pages,
                        const void *value_pages, int64_t P, int64_t page_size, int kv_dtype,
                        const float *key_scales, const float *value_scales,
                        const int32_t *block_table, int64_t B, int64_t max_pages,
                        const int32_t *context_lens, float scale, int is_causal,
                        int num_kv_heads, int num_heads, int out_dtype, void *out,
                        void *workspace, size_t workspace_bytes, nvm_stream_t stream);

/*
 * Causal attention of an initial prefill: every request attends over its own
 * new tokens only.  Replaces the float32
 * `mx.fast.scaled_dot_product_attention(q, k, v, scale, mask="causal")` of
 * the model's initial prefill (models/qwen3.py:134-141).
 *
 *   q    [B * L, num_heads, D] float32
 *   k, v [B * L, num_kv_heads, D] float32
 *   out  [B * L, num_heads, D] of out_dtype (NVM_KV_F32, NVM_KV_BF16 or
 *        NVM_KV_F16: the float32 result rounded once)
 *
 * Token row b * L + i is position i of request b; query row i sees key rows
 * j <= i of its request, query head h reads kv head h / (num_heads /
 * num_kv_heads).  q, k and v must hold values of the activation dtype `dtype`
 * (NVM_DTYPE_BF16 or NVM_DTYPE_F16; the model's q/k norm and RoPE round
 * them): the products are then exact, the sums float32.  D of 64 or 128,
 * 1, 2, 4, 8 or 16 query heads per kv head, and a positive finite scale (the
 * model's head_dim ** -0.5) (else NVM_ERR_UNSUPPORTED).
 */
int nvm_causal_attention(const float *q, const float *k, const float *v, int64_t B, int64_t L,
                         int num_heads, int num_kv_heads, int64_t D, float scale, int dtype,
                         int out_dtype, void *out, nvm_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* NVM_ATTENTION_H */
