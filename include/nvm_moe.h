/*
 * nvm_moe.h — C ABI of the MI355X (gfx950) Qwen3 sparse-MoE block.
 *
 * This shared library replaces, for the MoE hot path of nano-vllm-metal, the
 * reference's native op binding and the MLX built-ins that `layers/moe.py`
 * calls.  Paths below are relative to the reference's `src/nano_vllm_metal`.
 *
 * Conventions shared by every entry point:
 *   - Pointers are HIP device pointers; sizes are element counts (int64_t).
 *   - Activation tensors ("act") are fp16 or bf16, selected by `dtype`
 *     (NVM_DTYPE_F16 / NVM_DTYPE_BF16); scales and biases share that dtype
 *     (the reference checks the same, metal/src/quantized_matmul.cpp:26-37).
 *   - Quantised weights use the MLX affine layout: `bits` = 4, uint32 words
 *     packing 8 codes each, code j of a word in bits [4j, 4j+4); per-group
 *     scale and bias with `group_size` in {64, 128}; w = q*scale + bias.
 *     Expert tensors are [E, out, in/8] words and [E, out, in/group] scales.
 *   - All tensors are dense row-major (the reference requires row-contiguous
 *     inputs, quantized_matmul.cpp:96-101).
 *   - Work is enqueued on `stream` (a hipStream_t); nothing synchronises the
 *     host.  The library allocates no device memory: callers pass outputs and,
 *     where stated, a workspace sized by the matching *_workspace_size call.
 *   - Return value: NVM_OK (0) or a negative NVM_ERR_* code; the message is
 *     available from nvm_last_error() on the calling thread.  No C++
 *     exception crosses this boundary.
 *   - Calls on one stream are ordered; calls sharing a workspace must not
 *     overlap in time.
 */
#ifndef NVM_MOE_H
#define NVM_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NVM_ABI_VERSION 2

enum nvm_dtype { NVM_DTYPE_F16 = 0, NVM_DTYPE_BF16 = 1 };

enum nvm_status {
  NVM_OK = 0,
  NVM_ERR_INVALID = -1,     /* bad argument: shape, dtype, null pointer  */
  NVM_ERR_UNSUPPORTED = -2, /* valid request this build does not handle  */
  NVM_ERR_WORKSPACE = -3,   /* workspace missing or too small            */
  NVM_ERR_HIP = -4          /* a HIP runtime call failed                 */
};

/* Expert-product regime: the decode MFMA-GEMV or the prefill LDS/MFMA GEMM.
 * NVM_REGIME_AUTO picks by routed pairs per expert. */
enum nvm_regime { NVM_REGIME_AUTO = 0, NVM_REGIME_DECODE = 1, NVM_REGIME_PREFILL = 2 };

typedef void *nvm_stream_t; /* hipStream_t */

int nvm_abi_version(void);
const char *nvm_last_error(void);

/*
 * Dense W4A16 matmul: out[M,K] = a[M,N] . dequant(b[K,N/8])^T.
 * Replaces `_ext.quantized_matmul(scales, biases, group_size, bits, a, b,
 * transpose_b)` (metal/bindings.cpp:16-32; op metal/src/quantized_matmul.cpp:17-82,
 * CPU loop :84-148), which `quantized_linear` uses for the router logits
 * (layers/linear.py:92-126, layers/moe.py:43).  Like the reference, only
 * transpose_b = 1 and bits = 4 are accepted; group_size may be 64 or 128.
 * Router-sized products (K <= 512 outputs, M <= 64 rows) accumulate in
 * float64 and are rounded once to act.  The rest (the projections of a dense
 * layer, prefill batches) run on the expert-product kernels as one expert,
 * accumulating in float32 as the reference's kernels do
 * (quantized_matmul.metal:25-44, :100-110), when N is a multiple of 64 up to
 * 8192 and K a multiple of 16; other shapes take the float64 path (exact,
 * but bound by the float64 matrix cores: slow for large products).  Operands
 * of more than 2 GiB (a or b) are rejected with NVM_ERR_UNSUPPORTED.
 * Needs no workspace.
 */
int nvm_quantized_matmul(const void *scales, const void *biases, int group_size, int bits,
                         const void *a, const uint32_t *b, int transpose_b, void *out,
                         int64_t M, int64_t N, int64_t K, int dtype, nvm_stream_t stream);

/*
 * Router: logits = x . dequant(Wr)^T rounded to act, probs = act-rounded
 * softmax (float64 inside), ids = top-k with ties to the lower expert index
 * in (prob desc, index asc) slot order, scores = probs[ids], renormalised to
 * rnd(s / rnd(sum s)) when norm_topk_prob != 0.
 * Replaces `route_topk` (layers/moe.py:37-49).
 *   x [T,H] act; wr [E,H/8]; sr, br [E,H/group] act
 *   probs [T,E] act (may be NULL); ids [T,k] int32; scores [T,k] act
 * x and the router weights must each stay below 2 GiB (NVM_ERR_UNSUPPORTED).
 * Workspace: nvm_route_workspace_size.
 */
int nvm_route_workspace_size(int64_t T, int64_t H, int64_t E, size_t *bytes);
int nvm_moe_route(const void *x, int64_t T, int64_t H, const uint32_t *wr, const void *sr,
                  const void *br, int64_t E, int group_size, int bits, int top_k,
                  int norm_topk_prob, int dtype, void *probs, int32_t *ids, void *scores,
                  void *workspace, size_t workspace_bytes, nvm_stream_t stream);

/*
 * Dispatch: counting sort of the flat expert ids (n = pairs, usually T*k)
 * into expert order, stable in pair index.  Replaces the `argsort` pair of
 * `grouped_expert_linear` (layers/moe.py:16-17).
 *   ids [n] int32 in [0,E); expert_offsets [E+1] int32 (exclusive prefix of
 *   the histogram); sorted_pairs [n] int32 (pair indices, expert-major).
 * Pairs whose id lies outside [0,E) are left out: they fall in no expert's
 * range, offsets[E] counts only the valid pairs, and sorted_pairs[offsets[E]..n)
 * is not written.  1 <= E <= 512.  Workspace: nvm_dispatch_workspace_size
 * (zero bytes, and workspace may be NULL, up to 4096 pairs).
 */
int nvm_dispatch_workspace_size(int64_t n, int64_t E, size_t *bytes);
int nvm_moe_dispatch(const int32_t *ids, int64_t n, int64_t E, int32_t *expert_offsets,
                     int32_t *sorted_pairs, void *workspace, size_t workspace_bytes,
                     nvm_stream_t stream);

/*
 * Routing followed by dispatch, as nvm_moe_forward runs them: the outputs of
 * nvm_moe_route (probs may be NULL) and of nvm_moe_dispatch over the T*k ids.
 * Decode batches (T <= 64) finalise and sort in a single launch.
 * Replaces `route_topk` plus the `argsort` pair (layers/moe.py:37-49, 16-17).
 * Workspace: nvm_route_dispatch_workspace_size.
 */
int nvm_route_dispatch_workspace_size(int64_t T, int64_t H, int64_t E, int top_k, size_t *bytes);
int nvm_moe_route_dispatch(const void *x, int64_t T, int64_t H, const uint32_t *wr,
                           const void *sr, const void *br, int64_t E, int group_size, int bits,
                           int top_k, int norm_topk_prob, int dtype, void *probs, int32_t *ids,
                           void *scores, int32_t *expert_offsets, int32_t *sorted_pairs,
                           void *workspace, size_t workspace_bytes, nvm_stream_t stream);

/*
 * Grouped expert linear: out[r] = x[r] . dequant(W[ids[r]])^T rounded to act,
 * for every row r of x [n, D].  Replaces `grouped_expert_linear`
 * (layers/moe.py:8-34, whose product runs in MLX `gather_qmm`).
 *   w [E,O,D/8]; s, b [E,O,D/group]; ids [n] int32; out [n,O] act
 * Workspace: nvm_grouped_linear_workspace_size.
 */
int nvm_grouped_linear_workspace_size(int64_t n, int64_t D, int64_t O, int64_t E, size_t *bytes);
int nvm_grouped_expert_linear(const void *x, int64_t n, int64_t D, const uint32_t *w,
                              const void *s, const void *b, int64_t E, int64_t O,
                              int group_size, int bits, const int32_t *ids, int dtype,
                              void *out, int regime, void *workspace, size_t workspace_bytes,
                              nvm_stream_t stream);

/*
 * Stages of the block after routing and dispatch, callable one at a time
 * (the fused nvm_moe_forward runs exactly these).  `expert_offsets` and
 * `sorted_pairs` are the outputs of nvm_moe_dispatch over the T*k flat ids.
 *
 * Gate/up products with fused SwiGLU: for sorted slot n (pair p =
 * sorted_pairs[n], token p / k, expert e), h[n] = rnd(silu(rnd(x.Wg[e]^T)) *
 * rnd(x.Wu[e]^T)).  Replaces the gate and up `grouped_expert_linear` calls and
 * `silu(gate) * up` of layers/moe.py:81-84 (layers/activation.py:21-24).
 *   x [T,H] act; wg/wu [E,I,H/8]; sg,bg,su,bu [E,I,H/group]; h [T*k, I] act
 */
int nvm_moe_expert_gateup(const void *x, int64_t T, int64_t H, int64_t I, int64_t E, int top_k,
                          int group_size, int bits, int dtype, const uint32_t *wg,
                          const void *sg, const void *bg, const uint32_t *wu, const void *su,
                          const void *bu, const int32_t *expert_offsets,
                          const int32_t *sorted_pairs, void *h, int regime,
                          nvm_stream_t stream);

/*
 * Down product: down[sorted_pairs[n]] = rnd(h[n] . Wd[e]^T), written in flat
 * pair order (the `out[inv_sort_idx]` un-permute of layers/moe.py:33).
 * Replaces the down `grouped_expert_linear` call of layers/moe.py:83-85.
 *   h [n_pairs, I] act; wd [E,H,I/8]; sd,bd [E,H,I/group]; down [n_pairs, H] act
 */
int nvm_moe_expert_down(const void *h, int64_t n_pairs, int64_t H, int64_t I, int64_t E,
                        int group_size, int bits, int dtype, const uint32_t *wd, const void *sd,
                        const void *bd, const int32_t *expert_offsets,
                        const int32_t *sorted_pairs, void *down, int regime,
                        nvm_stream_t stream);

/*
 * Combine: y[t] = rnd(sum_j rnd(down[t*k+j] * scores[t,j])), j in slot order.
 * Replaces `mx.sum(expert_output * expert_scores[..., None], axis=-2)`
 * (layers/moe.py:85-86).  H must be a multiple of 8.
 */
int nvm_moe_combine(const void *down, const void *scores, int64_t T, int top_k, int64_t H,
                    int dtype, void *y, nvm_stream_t stream);

/*
 * The whole sparse-MoE block: route -> dispatch -> gate/up products with
 * fused SwiGLU -> down product -> weighted combine.  Replaces `Moe.__call__`
 * (layers/moe.py:69-86).
 *   x [T,H] act -> y [T,H] act
 *   wr/sr/br router [E,H/8], [E,H/group]
 *   wg/sg/bg, wu/su/bu gate and up [E,I,H/8], [E,I,H/group]
 *   wd/sd/bd down [E,H,I/8], [E,H,I/group]
 *   ids_out [T,k] int32 and scores_out [T,k] act are optional (NULL).
 * Workspace: nvm_moe_workspace_size.
 */
int nvm_moe_workspace_size(int64_t T, int64_t H, int64_t I, int64_t E, int top_k, size_t *bytes);
int nvm_moe_forward(const void *x, int64_t T, int64_t H, int64_t I, int64_t E, int top_k,
                    int norm_topk_prob, int group_size, int bits, int dtype,
                    const uint32_t *wr, const void *sr, const void *br,
                    const uint32_t *wg, const void *sg, const void *bg,
                    const uint32_t *wu, const void *su, const void *bu,
                    const uint32_t *wd, const void *sd, const void *bd,
                    void *y, int32_t *ids_out, void *scores_out, int regime,
                    void *workspace, size_t workspace_bytes, nvm_stream_t stream);

/*
 * One stage of nvm_moe_forward's launch sequence, for timing the block's
 * kernels one at a time: 0 = routing and dispatch (decode batches: the
 * partial logits only, the gate/up stage finalising the routing), 1 = gate/up
 * products with SwiGLU, 2 = down products, 3 = combine.  Stage s reads what
 * stages 0..s-1 of a call with the same arguments and workspace left there;
 * stages 0..3 in order compute exactly what nvm_moe_forward computes (the
 * Moe.__call__ steps of layers/moe.py:77-86, one at a time).  ids_out and
 * scores_out, when given, must be the same in every stage; y is written by
 * stage 3 only.  (For decode batches of at most 16 pairs nvm_moe_forward
 * runs stages 2 and 3 as one launch, the down product with the combine in
 * its epilogue; its y is bit-identical to stages 2 and 3 run apart.)
 *
 * Stages 4 and 5 are the forward's own grouping where it runs both products
 * in one launch (nvm_moe_forward_plan): 4 = gate/up and down products as
 * nvm_moe_forward launches them (one launch where it fuses them, leaving the
 * down output in the workspace as float32 sums of the two halves of its
 * reduction; else stages 1 and 2), 5 = the combine that follows stage 4.
 * Stages 0, 4, 5 in order compute exactly what nvm_moe_forward computes; y
 * is bit-identical to stages 0..3.
 */
int nvm_moe_forward_stage(int stage, const void *x, int64_t T, int64_t H, int64_t I, int64_t E,
                          int top_k, int norm_topk_prob, int group_size, int bits, int dtype,
                          const uint32_t *wr, const void *sr, const void *br,
                          const uint32_t *wg, const void *sg, const void *bg,
                          const uint32_t *wu, const void *su, const void *bu,
                          const uint32_t *wd, const void *sd, const void *bd,
                          void *y, int32_t *ids_out, void *scores_out, int regime,
                          void *workspace, size_t workspace_bytes, nvm_stream_t stream);

/*
 * Which launches nvm_moe_forward makes for these arguments (no device work):
 * *fused_products = 1 when it runs the gate/up and down products of a decode
 * batch as one launch (expert-major blocks, two per expert, each over one
 * half of the down reduction; the combine then adds the halves), else 0.  The
 * choice depends on the shapes, T, top_k, regime and the NVM_FUSED_DOWN /
 * NVM_GEMV_STATIC environment overrides; y is bit-identical either way.  No
 * counterpart in the reference: for callers that time or profile the block's
 * kernels (stages 4 and 5 of nvm_moe_forward_stage).
 */
int nvm_moe_forward_plan(int64_t T, int64_t H, int64_t I, int64_t E, int top_k, int group_size,
                         int regime, int *fused_products);

/*
 * nvm_moe_forward without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference: it is
 * nvm_moe_forward with its workspace taken from a static device array of
 * nvm_moe_scratch_bytes() bytes (32 MiB) that every GPU the library runs on
 * holds until the process ends.  Calls needing more workspace than that
 * (nvm_moe_workspace_size) return NVM_ERR_UNSUPPORTED; at the 30B-A3B shape
 * (hidden 2048, 128 experts, top-8, intermediate 768) that is beyond about
 * 540 tokens.  The call allocates nothing (no
 * hipMalloc, no library allocation).  All calls on one GPU share the array:
 * calls that overlap in time on one GPU (other streams, other threads) race.
 * Nothing in the array needs to start at zero (the routing kernels reset
 * the one counter they use).  The current device must be the stream's.
 * nvm_moe_scratch_bytes also locates the current device's array: call it on
 * each device before capturing a noalloc call into a HIP graph (otherwise
 * the first call on a device locates it, which may load the code object).
 */
int nvm_moe_scratch_bytes(size_t *bytes);
int nvm_moe_forward_noalloc(const void *x, int64_t T, int64_t H, int64_t I, int64_t E, int top_k,
                            int norm_topk_prob, int group_size, int bits, int dtype,
                            const uint32_t *wr, const void *sr, const void *br,
                            const uint32_t *wg, const void *sg, const void *bg,
                            const uint32_t *wu, const void *su, const void *bu,
                            const uint32_t *wd, const void *sd, const void *bd, void *y,
                            int32_t *ids_out, void *scores_out, int regime, nvm_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* NVM_MOE_H */
