// Host-side launch interface shared between the kernel files and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace nvm {

// Records the message that nvm_last_error() returns on this thread; returns
// `code` (a negative NVM_ERR_* status).
int set_error(int code, const char *fmt, ...);

// Arguments of the grouped expert products (decode GEMV and prefill GEMM).
//   Sorted slot n (expert-major, see dispatch) reads activation row
//   a_map ? a_map[n] / a_div : n  and writes output row  o_map ? o_map[n] : n.
//   mat0 = (w0, s0, b0) and, for the fused gate/up product, mat1 = (w1, s1, b1)
//   are [E, R, K/8] words with [E, R, K/gs] scales and biases.
struct GroupedArgs {
  const uint16_t *act;
  int64_t act_ld;
  int64_t act_rows;  // rows of `act` (bounds of the activation buffer)
  const int32_t *a_map;
  int a_div;
  const int32_t *offsets;  // [E+1] slot ranges per expert; NULL (E = 1): all act_rows rows
  const uint32_t *w0;
  const uint16_t *s0, *b0;
  const uint32_t *w1;
  const uint16_t *s1, *b1;
  int R, K, gs, E;
  uint16_t *out;
  const int32_t *o_map;
  int64_t out_ld;
  // Routing finalised in the gate/up product's prologue (decode batches,
  // fused_route_supports): with route_part set, every block finalises the
  // act_rows tokens from these partial logits [act_rows][E][route_splits]
  // (top-k = a_div, renormalised when route_norm) and sorts the pairs in LDS;
  // offsets, a_map and o_map are then not read.  Block 0 writes the routing
  // for the stages after it: r_ids/r_scores [act_rows * a_div], r_offsets
  // [E + 1], r_sorted [act_rows * a_div].
  const double *route_part;
  int route_splits, route_norm;
  int32_t *r_ids;
  uint16_t *r_scores;
  int32_t *r_offsets, *r_sorted;
  // Prefill GEMM with bf16 activations only: act_h says `act` holds the
  // activations already in the fp16 form the GEMM's staging makes of them
  // (launch_act_to_f16), each 16-byte chunk x0..x7 stored in the pair order
  // (x0,x4)(x1,x5)(x2,x6)(x3,x7) of its MFMA operands, and out_h has the
  // gate/up epilogue store its bf16-rounded outputs in that form too (the act
  // of a down product with act_h set; R a multiple of 8).  The decode
  // products ignore both.
  int act_h, out_h;
  // With act_h and bf16 activations: the shift of each fp16 row group
  // (bf16_to_f16_pairs), act_sh[row * K / 64 + k-step] for activation row
  // `row` (NULL: no group shifted).  The gate/up epilogue with out_h writes
  // the shifts of the h it stores into out_sh [rows, R / 64] (may be NULL).
  const uint8_t *act_sh;
  uint8_t *out_sh;
  // Down product with the combine in its epilogue (launch_gemv3_down_combine,
  // act_rows = T * c_k pairs in sorted order, o_map = sorted): the scores
  // [pairs] (act bits, pair order) and y [T, out_ld] it writes.
  const uint16_t *c_scores;
  uint16_t *c_y;
  int c_k;
  // Gate/up product followed by the down product in the same launch
  // (launch_gemv3_fused_down): the down weights d_w/d_s/d_b [E, d_R, R]
  // (d_R rows over the R = I columns of h) and the float32 sums of each
  // half of its reduction, d_part [2][act_rows * a_div][d_R] by pair.
  const uint32_t *d_w;
  const uint16_t *d_s, *d_b;
  float *d_part;
  int d_R;
};

// Decode batches whose routing the gate/up product can finalise: at most
// kFusedPairs pairs, E <= 128 experts, top-k <= 16.
constexpr int kFusedPairs = 1024;
bool fused_route_supports(int64_t T, int64_t E, int k);

// Decode down product with the combine in its epilogue (gemv3.hip): one
// block per 16 rows of y, each over every pair of the batch (at most
// kTilePairs), y bit-identical to the down product followed by
// launch_combine.
constexpr int kTilePairs = 256;
bool gemv3_down_combine_supports(int K, int R, int E, int gs, int64_t pairs, int k);
hipError_t launch_gemv3_down_combine(int dtype, const GroupedArgs &a, hipStream_t st);

// Decode gate/up product with the down product of the same expert-major
// blocks (gemv3.hip, FDOWN): two blocks per expert, each over one half of
// the down reduction, writing float32 half sums to d_part; combined by
// launch_combine_split.  Shapes: K = 2048, R = 768, d_R a multiple of 256,
// at most 64 tokens; the routing finalised in the launch (route_part).
bool gemv3_fused_down_supports(int K, int R, int dR, int E, int gs, int64_t T, int k);
hipError_t launch_gemv3_fused_down(int dtype, const GroupedArgs &a, hipStream_t st);
// y[t] = rnd(sum_j rnd(rnd(part[0][t k + j] + part[1][t k + j]) * score[t k + j])):
// combine_kernel's arithmetic on the down output rnd(lo + hi).
hipError_t launch_combine_split(int dtype, const float *part, const void *scores, int64_t T, int k,
                                int64_t H, void *y, hipStream_t st);

// Router.  Partial float64 logits over hidden splits, then per-token finalise.
// With final_act the logits are rounded and stored as act [T, E] directly.
// route_splits: the splits launch_route_partial writes (read the environment
// override of route_i8_applies at each call); route_workspace_splits: an
// upper bound of them for any setting, for workspace sizes.
int route_splits(int64_t T, int64_t H, int64_t E);
int route_workspace_splits(int64_t T, int64_t H, int64_t E);
// The exact int8-MFMA partial logits (route_i8.hip), taken by
// launch_route_partial (without final_act) when route_i8_applies.
bool route_i8_applies(int64_t T, int64_t H);
int route_i8_splits(int64_t T, int64_t H, int64_t E);
hipError_t launch_route_i8(int dtype, const void *x, int64_t T, int64_t H, const uint32_t *wr,
                           const void *sr, const void *br, int64_t E, int gs, double *partial,
                           unsigned *done, hipStream_t st);
// The whole routing of batches the int8 router takes, for E <= 128 and
// top-k <= 16 (and at most 64 groups a row): logits, softmax, top-k and
// renormalisation in one launch of one block per 16 tokens, which writes
// ids/scores [T][k], its expert histogram counts[T/16][E] (for
// launch_dispatch_hist) and, with xh (bf16 x only), the fp16 copy of x that
// launch_act_to_f16 makes.
// (xsh [T][H / 64]: the shifts of the fp16 copy's groups, written with xh)
bool route_i8_fin_supports(int64_t T, int64_t H, int64_t E, int gs, int k);
hipError_t launch_route_i8_fin(int dtype, const void *x, int64_t T, int64_t H, const uint32_t *wr,
                               const void *sr, const void *br, int64_t E, int gs, int k, int norm,
                               int32_t *ids, void *scores, int32_t *counts, void *xh,
                               uint8_t *xsh, hipStream_t st);
// `done` (may be NULL) is a counter the partial launch zeroes for the fused
// finalise-and-dispatch launch that follows it.
hipError_t launch_route_partial(int dtype, const void *x, int64_t T, int64_t H, const uint32_t *wr,
                                const void *sr, const void *br, int64_t E, int gs, bool final_act,
                                double *partial, void *final_out, unsigned *done, hipStream_t st);
hipError_t launch_route_finalize(int dtype, const double *partial, int splits, int64_t T,
                                 int64_t E, int k, int norm, void *probs, int32_t *ids,
                                 void *scores, hipStream_t st);

// Decode batches of nvm_moe_forward (routed inside the gate/up product, see
// fused_route_supports): partial logits [T][E][decode_route_splits] float64.
int decode_route_splits(int64_t T, int64_t H, int64_t E);
hipError_t launch_route_partial_decode(int dtype, const void *x, int64_t T, int64_t H,
                                       const uint32_t *wr, const void *sr, const void *br,
                                       int64_t E, int gs, double *partial, hipStream_t st);

constexpr int kMaxExperts = 512;

// Decode batches (T <= kFusedRouteTokens): finalise the tokens and sort the
// pairs into expert order in one launch (its last block sorts; `done` is the
// block counter zeroed by launch_route_partial).
constexpr int64_t kFusedRouteTokens = 64;
bool route_fused_dispatch(int64_t T, int k);
hipError_t launch_route_finalize_dispatch(int dtype, const double *partial, int splits, int64_t T,
                                          int64_t E, int k, int norm, void *probs, int32_t *ids,
                                          void *scores, int32_t *offsets, int32_t *sorted,
                                          unsigned *done, hipStream_t st);

// Dispatch: stable counting sort of ids into expert order.  Up to
// kSortChunk pairs sort in one block; more take per-block histograms in a
// workspace of dispatch_workspace_bytes().
constexpr int64_t kSortChunk = 4096;
int64_t dispatch_workspace_bytes(int64_t n, int64_t E);
hipError_t launch_dispatch(const int32_t *ids, int64_t n, int64_t E, int32_t *offsets,
                           int32_t *sorted, void *workspace, hipStream_t st);
// The same sort from per-block histograms counts[n_cb][E] of consecutive
// runs of cb_pairs pairs (the last run may be short), as route_i8_fin writes
// them: one launch.
hipError_t launch_dispatch_hist(const int32_t *ids, int64_t n, int64_t E, const int32_t *counts,
                                int64_t n_cb, int cb_pairs, int32_t *offsets, int32_t *sorted,
                                hipStream_t st);

// Grouped products.  dual = fused gate/up with SwiGLU epilogue.
// Decode products need the reduction dimension in at most 8 slices of 1, 2,
// 4 or 8 whole 64-wide groups.
bool gemv_supports(int K);
int cu_count();  // compute units of the current device
hipError_t launch_gemv(int dtype, bool dual, const GroupedArgs &a, hipStream_t st);
// The one-wavefront-per-unit decode products (gemv3.hip): group size 64,
// K in {768, 1536, 2048, 4096}; launch_gemv takes them when supported.
bool gemv3_supports(int K, int R, int E, int gs);
hipError_t launch_gemv3(int dtype, bool dual, const GroupedArgs &a, hipStream_t st);
constexpr int kGemmBM = 128;   // prefill tile rows (routed pairs)
constexpr int kGemmBN = 128;   // prefill tile columns per weight matrix
hipError_t launch_gemm(int dtype, bool dual, const GroupedArgs &a, int64_t max_m_tiles,
                       hipStream_t st);
// bf16 x [n] -> its fp16 copy for the prefill GEMMs: each 64-value group
// shifted (bf16_to_f16_pairs) with its shift in sh [n / 64], each 16-byte
// chunk in the pair order of GroupedArgs::act_h; n a multiple of 64, `out`
// 16-byte aligned.
hipError_t launch_act_to_f16(const void *x, int64_t n, void *out, uint8_t *sh, hipStream_t st);

// Combine fused with the residual add and RMSNorm that follow the MoE block
// in the model (rows of H <= 8192, a multiple of 8).  split: `down` holds the
// float32 half sums [2][T * k][H] of launch_gemv3_fused_down.
hipError_t launch_combine_residual_norm(int dtype, const void *down, const void *scores,
                                        int64_t T, int k, int64_t H, const void *h,
                                        const void *w, float eps, void *h_out, void *x_out,
                                        hipStream_t st, bool split = false);
bool combine_residual_norm_supports(int64_t H);

// Multi-query paged attention on the matrix cores (paged_prefill.hip): L > 1
// query rows per request over f16/bf16 pages, head dims 64 and 128, 1, 2, 4,
// 8 or 16 query heads per kv head; the arguments of nvm_paged_attention.
bool paged_prefill_supports(int64_t L, int64_t D, int kv_dtype, int Hkv, int Hq);
hipError_t launch_paged_prefill(const float *q, int64_t B, int64_t L, int64_t D, const void *kp,
                                const void *vp, int64_t P, int64_t page_size, int kv_dtype,
                                const int32_t *bt, int64_t max_pages, const int32_t *lens,
                                float scale, int causal, int Hkv, int Hq, int out_dtype,
                                void *out, hipStream_t st);

// Combine: y[t] = rnd(sum_j rnd(down[t*k+j] * score[t,j])).
hipError_t launch_combine(int dtype, const void *down, const void *scores, int64_t T, int k,
                          int64_t H, void *y, hipStream_t st);

}  // namespace nvm
