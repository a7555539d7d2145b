// Routing finalise of decode batches, as a device building block: from the
// float64 partial logits of the router, the rest of route_topk
// (layers/moe.py:37-49) for four tokens per wavefront.
//
// The arithmetic is route_finalize_kernel's: the partials of a logit are
// added in split order and the sum is rounded once to the activation dtype;
// the softmax of those act logits runs in float64 and each probability is
// rounded once; top-k takes (probability desc, expert index asc); with
// norm_topk_prob the scores are rnd(p / rnd(sum of the k probabilities)).
// A token occupies one 16-lane row of the wavefront, so every reduction is a
// four-step DPP butterfly inside the row (quad_perm [1,0,3,2], quad_perm
// [2,3,0,1], row_half_mirror, row_mirror), after which all 16 lanes hold the
// same value (each step combines a lane with a partner that computes the
// same pair).
#pragma once

#include "common.h"
#include "sort.h"

namespace nvm {

constexpr int kRowExperts = 128;  // experts per 16-lane row: 8 per lane
constexpr int kRowTopK = 16;      // slots per token (one lane each)

template <class Op>
__device__ __forceinline__ double row_reduce_f64(double v, Op op) {
  v = op(v, dpp_f64<0xB1>(v));
  v = op(v, dpp_f64<0x4E>(v));
  v = op(v, dpp_f64<0x141>(v));
  return op(v, dpp_f64<0x140>(v));
}
__device__ __forceinline__ uint32_t row_max_u32(uint32_t v) {
  v = max(v, dpp_u32<0xB1>(v));
  v = max(v, dpp_u32<0x4E>(v));
  v = max(v, dpp_u32<0x141>(v));
  return max(v, dpp_u32<0x140>(v));
}

// A callable that issues nothing (the default `after_loads` below).
struct NoIssue {
  __device__ void operator()() const {}
};

// The rest of route_topk for the token of this lane's 16-lane row, from the
// float64 logit sums of its experts c + 16 j (c = lane % 16; experts past E
// ignored): the sums are rounded once to the activation dtype, the softmax
// of those act logits runs in float64 and each probability is rounded once,
// top-k takes (probability desc, expert index asc), and with norm_topk_prob
// the scores are rnd(p / rnd(sum of the k probabilities)).  With `tok`, slot i
// goes to s_ids[t*k + i] / s_sc[t*k + i] (act bits) and bit t is set in
// s_mask[expert] (LDS).  Every lane of the wavefront must call it.
template <int DT>
__device__ __forceinline__ void finalize_sums(const double (&sum)[8], int t, bool tok, int E, int k,
                                              int norm, int *s_ids, uint16_t *s_sc,
                                              uint64_t *s_mask) {
  using A = Act<DT>;
  constexpr int P = A::kPrec, EMIN = A::kEmin;
  const int lane = threadIdx.x & 63, c = lane & 15;
  double lg[8];
  double m = -INFINITY;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    lg[j] = c + 16 * j < E ? round_f64_to(sum[j], P, EMIN) : -INFINITY;
    m = fmax(m, lg[j]);
  }
  m = row_reduce_f64(m, [](double a, double b) { return fmax(a, b); });
  double p[8];
  double s = 0.0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    p[j] = c + 16 * j < E ? exp(lg[j] - m) : 0.0;
    s += p[j];
  }
  s = row_reduce_f64(s, [](double a, double b) { return a + b; });
  uint32_t key[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int e = c + 16 * j;
    // probabilities are >= +0, so their bit patterns order like their values;
    // the low half prefers the lower expert index on ties
    key[j] = e < E ? ((uint32_t)act_from_f64<DT>(p[j] / s) << 16) | (uint32_t)(0xFFFF - e) : 0u;
  }
  int my_id = 0;
  double my_p = 0.0, psum = 0.0;
  for (int i = 0; i < k; ++i) {
    uint32_t best = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) best = max(best, key[j]);
    best = row_max_u32(best);
    const int e = 0xFFFF - (int)(best & 0xFFFFu);
    const double pv = (double)A::to_f32(best >> 16);
    psum += pv;  // at most k act values: exact in float64
    if (c == i) {
      my_id = e;
      my_p = pv;
    }
    if ((e & 15) == c) {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (j == (e >> 4)) key[j] = 0u;
    }
  }
  if (tok && c < k) {
    double sc = my_p;
    if (norm) sc = my_p / round_f64_to(psum, P, EMIN);
    s_ids[t * k + c] = my_id;
    s_sc[t * k + c] = act_from_f64<DT>(sc);
    // (an OR commutes: the mask does not depend on the order of the lanes)
    __hip_atomic_fetch_or(&s_mask[my_id], 1ull << t, __ATOMIC_RELAXED,
                          __HIP_MEMORY_SCOPE_WORKGROUP);
  }
}

// Tokens t0 .. t0+3 (row r of the wavefront holds token t0 + r; rows past T
// compute and store nothing).  part is [T][E][splits] float64; E <= 128,
// k <= 16, T <= 64.  Slot i of token t goes to s_ids[t*k + i] and
// s_sc[t*k + i] (act bits), and bit t is set in s_mask[expert] (LDS, zeroed
// by the caller).  Every lane of the wavefront must call it.  after_loads()
// runs once, right after the partial logits are requested and before they
// are used (a caller's own loads issued there queue behind them).
template <int DT, class Issue = NoIssue>
__device__ __forceinline__ void finalize_rows(const double *__restrict__ part, int splits, int t0,
                                              int T, int E, int k, int norm, int *s_ids,
                                              uint16_t *s_sc, uint64_t *s_mask,
                                              Issue after_loads = Issue{}) {
  const int lane = threadIdx.x & 63, c = lane & 15;
  const int t = t0 + (lane >> 4);
  const bool tok = t < T;
  // all loads of the lane in flight together; absent tokens/experts read zeros
  const rsrc_t pr = make_rsrc(part, (uint32_t)((int64_t)T * E * splits * 8));
  double sum[8];
  if (splits == 2) {
    u32x4 v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int e = c + 16 * j;
      v[j] = bload16(pr, tok && e < E ? ((t * E + e) * 2) * 8 : kMaskedOffset, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    after_loads();
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < 8; ++j)
      sum[j] = (0.0 + __builtin_bit_cast(double, u32x2{v[j].x, v[j].y})) +
               __builtin_bit_cast(double, u32x2{v[j].z, v[j].w});
  } else {
    after_loads();
#pragma unroll
    for (int j = 0; j < 8; ++j) sum[j] = 0.0;
    for (int z = 0; z < splits; ++z) {
      u32x2 v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int e = c + 16 * j;
        v[j] = bload8(pr, tok && e < E ? ((t * E + e) * splits + z) * 8 : kMaskedOffset, 0);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) sum[j] += __builtin_bit_cast(double, v[j]);
    }
  }
  finalize_sums<DT>(sum, t, tok, E, k, norm, s_ids, s_sc, s_mask);
}

// finalize_rows for one token with the whole wavefront (T up to the number
// of wavefronts: small decode batches, where four tokens a wavefront would
// leave most lanes idle and the token's chain of float64 steps on 16 lanes).
// Lane c + 16 G holds the experts c + 16 j of finalize_sums for j = 2G and
// 2G + 1; every value is the one finalize_sums forms, in the same order:
// the softmax sum of row c is the sequential (0 + p_0) + p_1 + ... + p_7,
// carried from row G - 1 to row G, then the same 16-lane butterfly, so a
// token's routing is bit-identical to the four-tokens-a-wavefront path (the
// products stay batch-invariant).  after_loads() as in finalize_rows.
template <int DT, class Issue = NoIssue>
__device__ __forceinline__ void finalize_token64(const double *__restrict__ part, int splits, int t,
                                                 int T, int E, int k, int norm, int *s_ids,
                                                 uint16_t *s_sc, uint64_t *s_mask,
                                                 Issue after_loads = Issue{}) {
  using A = Act<DT>;
  constexpr int P = A::kPrec, EMIN = A::kEmin;
  const int lane = threadIdx.x & 63, c = lane & 15, G = lane >> 4;
  const bool tok = t < T;
  const rsrc_t pr = make_rsrc(part, (uint32_t)((int64_t)T * E * splits * 8));
  double sum[2];
  if (splits == 2) {
    u32x4 v[2];
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int e = c + 16 * (2 * G + jj);
      v[jj] = bload16(pr, tok && e < E ? ((t * E + e) * 2) * 8 : kMaskedOffset, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    after_loads();
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int jj = 0; jj < 2; ++jj)
      sum[jj] = (0.0 + __builtin_bit_cast(double, u32x2{v[jj].x, v[jj].y})) +
                __builtin_bit_cast(double, u32x2{v[jj].z, v[jj].w});
  } else {
    after_loads();
    sum[0] = sum[1] = 0.0;
    for (int z = 0; z < splits; ++z) {
      u32x2 v[2];
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const int e = c + 16 * (2 * G + jj);
        v[jj] = bload8(pr, tok && e < E ? ((t * E + e) * splits + z) * 8 : kMaskedOffset, 0);
      }
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) sum[jj] += __builtin_bit_cast(double, v[jj]);
    }
  }
  double lg[2], p[2];
  double m = -INFINITY;
#pragma unroll
  for (int jj = 0; jj < 2; ++jj) {
    const int e = c + 16 * (2 * G + jj);
    lg[jj] = e < E ? round_f64_to(sum[jj], P, EMIN) : -INFINITY;
    m = fmax(m, lg[jj]);
  }
  m = wave_reduce_f64(m, [](double a, double b) { return fmax(a, b); });
#pragma unroll
  for (int jj = 0; jj < 2; ++jj) {
    const int e = c + 16 * (2 * G + jj);
    p[jj] = e < E ? exp(lg[jj] - m) : 0.0;
  }
  // (0 + p_0) + p_1 in row 0, then + p_2 + p_3 in row 1 on row 0's value,
  // and so on: row 3 ends with finalize_sums' per-lane sum
  double s = (0.0 + p[0]) + p[1];
#pragma unroll
  for (int r = 1; r < 4; ++r) {
    const uint64_t u = __builtin_bit_cast(uint64_t, s);
    const uint32_t lo = (uint32_t)__shfl_up((int)(uint32_t)u, 16);
    const uint32_t hi = (uint32_t)__shfl_up((int)(uint32_t)(u >> 32), 16);
    const double in = __builtin_bit_cast(double, (uint64_t)lo | ((uint64_t)hi << 32));
    if (G == r) s = (in + p[0]) + p[1];
  }
  s = row_reduce_f64(s, [](double a, double b) { return a + b; });
  s = readlane_f64(s, 48);
  uint32_t key[2];
#pragma unroll
  for (int jj = 0; jj < 2; ++jj) {
    const int e = c + 16 * (2 * G + jj);
    key[jj] = e < E ? ((uint32_t)act_from_f64<DT>(p[jj] / s) << 16) | (uint32_t)(0xFFFF - e) : 0u;
  }
  int my_id = 0;
  double my_p = 0.0, psum = 0.0;
  for (int i = 0; i < k; ++i) {
    const uint32_t best = wave_max_u32(max(key[0], key[1]));
    const int e = 0xFFFF - (int)(best & 0xFFFFu);
    const double pv = (double)A::to_f32(best >> 16);
    psum += pv;  // at most k act values: exact in float64
    if (lane == i) {
      my_id = e;
      my_p = pv;
    }
    // expert e = c' + 16 j' lives in lane c' + 16 (j' >> 1), slot j' & 1
    if ((e & 15) == c && ((e >> 4) >> 1) == G) key[(e >> 4) & 1] = 0u;
  }
  if (tok && lane < k) {
    double sc = my_p;
    if (norm) sc = my_p / round_f64_to(psum, P, EMIN);
    s_ids[t * k + lane] = my_id;
    s_sc[t * k + lane] = act_from_f64<DT>(sc);
    __hip_atomic_fetch_or(&s_mask[my_id], 1ull << t, __ATOMIC_RELAXED,
                          __HIP_MEMORY_SCOPE_WORKGROUP);
  }
}

// The routing of a decode batch (T <= 64 tokens, E <= 128 experts, k <= 16)
// finalised and sorted inside one block, from the router's partial logits:
// the result of route_finalize followed by the dispatch sort
// (layers/moe.py:37-49, 16-17).  A token's k experts are distinct, so the
// pairs of expert e are one per token that chose it, in token order: with
// the token set of every expert as a 64-bit mask, the stable rank of pair
// (t, j) is the number of tokens below t in its expert's mask.
// Fills s_ids/s_sc [T*k], s_off [E+1] (slot offsets), s_cb [E+1] (exclusive
// prefix of ceil(count / chunk_rows)) and s_sorted [T*k].  All threads of
// the block must call it; it ends with a barrier.  With T no more than the
// wavefronts of the block, wavefront t finalises token t alone on all 64
// lanes (finalize_token64, the same bits as the four-token rows).  issue()
// runs once per wavefront: behind its partial-logit requests when it
// finalises one token or one group of four, else before them.
template <int DT, class Issue = NoIssue>
__device__ __forceinline__ void route_in_block(const double *__restrict__ part, int splits, int T, int E, int k,
                               int norm, int chunk_rows, int *s_ids, uint16_t *s_sc,
                               uint64_t *s_mask, int *s_off, int *s_cb, int *s_sorted,
                               Issue issue = Issue{}) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, NW = blockDim.x >> 6;
  for (int e = tid; e < E; e += blockDim.x) s_mask[e] = 0ull;
  __syncthreads();
  if (T <= NW) {
    // a token a wavefront
    if (wv < T)
      finalize_token64<DT>(part, splits, wv, T, E, k, norm, s_ids, s_sc, s_mask, issue);
    else
      issue();
  } else if (4 * wv < T && 4 * (wv + NW) >= T) {
    finalize_rows<DT>(part, splits, 4 * wv, T, E, k, norm, s_ids, s_sc, s_mask, issue);
  } else {
    issue();
    for (int t0 = 4 * wv; t0 < T; t0 += 4 * NW)
      finalize_rows<DT>(part, splits, t0, T, E, k, norm, s_ids, s_sc, s_mask);
  }
  __syncthreads();
  if (wv == 0) {
    int carry = 0, ccarry = 0;
    for (int e0 = 0; e0 < E; e0 += 64) {
      const int e = e0 + lane;
      const int n = e < E ? __popcll(s_mask[e]) : 0;
      const int nc = (n + chunk_rows - 1) / chunk_rows;
      const int inc = wave_incl_scan(n, lane), cinc = wave_incl_scan(nc, lane);
      if (e < E) {
        s_off[e] = carry + inc - n;
        s_cb[e] = ccarry + cinc - nc;
      }
      carry += __shfl(inc, 63);
      ccarry += __shfl(cinc, 63);
    }
    if (lane == 0) {
      s_off[E] = carry;
      s_cb[E] = ccarry;
    }
  }
  __syncthreads();
  for (int p = tid; p < T * k; p += blockDim.x) {
    const int e = s_ids[p], t = p / k;
    s_sorted[s_off[e] + __popcll(s_mask[e] & ((1ull << t) - 1ull))] = p;
  }
  __syncthreads();
}

}  // namespace nvm
