// Router: logits = x . dequant(Wr)^T, precise softmax, top-k, renormalisation.
//
// Restates layers/moe.py:37-49 (route_topk) and the router GEMV it calls
// (layers/linear.py:92-126 -> metal/src/quantized_matmul.cpp:117-145).
//
// Every value the reference materialises in the activation dtype (logits,
// probabilities, scores) is produced here as the correctly rounded value of
// the exact mathematical result: the dot products (on the float64 matrix
// cores) and the softmax run in float64 and are rounded once, directly from
// float64.  A float64 sum of at
// most a few thousand products of a bf16/fp16 activation and an fp32-exact
// weight is within ~2^-40 relative of the exact sum, so the rounded logits,
// and with them the top-k ids, do not depend on summation order.
#include <algorithm>

#include "common.h"
#include "finalize.h"
#include "internal.h"
#include "sort.h"

namespace nvm {

namespace {

typedef double f64x4 __attribute__((ext_vector_type(4)));

// Partial float64 logits on the matrix cores (v_mfma_f64_16x16x4_f64).
//
// One wavefront owns a tile of 16 tokens x (16*EB) experts over the hidden
// range [z*KR, (z+1)*KR).  Per 32-wide hidden chunk, lane (c, G) (c = l%16,
// G = l/16) supplies activations x[t0+c][k] and dequantised weights
// w[e0+c][k] = q*s + b (exact in float64) for k = chunk + 8G + m, m = 0..7, so
// MFMA m covers hidden columns {chunk + m, +8, +16, +24}: every column of the
// chunk exactly once, 8 consecutive bf16/fp16 values and one packed word per
// lane.  The D fragment of the float64 MFMA is row-interleaved: element i of
// lane (c, G) is token t0+G+4i of expert e0+c.
//
// Items are (token tile, expert tile, output split z < splits).  With
// wpb > 1 a block owns one item and its wpb wavefronts split the item's hidden
// range further; their float64 partials meet in LDS and are added in
// wavefront order.  With `fin` (logits rounded straight to the activation
// dtype, no partial buffer) splits is 1.
constexpr int kMaxBlockSplits = 8;  // wavefronts of an in-block hidden split

template <int DT, int EB, bool SB_VEC>
__global__ __launch_bounds__(512) void route_mfma_kernel(
    const uint16_t *__restrict__ x, int T, int H, const uint32_t *__restrict__ wr,
    const uint16_t *__restrict__ sr, const uint16_t *__restrict__ br, int E, int gs, int KR,
    int n_tt, int n_eb, int splits, int wpb, double *__restrict__ part,
    uint16_t *__restrict__ fin, unsigned *__restrict__ done) {
  using A = Act<DT>;
  constexpr int NC = 8;  // 32-wide chunks per batch; all loads of a batch are in flight together
  hoist_args(x, T, H, wr, sr, br, E, gs, KR, n_tt, n_eb, splits, wpb, part, fin, done);
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  // the finalising launch that follows counts its blocks from zero
  if (done && blockIdx.x == 0 && threadIdx.x == 0) *done = 0u;
  // in-block splits: one item per block (uniform exit, the block meets at a
  // barrier); else one item per wavefront
  const bool in_block = wpb > 1;
  const int item = in_block ? blockIdx.x : blockIdx.x * (blockDim.x >> 6) + wv;
  if (item >= n_tt * n_eb * splits) return;
  const int tt = item % n_tt;
  const int eb = (item / n_tt) % n_eb;
  const int z = item / (n_tt * n_eb);
  const int col = lane & 15, G = lane >> 4;
  const int t = tt * 16 + col;
  const int k_begin = (in_block ? z * wpb + wv : z) * KR;
  const int HW = H / 8, GPR = H / gs;

  const rsrc_t xr = make_rsrc(x, (uint32_t)((int64_t)T * H * 2));
  const rsrc_t wrr = make_rsrc(wr, (uint32_t)((int64_t)E * HW * 4));
  const rsrc_t srr = make_rsrc(sr, (uint32_t)((int64_t)E * GPR * 2));
  const rsrc_t brr = make_rsrc(br, (uint32_t)((int64_t)E * GPR * 2));
  // lanes of tokens >= T or experts >= E read zeros
  const int xo = t < T ? (t * H + k_begin + 8 * G) * 2 : kMaskedOffset;
  int wo[EB], so[EB];
  bool e_ok[EB];
#pragma unroll
  for (int b = 0; b < EB; ++b) {
    const int e = (eb * EB + b) * 16 + col;
    e_ok[b] = e < E;
    wo[b] = e_ok[b] ? (e * HW + k_begin / 8 + G) * 4 : kMaskedOffset;
    so[b] = e_ok[b] ? e * GPR * 2 : kMaskedOffset;
  }

  // CH independent accumulator chains per expert tile shorten the dependent
  // MFMA chain (four chains in all); they are added once at the end
  constexpr int CH = 4 / EB;
  f64x4 acc[EB][CH];
#pragma unroll
  for (int b = 0; b < EB; ++b)
#pragma unroll
    for (int h = 0; h < CH; ++h) acc[b][h] = f64x4{0.0, 0.0, 0.0, 0.0};

  for (int kb = 0; kb < KR; kb += 32 * NC) {
    const int kbs = __builtin_amdgcn_readfirstlane(kb);
    // group of chunk c for every lane: (k_begin + kb)/gs + c*32/gs
    const int g0 = (k_begin + kbs) / gs;
    u32x4 xv[NC];
    uint32_t qv[EB][NC];
    // packed scales/biases: the 16-bit value of group i is half (i & 1) of dword i >> 1
    u32x2 sv[EB], bv[EB];
    // chunks past the split's range read through masked offsets
#pragma unroll
    for (int c = 0; c < NC; ++c)
      xv[c] = bload16(xr, kbs + 32 * c < KR ? xo + 64 * c : kMaskedOffset, 2 * kbs);
#pragma unroll
    for (int b = 0; b < EB; ++b) {
#pragma unroll
      for (int c = 0; c < NC; ++c)
        qv[b][c] = bload4(wrr, kbs + 32 * c < KR ? wo[b] + 16 * c : kMaskedOffset, kbs / 2);
      if constexpr (SB_VEC) {
        sv[b] = bload8(srr, so[b], 2 * g0);
        bv[b] = bload8(brr, so[b], 2 * g0);
      } else {
        uint32_t s4[4], b4[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          s4[i] = bload2(srr, so[b] + 2 * i, 2 * g0);
          b4[i] = bload2(brr, so[b] + 2 * i, 2 * g0);
        }
        sv[b] = u32x2{s4[0] | (s4[1] << 16), s4[2] | (s4[3] << 16)};
        bv[b] = u32x2{b4[0] | (b4[1] << 16), b4[2] | (b4[3] << 16)};
      }
    }
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      if (kb + 32 * c >= KR) break;
      double xd[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        xd[2 * i] = (double)A::lo(xv[c][i]);
        xd[2 * i + 1] = (double)A::hi(xv[c][i]);
      }
      const int gi = (32 * c) / gs;  // 0..3 (group 64) or 0..1 (group 128)
#pragma unroll
      for (int b = 0; b < EB; ++b) {
        const uint32_t sd = sv[b][gi >> 1], bd = bv[b][gi >> 1];
        const double s = (double)((gi & 1) ? A::hi(sd) : A::lo(sd));
        const double bb = (double)((gi & 1) ? A::hi(bd) : A::lo(bd));
#pragma unroll
        for (int m = 0; m < 8; ++m) {
          const double w = fma((double)((qv[b][c] >> (4 * m)) & 0xFu), s, bb);
          acc[b][m % CH] = __builtin_amdgcn_mfma_f64_16x16x4f64(xd[m], w, acc[b][m % CH], 0, 0, 0);
        }
      }
    }
  }
#pragma unroll
  for (int b = 0; b < EB; ++b)
#pragma unroll
    for (int h = 1; h < CH; ++h) acc[b][0] += acc[b][h];
  auto store = [&](int b, int i, double v) {
    const int e = (eb * EB + b) * 16 + col;
    const int tok = tt * 16 + G + 4 * i;
    if (!e_ok[b] || tok >= T) return;
    if (fin)
      fin[(int64_t)tok * E + e] = act_from_f64<DT>(v);
    else
      part[((int64_t)tok * E + e) * splits + z] = v;
  };
  if (in_block) {
    // [wavefront][tile b][element i][lane]; the EB * 4 (tile, element) sums
    // are dealt over the block's wavefronts, each adding its wpb (<= 8)
    // partials in wavefront order
    extern __shared__ double s_part[];
#pragma unroll
    for (int b = 0; b < EB; ++b)
#pragma unroll
      for (int i = 0; i < 4; ++i) s_part[((wv * EB + b) * 4 + i) * 64 + lane] = acc[b][0][i];
    __syncthreads();
    for (int j = wv; j < EB * 4; j += wpb) {
      const int b = j >> 2, i = j & 3;
      double v[kMaxBlockSplits];
#pragma unroll
      for (int w = 0; w < kMaxBlockSplits; ++w)
        v[w] = w < wpb ? s_part[((w * EB + b) * 4 + i) * 64 + lane] : 0.0;
      double sum = v[0];
#pragma unroll
      for (int w = 1; w < kMaxBlockSplits; ++w)
        if (w < wpb) sum += v[w];
      store(b, i, sum);
    }
    return;
  }
#pragma unroll
  for (int b = 0; b < EB; ++b)
#pragma unroll
    for (int i = 0; i < 4; ++i) store(b, i, acc[b][0][i]);
}

constexpr int kMaxExpertSlots = 8;  // experts per lane: E <= 512
constexpr int kMaxSplits = 16;      // hidden splits of the partial logits

// Token t, one wavefront: sum the split partials (in split order), round the
// logits, softmax in float64, select top-k by (prob desc, index asc),
// renormalise.  Lane i < k returns expert id and score of slot i.  Each lane
// holds experts lane + 64 j for j < NS (NS * 64 >= E).
template <int DT, int NS>
__device__ __forceinline__ void finalize_token(const double *__restrict__ part, int splits, int t,
                                               int E, int k, int norm, uint16_t *__restrict__ probs,
                                               int &my_id, uint16_t &my_score) {
  const int lane = threadIdx.x & 63;
  constexpr int P = Act<DT>::kPrec, EMIN = Act<DT>::kEmin;
  // all partials of a logit are contiguous: issue every load of a slot
  // before summing (loads past `splits` read zeros)
  const rsrc_t pr = make_rsrc(part + (int64_t)t * E * splits, (uint32_t)(E * splits * 8));
  double lg[NS];
  double mloc = -INFINITY;
#pragma unroll
  for (int j = 0; j < NS; ++j) lg[j] = -INFINITY;
  // slots are read two at a time, all loads of a pair of slots in flight
  // together (partials past `splits` read as +0.0 and leave the sums unchanged)
  constexpr int SB = NS < 2 ? NS : 2;
#pragma unroll
  for (int j0 = 0; j0 < NS; j0 += SB) {
    u32x4 v[SB][kMaxSplits / 2];
#pragma unroll
    for (int jb = 0; jb < SB; ++jb) {
      const int e = lane + 64 * (j0 + jb);
      const int off = e < E ? e * splits * 8 : kMaskedOffset;
#pragma unroll
      for (int z2 = 0; z2 < kMaxSplits / 2; ++z2)
        v[jb][z2] = bload16(pr, 2 * z2 < splits ? off + 16 * z2 : kMaskedOffset, 0);
    }
#pragma unroll
    for (int jb = 0; jb < SB; ++jb) {
      const int e = lane + 64 * (j0 + jb);
      double sum = 0.0;
#pragma unroll
      for (int z2 = 0; z2 < kMaxSplits / 2; ++z2) {
        sum += __builtin_bit_cast(double, u32x2{v[jb][z2].x, v[jb][z2].y});
        // an odd split count leaves the last pair's second value to the next
        // expert's row
        if (2 * z2 + 1 < splits) sum += __builtin_bit_cast(double, u32x2{v[jb][z2].z, v[jb][z2].w});
      }
#pragma unroll
      for (int jj = 0; jj < NS; ++jj)
        if (jj == j0 + jb && e < E) lg[jj] = round_f64_to(sum, P, EMIN);
    }
  }
#pragma unroll
  for (int j = 0; j < NS; ++j) mloc = fmax(mloc, lg[j]);
  const double m = wave_reduce_f64(mloc, [](double a, double b) { return fmax(a, b); });
  double p[NS];
  double sloc = 0.0;
#pragma unroll
  for (int j = 0; j < NS; ++j) {
    const int e = lane + 64 * j;
    p[j] = e < E ? exp(lg[j] - m) : 0.0;
    sloc += p[j];
  }
  const double sum = wave_reduce_f64(sloc, [](double a, double b) { return a + b; });
  uint32_t key[NS];
#pragma unroll
  for (int j = 0; j < NS; ++j) {
    const int e = lane + 64 * j;
    key[j] = 0;
    if (e < E) {
      const uint16_t pb = act_from_f64<DT>(p[j] / sum);
      if (probs) probs[(int64_t)t * E + e] = pb;
      // probabilities are >= +0, so their bit patterns order like their values;
      // the low half prefers the lower expert index on ties
      key[j] = ((uint32_t)pb << 16) | (uint32_t)(0xFFFF - e);
    }
  }
  int id = 0;
  double my_p = 0.0, psum = 0.0;
  for (int i = 0; i < k; ++i) {
    uint32_t best = 0;
#pragma unroll
    for (int j = 0; j < NS; ++j) best = max(best, key[j]);
    best = wave_max_u32(best);
    const int e = 0xFFFF - (int)(best & 0xFFFFu);
    const double pv = (double)Act<DT>::to_f32(best >> 16);
    psum += pv;  // at most k act values: exact in float64
    if (lane == i) {
      id = e;
      my_p = pv;
    }
    if ((e & 63) == lane) {
#pragma unroll
      for (int j = 0; j < NS; ++j)
        if (j == (e >> 6)) key[j] = 0;
    }
  }
  double sc = my_p;
  if (norm) sc = my_p / round_f64_to(psum, P, EMIN);
  my_id = id;
  my_score = act_from_f64<DT>(sc);
}

// One wavefront per token.
template <int DT, int NS>
__global__ __launch_bounds__(256) void route_finalize_kernel(
    const double *__restrict__ part, int splits, int T, int E, int k, int norm,
    uint16_t *__restrict__ probs, int32_t *__restrict__ ids, uint16_t *__restrict__ scores) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (t >= T) return;
  int id;
  uint16_t sc;
  finalize_token<DT, NS>(part, splits, t, E, k, norm, probs, id, sc);
  if (lane < k) {
    ids[(int64_t)t * k + lane] = id;
    scores[(int64_t)t * k + lane] = sc;
  }
}

// Small batches: one wavefront per token, four per block (one per SIMD);
// the last block to finish (a counter in the workspace, zeroed by the
// partial-logit launch that precedes this one) sorts the T*k ids into expert
// order (sort.h), so finalising and dispatch are one launch.
template <int DT, int NS>
__global__ __launch_bounds__(256) void route_finalize_dispatch_kernel(
    const double *__restrict__ part, int splits, int T, int E, int k, int norm, int nbits,
    uint16_t *__restrict__ probs, int32_t *__restrict__ ids, uint16_t *__restrict__ scores,
    int32_t *__restrict__ offsets, int32_t *__restrict__ sorted, unsigned *__restrict__ done) {
  hoist_args(part, splits, T, E, k, norm, nbits, probs, ids, scores, offsets, sorted, done);
  extern __shared__ int lds[];
  __shared__ int s_last;
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (t < T) {
    int id;
    uint16_t sc;
    finalize_token<DT, NS>(part, splits, t, E, k, norm, probs, id, sc);
    if (lane < k) {
      ids[(int64_t)t * k + lane] = id;
      scores[(int64_t)t * k + lane] = sc;
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    __threadfence();  // this block's ids are visible before it is counted
    s_last = atomicAdd(done, 1u) == gridDim.x - 1;
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();  // every block's ids are visible to the sort
  // one read of the ids into LDS serves both passes of the sort
  int *ids_lds = lds + 5 * E;
  for (int p = threadIdx.x; p < T * k; p += blockDim.x) ids_lds[p] = ids[p];
  __syncthreads();
  block_sort([&](int p) { return ids_lds[p]; }, T * k, E, nbits, lds, offsets, sorted);
}

constexpr int kFinSplits = 4;  // hidden splits of a rounded-logits block (its wavefronts)

struct RoutePlan {
  int eb, n_tt, n_eb, splits;
  int wpb = 1;  // wavefronts per item (in-block hidden splits)
};

// Work split of the router: expert tiles per wavefront and hidden splits
// chosen so that roughly 2048 wavefronts share the work.
RoutePlan route_plan(int64_t T, int64_t H, int64_t E) {
  RoutePlan p;
  const int64_t n_tt = (T + 15) / 16;
  p.eb = (T >= 256 && E >= 64) ? 4 : 1;
  p.n_tt = (int)n_tt;
  p.n_eb = (int)((E + 16 * p.eb - 1) / (16 * p.eb));
  p.splits = 1;
  // hidden slices of whole 128-column blocks (so every slice, and every
  // 256-column batch inside it, starts on a quantisation group of 64 or 128:
  // the partial kernel takes a chunk's group from its offset in the batch), at
  // most kMaxSplits of them; about 2048 wavefronts share the work
  const int64_t blocks128 = H / 128;
  while (p.splits * 2 <= kMaxSplits && H % 128 == 0 && blocks128 % (p.splits * 2) == 0 &&
         n_tt * p.n_eb * p.splits * 2 <= 2048)
    p.splits *= 2;
  return p;
}

// Decode batches whose routing the gate/up product finalises (its prologue
// reads every partial of every token, so few partials per logit): one block
// per (token tile, expert tile, output split), whose wpb wavefronts split the
// hidden range again in whole 128-column blocks; 16 sub-splits in all where
// H allows, at most 8 per block.
RoutePlan decode_route_plan(int64_t T, int64_t H, int64_t E) {
  RoutePlan p;
  p.eb = 1;
  p.n_tt = (int)((T + 15) / 16);
  p.n_eb = (int)((E + 15) / 16);
  int n = 1;
  const int64_t blocks128 = H % 128 == 0 ? H / 128 : 1;
  while (n * 2 <= kMaxSplits && blocks128 % (n * 2) == 0) n *= 2;
  p.wpb = n < kMaxBlockSplits ? n : kMaxBlockSplits;
  p.splits = n / p.wpb;
  return p;
}

template <int DT, int EB>
hipError_t launch_mfma_t(const void *x, int64_t T, int64_t H, const uint32_t *wr, const void *sr,
                         const void *br, int64_t E, int gs, const RoutePlan &p, double *partial,
                         void *fin, unsigned *done, hipStream_t st) {
  const bool in_block = p.wpb > 1;
  const int64_t items = (int64_t)p.n_tt * p.n_eb * p.splits;
  dim3 grid((unsigned)(in_block ? items : (items + 3) / 4));
  dim3 block(in_block ? 64 * p.wpb : 256);
  const size_t lds = in_block ? sizeof(double) * p.wpb * EB * 4 * 64 : 0;
  const int64_t KR = H / (p.splits * p.wpb);
  // 8-byte scale loads (the four values from the batch's first group on)
  // need that group's value to start a dword in every row: an even group
  // index at every batch start (a batch of fewer than four groups reads
  // values past its range and leaves them unused; past the tensor's end the
  // load reads zeros)
  const int64_t gpr = H / gs;
  const int sb_vec = gpr % 2 == 0 && KR % (2 * gs) == 0;
  if (sb_vec)
    hipLaunchKernelGGL((route_mfma_kernel<DT, EB, true>), grid, block, lds, st,
                       (const uint16_t *)x, (int)T, (int)H, wr, (const uint16_t *)sr,
                       (const uint16_t *)br, (int)E, gs, (int)KR, p.n_tt, p.n_eb, p.splits, p.wpb,
                       partial, (uint16_t *)fin, done);
  else
    hipLaunchKernelGGL((route_mfma_kernel<DT, EB, false>), grid, block, lds, st,
                       (const uint16_t *)x, (int)T, (int)H, wr, (const uint16_t *)sr,
                       (const uint16_t *)br, (int)E, gs, (int)KR, p.n_tt, p.n_eb, p.splits, p.wpb,
                       partial, (uint16_t *)fin, done);
  return hipGetLastError();
}

template <int DT>
hipError_t launch_route_t(const void *x, int64_t T, int64_t H, const uint32_t *wr, const void *sr,
                          const void *br, int64_t E, int gs, const RoutePlan &p, double *partial,
                          void *fin, unsigned *done, hipStream_t st) {
  return p.eb == 4 ? launch_mfma_t<DT, 4>(x, T, H, wr, sr, br, E, gs, p, partial, fin, done, st)
                   : launch_mfma_t<DT, 1>(x, T, H, wr, sr, br, E, gs, p, partial, fin, done, st);
}

}  // namespace

int route_splits(int64_t T, int64_t H, int64_t E) {
  return route_i8_applies(T, H) ? route_i8_splits(T, H, E) : route_plan(T, H, E).splits;
}

int route_workspace_splits(int64_t T, int64_t H, int64_t E) {
  const int f = route_plan(T, H, E).splits;
  return H % 64 == 0 ? std::max(f, route_i8_splits(T, H, E)) : f;
}

int decode_route_splits(int64_t T, int64_t H, int64_t E) {
  return decode_route_plan(T, H, E).splits;
}

hipError_t launch_route_partial_decode(int dtype, const void *x, int64_t T, int64_t H,
                                       const uint32_t *wr, const void *sr, const void *br,
                                       int64_t E, int gs, double *partial, hipStream_t st) {
  const RoutePlan p = decode_route_plan(T, H, E);
  return dtype == DT_BF16
             ? launch_mfma_t<DT_BF16, 1>(x, T, H, wr, sr, br, E, gs, p, partial, nullptr, nullptr, st)
             : launch_mfma_t<DT_F16, 1>(x, T, H, wr, sr, br, E, gs, p, partial, nullptr, nullptr, st);
}

hipError_t launch_route_partial(int dtype, const void *x, int64_t T, int64_t H,
                                const uint32_t *wr, const void *sr, const void *br, int64_t E,
                                int gs, bool final_act, double *partial, void *fin,
                                unsigned *done, hipStream_t st) {
  if (!final_act && route_i8_applies(T, H))
    return launch_route_i8(dtype, x, T, H, wr, sr, br, E, gs, partial, done, st);
  RoutePlan p = route_plan(T, H, E);
  // rounded logits: the four wavefronts of a block split the hidden range
  // when it is whole 128-column blocks per split
  if (final_act) {
    p.splits = 1;
    p.wpb = H % (128 * kFinSplits) == 0 ? kFinSplits : 1;
  }
  return dtype == DT_BF16
             ? launch_route_t<DT_BF16>(x, T, H, wr, sr, br, E, gs, p, partial, fin, done, st)
             : launch_route_t<DT_F16>(x, T, H, wr, sr, br, E, gs, p, partial, fin, done, st);
}

bool route_fused_dispatch(int64_t T, int k) { return T <= kFusedRouteTokens && T * k <= kSortChunk; }

bool fused_route_supports(int64_t T, int64_t E, int k) {
  return T >= 1 && T <= kFusedRouteTokens && T * k <= kFusedPairs && E <= kRowExperts &&
         k <= kRowTopK;
}

namespace {

template <int DT, int NS>
void launch_fin_dispatch(const double *partial, int splits, int64_t T, int64_t E, int k, int norm,
                         int nbits, void *probs, int32_t *ids, void *scores, int32_t *offsets,
                         int32_t *sorted, unsigned *done, hipStream_t st) {
  // block_sort: (4 wavefronts + 1) * E, then the T*k ids
  const size_t lds = sizeof(int) * (size_t)(5 * E + T * k);
  hipLaunchKernelGGL((route_finalize_dispatch_kernel<DT, NS>), dim3((unsigned)((T + 3) / 4)),
                     dim3(256), lds, st, partial, splits, (int)T, (int)E, k, norm, nbits,
                     (uint16_t *)probs, ids, (uint16_t *)scores, offsets, sorted, done);
}

template <int DT, int NS>
void launch_fin(const double *partial, int splits, int64_t T, int64_t E, int k, int norm,
                void *probs, int32_t *ids, void *scores, hipStream_t st) {
  hipLaunchKernelGGL((route_finalize_kernel<DT, NS>), dim3((unsigned)((T + 3) / 4)), dim3(256), 0,
                     st, partial, splits, (int)T, (int)E, k, norm, (uint16_t *)probs, ids,
                     (uint16_t *)scores);
}

// Slots of 64 experts per lane: the smallest of 1, 2, 4, 8 covering E.
template <int DT, template <int, int> class F, class... Args>
void by_slots(int64_t E, Args... args) {
  if (E <= 64)
    F<DT, 1>::run(args...);
  else if (E <= 128)
    F<DT, 2>::run(args...);
  else if (E <= 256)
    F<DT, 4>::run(args...);
  else
    F<DT, 8>::run(args...);
}

template <int DT, int NS>
struct FinDispatch {
  template <class... Args>
  static void run(Args... args) { launch_fin_dispatch<DT, NS>(args...); }
};
template <int DT, int NS>
struct Fin {
  template <class... Args>
  static void run(Args... args) { launch_fin<DT, NS>(args...); }
};

}  // namespace

hipError_t launch_route_finalize_dispatch(int dtype, const double *partial, int splits, int64_t T,
                                          int64_t E, int k, int norm, void *probs, int32_t *ids,
                                          void *scores, int32_t *offsets, int32_t *sorted,
                                          unsigned *done, hipStream_t st) {
  int nbits = 0;
  while ((1ll << nbits) < E) ++nbits;
  if (dtype == DT_BF16)
    by_slots<DT_BF16, FinDispatch>(E, partial, splits, T, E, k, norm, nbits, probs, ids, scores,
                                   offsets, sorted, done, st);
  else
    by_slots<DT_F16, FinDispatch>(E, partial, splits, T, E, k, norm, nbits, probs, ids, scores,
                                  offsets, sorted, done, st);
  return hipGetLastError();
}

hipError_t launch_route_finalize(int dtype, const double *partial, int splits, int64_t T,
                                 int64_t E, int k, int norm, void *probs, int32_t *ids,
                                 void *scores, hipStream_t st) {
  if (dtype == DT_BF16)
    by_slots<DT_BF16, Fin>(E, partial, splits, T, E, k, norm, probs, ids, scores, st);
  else
    by_slots<DT_F16, Fin>(E, partial, splits, T, E, k, norm, probs, ids, scores, st);
  return hipGetLastError();
}

}  // namespace nvm
