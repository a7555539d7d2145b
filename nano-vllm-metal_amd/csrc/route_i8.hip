// Router partial logits of prefill-sized batches on the int8 matrix cores,
// exactly.
//
// Restates the router GEMV of route_topk (layers/moe.py:37-49 ->
// layers/linear.py:92-126 -> metal/src/quantized_matmul.cpp:117-145) with
// the same values as the float64 kernel (route.hip): every partial logit is
// the exact sum  sum_h x[t,h] * (s[e,g] q[e,h] + b[e,g])  over its hidden
// range, held in float64.
//
// Exactness.  A 64-wide k-step lies in one quantisation group (group sizes 64
// and 128), so its contribution to logit (t, e) is
//     s[e,g] * sum_h x_h q_h  +  b[e,g] * sum_h x_h.
// An activation is x = +-M 2^(en - BIAS) with an integer significand M of P
// bits (bf16 8, fp16 11).  For a band of exponents [lo, lo + W], W = 30 - P,
// every x of the band is X 2^(lo - BIAS) with the integer X = +-M << (en - lo),
// |X| < 2^30.  X has four balanced base-256 digits d0..d3 (each in
// [-128, 127]: the bytes of (X + 0x80808080) xor 0x80808080), so
//     sum_h X_h q_h = S0 + 2^8 S1 + 2^16 S2 + 2^24 S3,  S_d = sum_h d_d,h q_h,
// and each S_d is one v_mfma_i32_16x16x64_i8 (int8 digits against the int8
// codes 0..15; |S_d| < 2^17, exact in int32).  sum_h X_h comes the same way
// against a column of ones.  The digit sums are recombined in int32 and
// float64 without rounding (|sum X q| < 2^40), scaled by the power of two
// 2^(lo - BIAS) and by s and b (8 or 11 significant bits: products below 2^52,
// exact), and accumulated in float64 -- the sums the float64 kernel forms, and
// like them exact while a logit's terms span fewer than 53 bits.
//
// Bands.  A wavefront takes the largest exponent among its 16 tokens' 64
// activations of the k-step and covers the W + 1 exponents below it; the
// values below that band (rare: |x| under 2^-22 of the largest) take further
// passes with their own band, until every nonzero activation is covered.
// Zeros need no pass.  Activations must be finite.
//
// Work.  A block of four wavefronts owns 16 tokens, 64 experts and one hidden
// split; its wavefronts split the split's k-steps (each k-step's operands
// requested one k-step ahead), every wavefront covers the block's 64 experts
// (four 16-expert tiles, the digits of a k-step shared by all of them), and
// their float64 partials meet in LDS.  Output: partial [T][E][splits], the
// layout the finalise kernels read.
#include <cstdlib>
#include <type_traits>

#include "common.h"
#include "finalize.h"
#include "internal.h"

namespace nvm {

namespace {

constexpr int kI8Waves = 4;     // wavefronts per block (hidden sub-splits)
constexpr int kI8Tiles = 4;     // 16-expert tiles per block (64 experts)
constexpr int kI8MaxSplits = 16;
// scales and biases of a block's experts over its hidden split, staged in LDS:
// at most kSbGroups groups a row (kSbDw dwords, the first aligned down)
constexpr int kSbGroups = 64;
constexpr int kSbDw = kSbGroups / 2 + 1;

typedef int i32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ i32x4 mfma_i8(u32x4 a, u32x4 b) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4, a),
                                               __builtin_bit_cast(i32x4, b),
                                               i32x4{0, 0, 0, 0}, 0, 0, 0);
}

// sum_d 2^(8d) S_d of four digit sums, exactly (|result| < 2^53)
__device__ __forceinline__ double digits_value(int s0, int s1, int s2, int s3) {
  const int lo = s0 + (s1 << 8), hi = s2 + (s3 << 8);  // each below 2^25 in magnitude
  return fma((double)hi, 65536.0, (double)lo);
}

// Block-cooperative: the scales and biases of experts [e0, e0 + 64) for the
// groups [g0, g1) into s_sb, staged once per block: row e holds the dwords
// from the one containing its group g0 (one 16-bit value, two to a dword)
// on, scales first, then biases kSbArr bytes on.  (Per-lane 2-byte loads per
// k-step would move a 64-byte line for every value.)  Rows past E read zeros.
constexpr int kSbArr = 16 * kI8Tiles * kSbDw * 4;  // bytes of one array
__device__ __forceinline__ void i8_stage_sb(rsrc_t srr, rsrc_t brr, int e0, int GPR, int g0, int g1,
                                            uint8_t *s_sb, int tid, int nthreads) {
  const int nd = (g1 - g0 + 2) / 2;  // dwords a row (<= kSbDw)
  for (int it = tid; it < 2 * 16 * kI8Tiles * nd; it += nthreads) {
    const int arr = it / (16 * kI8Tiles * nd), rem = it - arr * 16 * kI8Tiles * nd;
    const int e = rem / nd, d = rem - e * nd;
    const int base = ((e0 + e) * GPR + g0) & ~1;
    *(uint32_t *)(s_sb + arr * kSbArr + (e * kSbDw + d) * 4) =
        bload4(arr ? brr : srr, (base + 2 * d) * 2, 0);
  }
}

// One wavefront's exact float64 sums over k-steps [k0, k1) for 16 tokens and
// the 64 experts from e0: acc[j][i] is token (row) 4G + i of expert e0 + 16 j
// + c (lane (c, G)).  Lane (c, G) supplies the A operand of token row c: its
// activations at byte offset xo (kMaskedOffset past T) of x, hidden columns
// 16G..16G+15 of each k-step.  s_sb: the staged scales and biases from group
// g0.  With xh (bf16 activations), the lane also stores its activations
// converted to fp16 as act_to_f16 does, at xh + xo / 2 (xh_ok: a real token),
// and the k-step's group shift at xsh_row[ks] (xsh_row: the token's row of
// shifts).
template <int DT>
__device__ __forceinline__ void i8_wave_sums(rsrc_t xr, rsrc_t wrr, int xo, int e0, int HW, int gs,
                                             int GPR, int g0, int k0, int k1,
                                             const uint8_t *s_sb, double (&acc)[kI8Tiles][4],
                                             uint16_t *xh, bool xh_ok, uint8_t *xsh_row) {
  using A = Act<DT>;
  constexpr bool BF = DT == DT_BF16;
  constexpr int MB = BF ? 7 : 10;  // stored significand bits
  // lsb exponent of the source format's subnormals (bf16 2^-133, fp16 2^-24):
  // a band with Lb at or below it holds every smaller activation exactly
  constexpr int kLbAll = BF ? -133 : -24;
  const int lane = threadIdx.x & 63, c = lane & 15, G = lane >> 4;
  const u32x4 ones = {0x01010101u, 0x01010101u, 0x01010101u, 0x01010101u};
  // B operand / output column of tile j: expert e0 + 16 j + c (codes of
  // hidden columns 16G..16G+15 of the k-step: two packed words).  Experts
  // past E lie beyond the descriptor's range and read zeros.
  const int wo = ((e0 + c) * HW + 2 * G) * 4;
  // this lane's value of group g, tile j: 16 bits at sbo[j] + 2 g (scales;
  // biases kSbArr further)
  int sbo[kI8Tiles];
#pragma unroll
  for (int j = 0; j < kI8Tiles; ++j) {
    const int e = 16 * j + c;
    sbo[j] = (e * kSbDw) * 4 + 2 * ((((e0 + e) * GPR + g0) & 1) - g0);
  }
#pragma unroll
  for (int j = 0; j < kI8Tiles; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[j][i] = 0.0;

  // one k-step's operands, requested a k-step ahead of their use
  struct Step {
    u32x4 xv[2];
    u32x2 wq[kI8Tiles];
  };
  auto load = [&](Step &st, int ks) {
    const int ku = __builtin_amdgcn_readfirstlane(ks);
    st.xv[0] = bload16(xr, xo, 128 * ku);
    st.xv[1] = bload16(xr, xo + 16, 128 * ku);
#pragma unroll
    for (int j = 0; j < kI8Tiles; ++j) st.wq[j] = bload8(wrr, wo + j * 64 * HW, 32 * ku);
  };
  Step nx;
  if (k0 < k1) load(nx, k0);
  for (int ks = k0; ks < k1; ++ks) {
    const Step cu = nx;
    // the next k-step's operands (the last k-step requests its own again)
    load(nx, ks + 1 < k1 ? ks + 1 : ks);
    const u32x4 (&xv)[2] = cu.xv;
    const u32x2 (&wq)[kI8Tiles] = cu.wq;
    if constexpr (BF) {
      if (xh) {
        // the fp16 copy of this lane's 16 activations, each 16-byte chunk of
        // x0..x7 stored in the pair order (x0,x4)(x1,x5)(x2,x6)(x3,x7) the
        // prefill GEMM's MFMA operands use; the k-step's 64 values of token
        // row c (lanes c, c + 16, c + 32, c + 48) share one shift
        uint32_t m = max(bf16_absmax_bits(xv[0]), bf16_absmax_bits(xv[1]));
        m = max(m, (uint32_t)__shfl_xor((int)m, 16));
        m = max(m, (uint32_t)__shfl_xor((int)m, 32));
        const int sh = f16_shift_of(m);
        if (xh_ok) {
          u32x4 *dst = (u32x4 *)((uint8_t *)xh + (int64_t)xo + 128 * ks);
          dst[0] = bf16_to_f16_pairs(xv[0], sh);
          dst[1] = bf16_to_f16_pairs(xv[1], sh);
          if (G == 0) xsh_row[ks] = (uint8_t)sh;
        }
      }
    }
    const int g = (ks * 64) / gs;
    uint32_t sv[kI8Tiles], bv[kI8Tiles];
#pragma unroll
    for (int j = 0; j < kI8Tiles; ++j) {
      sv[j] = *(const uint16_t *)(s_sb + sbo[j] + 2 * g);
      bv[j] = *(const uint16_t *)(s_sb + kSbArr + sbo[j] + 2 * g);
    }
    // element i of A dword q (columns as in the codes below): the low (q
    // even) or high (q odd) half of dword i of xv[q / 2], as float32 (exact)
    auto xf = [&](int q, int i) -> float {
      const uint32_t d = xv[q >> 1][i];
      if constexpr (BF)
        return __uint_as_float((q & 1) ? (d & 0xFFFF0000u) : (d << 16));
      else
        return (float)__builtin_bit_cast(_Float16, (uint16_t)((q & 1) ? (d >> 16) : d));
    };
    // One band: the activations with |x| bits below `lim` (all: ~0) and at
    // least 2^(Lb + MB), as integers X = x 2^-Lb (exact, |X| < 2^30), where
    // the band's largest |x| is below 2^(Emax - 126) (float32 exponent field
    // Emax) and Lb = Emax - 156.  A band whose Lb is at most the source
    // format's subnormal exponent covers everything below it too.
    // (first: the band of the k-step's largest |x|, where nothing is covered
    // yet and lim is not consulted)
    auto band = [&](auto first, uint32_t lim, uint32_t mb) {
      constexpr bool kFirst = decltype(first)::value;
      const int Lb = max((int)(mb >> 23), 1) - 156;
      const bool all_in = Lb <= kLbAll;
      const float one = (float)(1u << MB);  // 2^MB: the smallest in-band |X| of a normal
      // the band's digits: ad[d] holds digit d of the four A dwords
      u32x4 ad[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint32_t zz[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float Xf = ldexpf(xf(q, i), -Lb);
          const bool in = (kFirst || (__float_as_uint(xf(q, i)) & 0x7FFFFFFFu) < lim) &&
                          (all_in || fabsf(Xf) >= one);
          const int X = in ? (int)Xf : 0;
          zz[i] = ((uint32_t)X + 0x80808080u) ^ 0x80808080u;
        }
        // 4x4 byte transpose: byte d of element i -> byte i of digit d
        const uint32_t t0 = __builtin_amdgcn_perm(zz[1], zz[0], 0x05010400u);
        const uint32_t t1 = __builtin_amdgcn_perm(zz[1], zz[0], 0x07030602u);
        const uint32_t t2 = __builtin_amdgcn_perm(zz[3], zz[2], 0x05010400u);
        const uint32_t t3 = __builtin_amdgcn_perm(zz[3], zz[2], 0x07030602u);
        ad[0][q] = __builtin_amdgcn_perm(t2, t0, 0x05040100u);
        ad[1][q] = __builtin_amdgcn_perm(t2, t0, 0x07060302u);
        ad[2][q] = __builtin_amdgcn_perm(t3, t1, 0x05040100u);
        ad[3][q] = __builtin_amdgcn_perm(t3, t1, 0x07060302u);
      }
      // sum_h X_h of the output rows' tokens (rows 4G..4G+3)
      i32x4 us[4];
#pragma unroll
      for (int d = 0; d < 4; ++d) us[d] = mfma_i8(ad[d], ones);
      double uf[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) uf[i] = digits_value(us[0][i], us[1][i], us[2][i], us[3][i]);
#pragma unroll
      for (int j = 0; j < kI8Tiles; ++j) {
        // codes as int8, in the element order of the A operand: dword 0
        // holds columns 0,2,4,6, dword 1 columns 1,3,5,7, dwords 2-3 the
        // same of 8..15 (the dot product only needs A and B in one order)
        const u32x4 bq = {wq[j].x & 0x0F0F0F0Fu, (wq[j].x >> 4) & 0x0F0F0F0Fu,
                          wq[j].y & 0x0F0F0F0Fu, (wq[j].y >> 4) & 0x0F0F0F0Fu};
        i32x4 sd[4];
#pragma unroll
        for (int d = 0; d < 4; ++d) sd[d] = mfma_i8(ad[d], bq);
        const double s2 = ldexp((double)A::to_f32(sv[j]), Lb);  // x = X 2^Lb
        const double b2 = ldexp((double)A::to_f32(bv[j]), Lb);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const double v = digits_value(sd[0][i], sd[1][i], sd[2][i], sd[3][i]);
          acc[j][i] = fma(s2, v, acc[j][i]);
          acc[j][i] = fma(b2, uf[i], acc[j][i]);
        }
        // one tile's digit sums live at a time
        __builtin_amdgcn_sched_barrier(0);
      }
      // below this band: |x| < 2^(Lb + MB), float32 exponent field under
      // Lb + MB + 127 (none when the band reached the subnormals)
      const int ef = Lb + MB + 127;
      return all_in || ef <= 0 ? 0u : (uint32_t)ef << 23;
    };
    // bands from the largest |x| down; one holds every activation of the
    // k-step unless some |x| is under 2^-22 of the largest (bf16)
    float amax = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int i = 0; i < 4; ++i) amax = fmaxf(amax, fabsf(xf(q, i)));
    const uint32_t mb0 = wave_max_u32(__float_as_uint(amax));
    uint32_t lim = mb0 ? band(std::true_type{}, 0u, mb0) : 0u;
    while (lim) {
      uint32_t mb = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t b = __float_as_uint(xf(q, i)) & 0x7FFFFFFFu;
          if (b < lim) mb = max(mb, b);
        }
      mb = wave_max_u32(mb);
      if (mb == 0) break;  // uniform over the wavefront
      lim = band(std::false_type{}, lim, mb);
    }
  }
}

// Partial logits [T][E][splits]: block (token tile, 64-expert range, hidden
// split), its four wavefronts splitting the split's k-steps.
template <int DT>
__global__ __launch_bounds__(64 * kI8Waves, 2) void route_i8_kernel(
    const uint16_t *__restrict__ x, int T, int H, const uint32_t *__restrict__ wr,
    const uint16_t *__restrict__ sr, const uint16_t *__restrict__ br, int E, int gs, int n_tt,
    int splits, double *__restrict__ part, unsigned *__restrict__ done) {
  hoist_args(x, T, H, wr, sr, br, E, gs, n_tt, splits, part, done);
  extern __shared__ double s_red[];  // [kI8Waves - 1][tile][row][lane], then the staged s/b
  // the finalising launch that follows counts its blocks from zero
  if (done && blockIdx.x == 0 && threadIdx.x == 0) *done = 0u;

  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane & 15, G = lane >> 4;
  const int n_ec = (E + 16 * kI8Tiles - 1) / (16 * kI8Tiles);
  const int tt = blockIdx.x % n_tt, ec = (blockIdx.x / n_tt) % n_ec;
  const int z = blockIdx.x / (n_tt * n_ec);
  const int e0 = ec * 16 * kI8Tiles;
  const int KS = H >> 6;
  // k-steps of split z, then this wavefront's share of them
  const int zs0 = z * KS / splits, zs1 = (z + 1) * KS / splits;
  const int k0 = zs0 + wv * (zs1 - zs0) / kI8Waves;
  const int k1 = zs0 + (wv + 1) * (zs1 - zs0) / kI8Waves;
  const int HW = H >> 3, GPR = H / gs;
  const rsrc_t xr = make_rsrc(x, (uint32_t)((int64_t)T * H * 2));
  const rsrc_t wrr = make_rsrc(wr, (uint32_t)((int64_t)E * HW * 4));
  const rsrc_t srr = make_rsrc(sr, (uint32_t)((int64_t)E * GPR * 2));
  const rsrc_t brr = make_rsrc(br, (uint32_t)((int64_t)E * GPR * 2));
  const int ta = tt * 16 + c;
  const int xo = ta < T ? ta * H * 2 + 32 * G : kMaskedOffset;

  uint8_t *s_sb = (uint8_t *)(s_red + (kI8Waves - 1) * kI8Tiles * 4 * 64);
  const int g0 = zs0 * 64 / gs, g1 = (zs1 * 64 + gs - 1) / gs;
  i8_stage_sb(srr, brr, e0, GPR, g0, g1, s_sb, threadIdx.x, 64 * kI8Waves);
  __syncthreads();
  double acc[kI8Tiles][4];
  i8_wave_sums<DT>(xr, wrr, xo, e0, HW, gs, GPR, g0, k0, k1, s_sb, acc, nullptr, false,
                   nullptr);

  // the wavefronts' partials meet in LDS, added in wavefront order
  // (a lane's slots are 512 bytes apart: compile-time offsets from one base)
  if (wv > 0) {
    double *mine = s_red + (wv - 1) * (kI8Tiles * 4 * 64) + lane;
#pragma unroll
    for (int j = 0; j < kI8Tiles; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) mine[(j * 4 + i) * 64] = acc[j][i];
  }
  __syncthreads();
  if (wv == 0) {
    const double *rd = s_red + lane;
#pragma unroll
    for (int j = 0; j < kI8Tiles; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        double v = acc[j][i];
#pragma unroll
        for (int w = 1; w < kI8Waves; ++w) v += rd[(((w - 1) * kI8Tiles + j) * 4 + i) * 64];
        const int t = tt * 16 + 4 * G + i, e = e0 + 16 * j + c;
        if (t < T && e < E) part[((int64_t)t * E + e) * splits + z] = v;
      }
  }
}

// The whole routing of 16 tokens in one block (E <= 128, k <= 16): 4 n_ec
// wavefronts (64-expert range ec = w / 4, hidden quarter w % 4) form the
// exact logit sums, which meet in LDS; four wavefronts finalise four tokens
// each as the decode kernels do (finalize_sums); the block stores the ids and
// scores [T][k] and its histogram counts[block][E] (pairs per expert, for
// dispatch_hist), and with xh the fp16 copy of its tokens' activations.
constexpr int kFinMaxWaves = 8;
template <int DT>
__global__ __launch_bounds__(64 * kFinMaxWaves) void route_i8_fin_kernel(
    const uint16_t *__restrict__ x, int T, int H, const uint32_t *__restrict__ wr,
    const uint16_t *__restrict__ sr, const uint16_t *__restrict__ br, int E, int gs, int k,
    int norm, int32_t *__restrict__ ids, uint16_t *__restrict__ scores,
    int32_t *__restrict__ counts, uint16_t *__restrict__ xh, uint8_t *__restrict__ xsh) {
  hoist_args(x, T, H, wr, sr, br, E, gs, k, norm, ids, scores, counts, xh, xsh);
  extern __shared__ double s_lds[];
  // [ec][quarter - 1][tile][row][lane] partials, then the logits [16][128],
  // then the staged s/b of each expert range
  constexpr int kSlots = 3 * kI8Tiles * 4 * 64;
  double *s_lg = s_lds + 2 * kSlots;
  uint8_t *s_sb0 = (uint8_t *)(s_lg + 16 * 128);
  __shared__ int s_ids[16 * kRowTopK];
  __shared__ uint16_t s_sc[16 * kRowTopK];
  __shared__ uint64_t s_mask[kRowExperts];

  const int tid = threadIdx.x, lane = tid & 63, nthr = blockDim.x;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15, G = lane >> 4;
  const int tt = blockIdx.x;
  const int ec = wv >> 2, qr = wv & 3;  // expert range, hidden quarter
  const int e0 = ec * 16 * kI8Tiles;
  const int KS = H >> 6;
  const int k0 = qr * KS / 4, k1 = (qr + 1) * KS / 4;
  const int HW = H >> 3, GPR = H / gs;
  const rsrc_t xr = make_rsrc(x, (uint32_t)((int64_t)T * H * 2));
  const rsrc_t wrr = make_rsrc(wr, (uint32_t)((int64_t)E * HW * 4));
  const rsrc_t srr = make_rsrc(sr, (uint32_t)((int64_t)E * GPR * 2));
  const rsrc_t brr = make_rsrc(br, (uint32_t)((int64_t)E * GPR * 2));
  const int ta = tt * 16 + c;
  const int xo = ta < T ? ta * H * 2 + 32 * G : kMaskedOffset;

  for (int e = tid; e < kRowExperts; e += nthr) s_mask[e] = 0ull;
  const int n_ec = nthr / (64 * 4);
  for (int r = 0; r < n_ec; ++r)
    i8_stage_sb(srr, brr, r * 16 * kI8Tiles, GPR, 0, GPR, s_sb0 + r * 2 * kSbArr, tid, nthr);
  __syncthreads();
  double acc[kI8Tiles][4];
  // (the first expert range's wavefronts write the fp16 copy)
  i8_wave_sums<DT>(xr, wrr, xo, e0, HW, gs, GPR, 0, k0, k1, s_sb0 + ec * 2 * kSbArr, acc,
                   ec == 0 ? xh : nullptr, ta < T,
                   xsh ? xsh + (int64_t)ta * KS : nullptr);

  // quarters 1-3 publish their sums; quarter 0 adds them in order and writes
  // the logit sums [token][expert]
  if (qr > 0) {
    double *mine = s_lds + ec * kSlots + (qr - 1) * (kI8Tiles * 4 * 64) + lane;
#pragma unroll
    for (int j = 0; j < kI8Tiles; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) mine[(j * 4 + i) * 64] = acc[j][i];
  }
  __syncthreads();
  if (qr == 0) {
    const double *rd = s_lds + ec * kSlots + lane;
#pragma unroll
    for (int j = 0; j < kI8Tiles; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        double v = acc[j][i];
#pragma unroll
        for (int w = 1; w < 4; ++w) v += rd[(((w - 1) * kI8Tiles + j) * 4 + i) * 64];
        s_lg[(4 * G + i) * 128 + e0 + 16 * j + c] = v;
      }
  }
  __syncthreads();
  // wavefront w < 4 finalises local tokens 4w..4w+3 (one per 16-lane row)
  if (wv < 4) {
    const int tl = 4 * wv + G;
    double sum[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) sum[j] = s_lg[tl * 128 + c + 16 * j];
    finalize_sums<DT>(sum, tl, tt * 16 + tl < T, E, k, norm, s_ids, s_sc, s_mask);
  }
  __syncthreads();
  const int nt = min(16, T - tt * 16);
  for (int i = tid; i < nt * k; i += nthr) {
    ids[(int64_t)tt * 16 * k + i] = s_ids[i];
    scores[(int64_t)tt * 16 * k + i] = s_sc[i];
  }
  for (int e = tid; e < E; e += nthr) counts[(int64_t)tt * E + e] = __popcll(s_mask[e]);
}

constexpr size_t kI8Lds = sizeof(double) * (kI8Waves - 1) * kI8Tiles * 4 * 64 + 2 * kSbArr;
// route_i8_fin_kernel: two ranges' partial slots, the logits, two ranges' s/b
constexpr size_t kFinLds =
    sizeof(double) * (2 * 3 * kI8Tiles * 4 * 64 + 16 * 128) + 2 * 2 * kSbArr;

}  // namespace

// Batches of at least 128 tokens (NVM_ROUTE_I8=0/1 overrides, for tests).
bool route_i8_applies(int64_t T, int64_t H) {
  if (H % 64 != 0 || (H / 64 + kI8MaxSplits - 1) / kI8MaxSplits + 1 > kSbGroups) return false;
  const char *v = getenv("NVM_ROUTE_I8");
  if (v && v[0] == '0') return false;
  if (v && v[0] == '1') return T > 0;
  return T >= 128;
}

// Hidden splits: about two blocks per compute unit, each wavefront at least
// one k-step where the hidden size allows.
int route_i8_splits(int64_t T, int64_t H, int64_t E) {
  const int64_t n_tt = (T + 15) / 16, KS = H / 64;
  const int64_t n_ec = (E + 16 * kI8Tiles - 1) / (16 * kI8Tiles);
  int s = 1;
  while (s * 2 <= kI8MaxSplits && s * 2 * kI8Waves <= KS && n_tt * n_ec * s < 2 * cu_count())
    s *= 2;
  // a split's groups fit the staged scale/bias rows (k-steps of 64 columns,
  // groups of 64 or 128: at most one group a k-step, one more when a split
  // starts inside a group)
  while (s < kI8MaxSplits && (KS + s - 1) / s + 1 > kSbGroups) s *= 2;
  return s;
}

bool route_i8_fin_supports(int64_t T, int64_t H, int64_t E, int gs, int k) {
  // (E a multiple of 4: the sort reads the histograms four experts at a time)
  return route_i8_applies(T, H) && gs % 64 == 0 && E <= 128 && E % 4 == 0 && k <= kRowTopK &&
         H / gs <= kSbGroups;
}

hipError_t launch_route_i8_fin(int dtype, const void *x, int64_t T, int64_t H, const uint32_t *wr,
                               const void *sr, const void *br, int64_t E, int gs, int k, int norm,
                               int32_t *ids, void *scores, int32_t *counts, void *xh,
                               uint8_t *xsh, hipStream_t st) {
  if (!route_i8_fin_supports(T, H, E, gs, k) || T <= 0) return hipErrorInvalidValue;
  if (xh && (dtype != DT_BF16 || !xsh)) return hipErrorInvalidValue;
  // more than 64 KB of dynamic LDS (once per device and dtype; a failure here
  // shows up as a failed launch below)
  static bool attr_set[2][64] = {};
  int dev = 0;
  const int di = dtype == DT_BF16 ? 1 : 0;
  if (hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64 && !attr_set[di][dev]) {
    (void)hipFuncSetAttribute(di ? (const void *)&route_i8_fin_kernel<DT_BF16>
                                 : (const void *)&route_i8_fin_kernel<DT_F16>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)kFinLds);
    attr_set[di][dev] = true;
  }
  const int n_tt = (int)((T + 15) / 16);
  const int n_ec = (int)((E + 16 * kI8Tiles - 1) / (16 * kI8Tiles));
  const dim3 grid((unsigned)n_tt), block(64 * 4 * n_ec);
  if (di)
    hipLaunchKernelGGL(route_i8_fin_kernel<DT_BF16>, grid, block, kFinLds, st, (const uint16_t *)x,
                       (int)T, (int)H, wr, (const uint16_t *)sr, (const uint16_t *)br, (int)E, gs,
                       k, norm, ids, (uint16_t *)scores, counts, (uint16_t *)xh, xsh);
  else
    hipLaunchKernelGGL(route_i8_fin_kernel<DT_F16>, grid, block, kFinLds, st, (const uint16_t *)x,
                       (int)T, (int)H, wr, (const uint16_t *)sr, (const uint16_t *)br, (int)E, gs,
                       k, norm, ids, (uint16_t *)scores, counts, nullptr, nullptr);
  return hipGetLastError();
}

hipError_t launch_route_i8(int dtype, const void *x, int64_t T, int64_t H, const uint32_t *wr,
                           const void *sr, const void *br, int64_t E, int gs, double *partial,
                           unsigned *done, hipStream_t st) {
  if (H % 64 != 0 || gs % 64 != 0 || T <= 0) return hipErrorInvalidValue;
  if ((H / 64 + kI8MaxSplits - 1) / kI8MaxSplits + 1 > kSbGroups) return hipErrorInvalidValue;
  const int n_tt = (int)((T + 15) / 16);
  const int n_ec = (int)((E + 16 * kI8Tiles - 1) / (16 * kI8Tiles));
  const int splits = route_i8_splits(T, H, E);
  const dim3 grid((unsigned)(n_tt * n_ec * splits)), block(64 * kI8Waves);
  if (dtype == DT_BF16)
    hipLaunchKernelGGL(route_i8_kernel<DT_BF16>, grid, block, kI8Lds, st, (const uint16_t *)x,
                       (int)T, (int)H, wr, (const uint16_t *)sr, (const uint16_t *)br, (int)E, gs,
                       n_tt, splits, partial, done);
  else
    hipLaunchKernelGGL(route_i8_kernel<DT_F16>, grid, block, kI8Lds, st, (const uint16_t *)x,
                       (int)T, (int)H, wr, (const uint16_t *)sr, (const uint16_t *)br, (int)E, gs,
                       n_tt, splits, partial, done);
  return hipGetLastError();
}

}  // namespace nvm
