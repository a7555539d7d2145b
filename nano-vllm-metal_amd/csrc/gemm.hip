// Prefill-regime grouped W4A16 expert products (many routed rows per expert).
//
// Replaces `mx.gather_qmm` inside grouped_expert_linear (layers/moe.py:21-32)
// for prefill-sized batches, with SwiGLU (layers/moe.py:84; silu op by op as
// layers/activation.py:21-24 evaluates it, silu_act) fused into the gate/up
// epilogue.  Work is a list of (expert, 128-row m-tile, n-tile)
// triples built on the device from the expert offsets (prefix sum of
// ceil(count_e / 128)), so no host synchronisation is needed and empty experts
// cost nothing.
//
// A tile is 128 routed rows x 256 weight rows (gate/up: 128 columns of each
// matrix; down: 256 columns).  Per 64-wide k-step the block stages the
// gathered activation rows (bf16/fp16) and the *packed* int4 weight rows in
// LDS, double-buffered, with the next k-step's global loads in flight during
// the current k-step's MFMAs.  The four wavefronts split the tile along N: a
// wavefront owns 2 x 32 weight rows (gate/up: the same 32 columns of both
// matrices, so the SwiGLU pair lands in one lane) and all 128 routed rows
// (4 x 2 tiles of v_mfma_f32_32x32x16).  Each weight word is dequantised once
// per tile, in registers, right before its MFMA.
//
// Operands are fp16 for both activation dtypes.  A weight q*s + b (s, b of
// 8 or 11 significant bits, q of 4) needs about 12 significant bits: rounded
// to bf16 it would carry a 2^-9 relative error, which at the 235B-A22B shape
// alone makes a mean output error above 1e-3 against the exact products;
// rounded to fp16 (one v_pk_fma_f16, single rounding) the error is 2^-12 and
// the outputs are those of exact weights.  bf16 activations convert to fp16
// exactly in fp16's range (|x| <= 65504; post-norm activations are far
// inside it), and the fp16 MFMA runs at the bf16 rate.
//
// k-order inside a k-step: MFMA chunk c (16 wide) and lane half h cover
// the eight k = 8*(4h + c) + i, i = 0..7, in both operands, in the slot
// order i = 0,4,1,5,2,6,3,7 that the nibble expansion of one packed word
// produces.  A lane's B operand for chunk c is then packed word 4h + c of its
// weight row (one 16-byte LDS read serves all four chunks) and its A operand
// is the 16 bytes at offset 16*(4h + c) of the activation row, which staging
// stores in that slot order.
#include "common.h"
#include "internal.h"

namespace nvm {

namespace {

constexpr int BM = kGemmBM;       // routed rows per tile
constexpr int WROWS = 256;        // weight rows per tile
constexpr int BK = 64;            // k per stage
constexpr int A_PITCH = 144;      // bytes per staged activation row (128 + 16 pad)
constexpr int B_PITCH = 48;       // bytes per staged weight row (32 + 16 pad)
constexpr int A_STAGE = BM * A_PITCH;
constexpr int B_STAGE = WROWS * B_PITCH;
constexpr int STAGE = A_STAGE + B_STAGE;
constexpr int kGemmLds = 2 * STAGE;

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pk_fma_h(uint32_t a, uint32_t b, uint32_t c) {  // v_pk_fma_f16
  return __builtin_bit_cast(uint32_t,
                            __builtin_elementwise_fma(__builtin_bit_cast(h2_t, a),
                                                      __builtin_bit_cast(h2_t, b),
                                                      __builtin_bit_cast(h2_t, c)));
}
__device__ __forceinline__ uint32_t pk_add_h(uint32_t a, uint32_t b) {  // v_pk_add_f16
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2_t, a) + __builtin_bit_cast(h2_t, b));
}

// One packed word (codes q0..q7, q_i at bits 4i) -> the 8 weights q_i*s + b
// as fp16, each the correctly rounded value of the exact q*s + b (one
// v_pk_fma_f16 per pair, single rounding), in the pair order
// (q0,q4)(q1,q5)(q2,q6)(q3,q7): the codes become the exact fp16 values
// 1024 + q by OR-ing them into the mantissa of 1024.0 (whose ulp is 1) and
// 1024 is then taken off exactly.  s2, b2: (s, s) and (b, b) as fp16 pairs.
__device__ __forceinline__ u32x4 dequant8_h(uint32_t w, uint32_t s2, uint32_t b2, uint32_t mask,
                                            uint32_t magic) {
  u32x4 d = nibble_pairs_v<0>(w, mask, magic);
#pragma unroll
  for (int i = 0; i < 4; ++i) d[i] = pk_fma_h(pk_add_h(d[i], 0xE400E400u), s2, b2);
  return d;
}

// Eight consecutive activations x0..x7 (one 16-byte chunk of a row) -> fp16
// in the pair order (x0,x4)(x1,x5)(x2,x6)(x3,x7) of dequant8_h.  bf16 values
// convert exactly (fp16 carries more significand bits) within fp16's range;
// v_cvt_pkrtz_f16_f32 only rounds below it (|x| < 2^-14, with a contribution
// far under the product's rounding) and saturates above 65504.
template <int DT>
__device__ __forceinline__ u32x4 act_to_h(u32x4 v) {
  if constexpr (DT == DT_F16) {
    return pair_order(v);
  } else {
    u32x4 o;
    const float x0 = __uint_as_float(v.x << 16), x1 = __uint_as_float(v.x & 0xFFFF0000u);
    const float x2 = __uint_as_float(v.y << 16), x3 = __uint_as_float(v.y & 0xFFFF0000u);
    const float x4 = __uint_as_float(v.z << 16), x5 = __uint_as_float(v.z & 0xFFFF0000u);
    const float x6 = __uint_as_float(v.w << 16), x7 = __uint_as_float(v.w & 0xFFFF0000u);
    o.x = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(x0, x4));
    o.y = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(x1, x5));
    o.z = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(x2, x6));
    o.w = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(x3, x7));
    return o;
  }
}

// A scale or bias (act bits) as the fp16 pair (v, v); bf16 values convert
// with round to nearest even (exactly, inside fp16's normal range).
template <int DT>
__device__ __forceinline__ uint32_t sb_pair_h(uint32_t bits) {
  uint32_t h;
  if constexpr (DT == DT_F16)
    h = bits & 0xFFFFu;
  else
    h = __builtin_bit_cast(uint16_t, (_Float16)__uint_as_float(bits << 16));
  return h | (h << 16);
}

__device__ __forceinline__ f32x16 mfma32_h(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

template <int DT, bool DUAL>
__global__ __launch_bounds__(256, 2) void gemm_kernel(const GroupedArgs a, int n_tiles) {
  using A = Act<DT>;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ int s_arow[BM];
  __shared__ int s_orow[BM];
  __shared__ int s_tiles[kMaxExperts + 1];

  hoist_args(a.act, a.act_ld, a.act_rows, a.a_map, a.a_div, a.offsets, a.w0, a.s0, a.b0, a.w1,
             a.s1, a.b1, a.R, a.K, a.gs, a.E, a.out, a.o_map, a.out_ld, n_tiles);
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int l32 = lane & 31, h = lane >> 5;

  // m-tile list: exclusive prefix over experts of ceil(count / BM), built by
  // wavefront 0 from the expert offsets (E <= kMaxExperts)
  // expert slot offsets (none: one expert over all act_rows rows, the dense
  // product)
  auto offs = [&](int i) { return a.offsets ? a.offsets[i] : (i == 0 ? 0 : (int)a.act_rows); };
  if (wv == 0) {
    int carry = 0;
    for (int c0 = 0; c0 < a.E; c0 += 64) {
      const int e = c0 + lane;
      const int tv = e < a.E ? (offs(e + 1) - offs(e) + BM - 1) / BM : 0;
      int inc = tv;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int u = __shfl_up(inc, o);
        if (lane >= o) inc += u;
      }
      if (e < a.E) s_tiles[e] = carry + inc - tv;
      carry += __shfl(inc, 63);
    }
    if (lane == 0) s_tiles[a.E] = carry;
  }
  __syncthreads();

  // Workgroups are dealt to the 8 XCDs round-robin by id; give each XCD a
  // contiguous range of (m-tile, n-tile) pairs so the tiles sharing activation
  // rows (same m-tile) and weights (same expert and n-tile) share an L2.
  const int total = s_tiles[a.E] * n_tiles;
  const int per_xcd = (total + 7) >> 3;
  const int local = blockIdx.x >> 3;
  if (local >= per_xcd) return;
  const int t = (blockIdx.x & 7) * per_xcd + local;
  if (t >= total) return;
  const int mt = t / n_tiles, nt = t - mt * n_tiles;

  // largest expert whose first tile is <= mt (skips experts with no tiles)
  int lo = 0, hi = a.E - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (s_tiles[mid] <= mt)
      lo = mid;
    else
      hi = mid - 1;
  }
  const int e = lo;
  const int m0 = offs(e) + (mt - s_tiles[e]) * BM;
  const int mcnt = min(BM, offs(e + 1) - m0);
  const int R = a.R, KW = a.K >> 3, GPR = a.K / a.gs;
  const int n0 = nt * (DUAL ? WROWS / 2 : WROWS);

  for (int i = tid; i < BM; i += 256) {
    const int slot = m0 + i;
    s_arow[i] = i < mcnt ? (a.a_map ? a.a_map[slot] / a.a_div : slot) : -1;
    s_orow[i] = i < mcnt ? (a.o_map ? a.o_map[slot] : slot) : -1;
  }
  __syncthreads();

  // ---- descriptors and per-thread offsets of the staging loads
  const rsrc_t ra = make_rsrc(a.act, (uint32_t)(a.act_rows * a.act_ld * 2));
  const int64_t eoff = (int64_t)e * R;
  const rsrc_t rw0 = make_rsrc(a.w0 + eoff * KW, (uint32_t)R * KW * 4);
  const rsrc_t rw1 = make_rsrc((DUAL ? a.w1 : a.w0) + eoff * KW, (uint32_t)R * KW * 4);
  const rsrc_t rs0 = make_rsrc(a.s0 + eoff * GPR, (uint32_t)R * GPR * 2);
  const rsrc_t rb0 = make_rsrc(a.b0 + eoff * GPR, (uint32_t)R * GPR * 2);
  const rsrc_t rs1 = make_rsrc((DUAL ? a.s1 : a.s0) + eoff * GPR, (uint32_t)R * GPR * 2);
  const rsrc_t rb1 = make_rsrc((DUAL ? a.b1 : a.b0) + eoff * GPR, (uint32_t)R * GPR * 2);

  // activations: thread loads rows (tid >> 3) + 32c, 16-byte chunk tid & 7
  int a_voff[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int ar = s_arow[(tid >> 3) + 32 * c];
    a_voff[c] = ar >= 0 ? (int)(((int64_t)ar * a.act_ld) * 2) + 16 * (tid & 7) : kMaskedOffset;
  }
  // packed weights: thread loads staged rows (tid >> 1) + 128c, half tid & 1
  int b_voff[2];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int wrow = (tid >> 1) + 128 * c;
    const int grow = DUAL ? n0 + (wrow & 127) : n0 + wrow;
    b_voff[c] = grow < R ? grow * KW * 4 + 16 * (tid & 1) : kMaskedOffset;
  }
  // this lane's two weight rows (sub 0/1) for the scale/bias loads and reads
  int srow[2], lrow[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    lrow[s] = DUAL ? 128 * s + 32 * wv + l32 : 64 * wv + 32 * s + l32;
    const int grow = DUAL ? n0 + 32 * wv + l32 : n0 + 64 * wv + 32 * s + l32;
    srow[s] = grow < R ? grow * GPR * 2 : kMaskedOffset;
  }

  const int nk = a.K / BK;
  // Global loads of one k-step, issued two k-steps ahead into one of two
  // register sets.  Every issue makes the same loads; k-steps past the end
  // read through masked offsets (zeros, no traffic), so the wait counts are
  // the same on every path.
  struct Stage {
    u32x4 a[4], b[2];
    uint32_t s[2], z[2];
  };
  auto issue = [&](Stage &g, int ks) {
    const bool ok = ks < nk;
    const int k0 = ok ? ks * BK : 0;
    const int sa = __builtin_amdgcn_readfirstlane(k0 * 2);
    const int sb = __builtin_amdgcn_readfirstlane(k0 >> 1);
    const int sg = __builtin_amdgcn_readfirstlane((k0 / a.gs) * 2);
#pragma unroll
    for (int c = 0; c < 4; ++c) g.a[c] = bload16(ra, ok ? a_voff[c] : kMaskedOffset, sa);
    g.b[0] = bload16(rw0, ok ? b_voff[0] : kMaskedOffset, sb);
    g.b[1] = bload16(rw1, ok ? b_voff[1] : kMaskedOffset, sb);
    g.s[0] = bload2(rs0, ok ? srow[0] : kMaskedOffset, sg);
    g.z[0] = bload2(rb0, ok ? srow[0] : kMaskedOffset, sg);
    g.s[1] = bload2(rs1, ok ? srow[1] : kMaskedOffset, sg);
    g.z[1] = bload2(rb1, ok ? srow[1] : kMaskedOffset, sg);
  };
  auto store = [&](const Stage &g, int buf) {
    uint8_t *As = smem + buf * STAGE;
    uint8_t *Bs = As + A_STAGE;
#pragma unroll
    for (int c = 0; c < 4; ++c)
      *(u32x4 *)(As + ((tid >> 3) + 32 * c) * A_PITCH + 16 * (tid & 7)) = act_to_h<DT>(g.a[c]);
#pragma unroll
    for (int c = 0; c < 2; ++c)
      *(u32x4 *)(Bs + ((tid >> 1) + 128 * c) * B_PITCH + 16 * (tid & 1)) = g.b[c];
  };

  f32x16 acc[2][4];
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[s][i][r] = 0.f;

  // this k-step's scale and bias of the lane's two weight rows, fp16 pairs
  uint32_t sc[2], bi[2];
  auto take_sb = [&](const Stage &g) {
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      sc[s] = sb_pair_h<DT>(g.s[s]);
      bi[s] = sb_pair_h<DT>(g.z[s]);
    }
  };
  // nibble-expansion constants in registers (one v_and_or_b32 per dword)
  const uint32_t nib_mask = sgpr_const(0x000F000Fu);
  const uint32_t magic = vgpr_const(0x64006400u);  // fp16 (1024, 1024)
  // Software-pipelined over the four 16-wide chunks: the A reads and the
  // dequantisation of chunk c + 1 are issued ahead of chunk c's MFMAs.
  auto compute = [&](int buf) {
    const uint8_t *As = smem + buf * STAGE;
    const uint8_t *Bs = As + A_STAGE;
    u32x4 bw[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) bw[s] = *(const u32x4 *)(Bs + lrow[s] * B_PITCH + 16 * h);
    auto load_a = [&](int c, u32x4 (&af)[4]) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        af[i] = *(const u32x4 *)(As + (32 * i + l32) * A_PITCH + 16 * (4 * h + c));
    };
    auto deq = [&](int c, u32x4 (&bf)[2]) {
#pragma unroll
      for (int s = 0; s < 2; ++s) bf[s] = dequant8_h(bw[s][c], sc[s], bi[s], nib_mask, magic);
    };
    u32x4 af[4], bf[2];
    load_a(0, af);
    deq(0, bf);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      u32x4 afn[4], bfn[2];
      if (c < 3) {
        load_a(c + 1, afn);
        deq(c + 1, bfn);
      }
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[s][i] = mfma32_h(af[i], bf[s], acc[s][i]);
      if (c < 3) {
#pragma unroll
        for (int i = 0; i < 4; ++i) af[i] = afn[i];
        bf[0] = bfn[0];
        bf[1] = bfn[1];
      }
    }
  };

  // k-step ks computes LDS buffer ks & 1 while the loads of ks + 2 are in
  // flight in the register set that held ks; then ks + 1 (issued a k-step
  // earlier) is stored into the other buffer.  Two k-steps per loop trip keep
  // the register sets static.
  Stage g0, g1;
  issue(g0, 0);
  issue(g1, 1);
  store(g0, 0);
  take_sb(g0);
  __syncthreads();
  auto step = [&](int ks, Stage &gi, Stage &gs) {
    issue(gi, ks + 2);
    compute(ks & 1);
    if (ks + 1 < nk) {
      store(gs, (ks + 1) & 1);
      take_sb(gs);
    }
    __syncthreads();
  };
  int ks = 0;
  for (; ks + 1 < nk; ks += 2) {
    step(ks, g0, g1);
    step(ks + 1, g1, g0);
  }
  if (ks < nk) step(ks, g0, g1);

  // C fragment of v_mfma_f32_32x32x16: lane l, register 4*q+j holds row
  // 8*q + 4*(l/32) + j, column l%32
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
      if (m >= mcnt) continue;
      uint16_t *op = a.out + (int64_t)s_orow[m] * a.out_ld;
      if (DUAL) {
        const int col = n0 + 32 * wv + l32;
        if (col < R) {
          const float gv = round_act<DT>(acc[0][i][r]);
          const float uv = round_act<DT>(acc[1][i][r]);
          op[col] = A::from_f32(silu_act<DT>(gv) * uv);
        }
      } else {
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          const int col = n0 + 64 * wv + 32 * s + l32;
          if (col < R) op[col] = A::from_f32(acc[s][i][r]);
        }
      }
    }
  }
}

template <int DT>
hipError_t launch_t(bool dual, const GroupedArgs &a, int64_t max_m_tiles, hipStream_t st) {
  const int cols = dual ? WROWS / 2 : WROWS;
  const int n_tiles = (a.R + cols - 1) / cols;
  const int64_t total = max_m_tiles * n_tiles;
  const unsigned grid = (unsigned)(8 * ((total + 7) / 8));
  if (dual)
    hipLaunchKernelGGL((gemm_kernel<DT, true>), dim3(grid), dim3(256), kGemmLds, st, a, n_tiles);
  else
    hipLaunchKernelGGL((gemm_kernel<DT, false>), dim3(grid), dim3(256), kGemmLds, st, a, n_tiles);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm(int dtype, bool dual, const GroupedArgs &a, int64_t max_m_tiles,
                       hipStream_t st) {
  return dtype == DT_BF16 ? launch_t<DT_BF16>(dual, a, max_m_tiles, st)
                          : launch_t<DT_F16>(dual, a, max_m_tiles, st);
}

}  // namespace nvm
