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
// gathered activation rows (bf16/fp16), and per pair of k-steps the *packed*
// int4 weight rows, in LDS, double-buffered, with the next global loads in
// flight during the current k-step's MFMAs.  The kernel is bound by the
// cache lines its loads touch, not by its arithmetic: a weight row's codes
// for a k-step pair are half a 128-byte line (one k-step's were a quarter,
// and the line was fetched again for every k-step), and the scales and
// biases come in windows of four groups.  The four wavefronts split the tile along N: a
// wavefront owns 2 x 32 weight rows (gate/up: the same 32 columns of both
// matrices, so the SwiGLU pair lands in one lane) and all 128 routed rows
// (4 x 2 tiles of v_mfma_f32_32x32x16, weights as the A operand).  Each
// weight word is dequantised once per tile, in registers, right before its
// MFMA.  Outputs leave through an LDS tile, as whole rows of 16-byte stores.
//
// Operands are fp16 for both activation dtypes.  A weight q*s + b (s, b of
// 8 or 11 significant bits, q of 4) needs about 12 significant bits: rounded
// to bf16 it would carry a 2^-9 relative error, which at the 235B-A22B shape
// alone makes a mean output error above 1e-3 against the exact products;
// rounded to fp16 (one v_pk_fma_f16, single rounding) the error is 2^-12 and
// the outputs are those of exact weights.  The fp16 MFMA runs at the bf16
// rate.  bf16 activations convert to fp16 exactly within fp16's range; the
// fp16 copies of x and h that the forward hands these GEMMs (act_h) carry a
// power-of-two shift per row and 64-value group (act_sh), which the k-loop
// undoes on its float32 sums, so there bf16's whole range is kept.  Rows
// converted here (the stage entry points) saturate beyond 65504.
//
// k-order inside a k-step: MFMA chunk c (16 wide) and lane half h cover
// the eight k = 8*(4h + c) + i, i = 0..7, in both operands, in the slot
// order i = 0,4,1,5,2,6,3,7 that the nibble expansion of one packed word
// produces.  A lane's B operand for chunk c is then packed word 4h + c of its
// weight row (one 16-byte LDS read serves all four chunks) and its A operand
// is the 16 bytes at offset 16*(4h + c) of the activation row, which staging
// stores in that slot order.
#include <stdlib.h>

#include "common.h"
#include "internal.h"

namespace nvm {

namespace {

constexpr int BM = kGemmBM;       // routed rows per tile
constexpr int WROWS = 256;        // weight rows per tile
constexpr int BK = 64;            // k per stage
constexpr int A_PITCH = 144;      // bytes per staged activation row (128 + 16 pad)
// bytes per staged weight row: the packed codes of two k-steps, as four
// 16-byte chunks, chunk c of row r at slot c ^ ((r >> 2) & 3) (16 consecutive
// rows' chunk c then fall in distinct banks)
constexpr int B_PITCH = 64;
constexpr int A_STAGE = BM * A_PITCH;
constexpr int B_STAGE = WROWS * B_PITCH;
// scales and biases of a wavefront's 32 (x 2) weight rows over one window of
// eight groups: per row and group the fp16 (scale 0, bias 0, scale 1, bias 1);
// 72-byte rows (eight groups + 8 pad: 32 rows' 8-byte reads in distinct banks)
constexpr int W_PITCH = 72;
constexpr int W_WAVE = 32 * W_PITCH;
// two activation stages (one k-step each), two weight stages (a k-step pair
// each) and the four wavefronts' scale/bias windows: 77 KB, two blocks per CU
constexpr int kGemmLds = 2 * A_STAGE + 2 * B_STAGE + 4 * W_WAVE;

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
// in the pair order (x0,x4)(x1,x5)(x2,x6)(x3,x7) of dequant8_h.  (Activations
// that arrive in fp16, GroupedArgs::act_h, are in that order already.)  bf16 values
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

// A scale or bias (act bits) as fp16 bits; bf16 values convert with round to
// nearest even (exactly, inside fp16's normal range).
template <int DT>
__device__ __forceinline__ uint32_t sb_h(uint32_t bits) {
  if constexpr (DT == DT_F16)
    return bits & 0xFFFFu;
  else
    return __builtin_bit_cast(uint16_t, (_Float16)__uint_as_float(bits << 16));
}

__device__ __forceinline__ f32x16 mfma32_h(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// AH: the activations arrive already in fp16 (GroupedArgs::act_h).
template <int DT, bool DUAL, bool AH>
__global__ __launch_bounds__(256, 2) void gemm_kernel(const GroupedArgs a, int n_tiles) {
  using A = Act<DT>;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ int s_arow[BM];
  __shared__ int s_orow[BM];
  // (the m-tile list, read only before the first stage is stored)
  int *const s_tiles = (int *)smem;
  static_assert((kMaxExperts + 1) * 4 <= A_STAGE, "m-tile list exceeds an activation stage");

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
  // fp16 activations stored with group shifts (bf16_to_f16_pairs): does any
  // group of this tile's rows carry one?  (Then the k-loop rescales the sums.)
  const int KSG = a.K >> 6;  // k-steps (groups of 64) per row
  bool shifted = false;
  if constexpr (AH && DT == DT_BF16) {
    uint32_t any = 0;
    if (a.act_sh) {
      if ((KSG & 3) == 0) {
        const int W = KSG >> 2;
        for (int j = tid; j < BM * W; j += 256) {
          const int r = s_arow[j / W];
          if (r >= 0) any |= *(const uint32_t *)(a.act_sh + (int64_t)r * KSG + 4 * (j % W));
        }
      } else {
        for (int j = tid; j < BM * KSG; j += 256) {
          const int r = s_arow[j / KSG];
          if (r >= 0) any |= a.act_sh[(int64_t)r * KSG + j % KSG];
        }
      }
    }
    shifted = __syncthreads_or(any != 0);
  }

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
  // packed weights of a k-step pair (64 bytes of each row: half of a
  // 128-byte line, where one k-step's 32 bytes were a quarter): thread loads
  // staged rows (tid >> 2) + 64c, quarter tid & 3; rows 0..127 of a dual
  // tile are gate rows, 128..255 up rows
  int b_voff[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int wrow = (tid >> 2) + 64 * c;
    const int grow = DUAL ? n0 + (wrow & 127) : n0 + wrow;
    b_voff[c] = grow < R ? grow * KW * 4 + 16 * (tid & 3) : kMaskedOffset;
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
  // (the activations of one k-step; the packed weights of a k-step pair,
  // requested with the pair's first k-step)
  struct Stage {
    u32x4 a[4];
  };
  struct PairB {
    u32x4 b[4];
  };
  auto issue = [&](Stage &g, int ks) {
    const bool ok = ks < nk;
    const int sa = __builtin_amdgcn_readfirstlane(ok ? ks * BK * 2 : 0);
#pragma unroll
    for (int c = 0; c < 4; ++c) g.a[c] = bload16(ra, ok ? a_voff[c] : kMaskedOffset, sa);
  };
  auto issue_b = [&](PairB &g, int ks) {  // ks even: k-steps ks, ks + 1
    const bool ok = ks < nk;
    const int sb = __builtin_amdgcn_readfirstlane(ok ? ks * BK / 2 : 0);
#pragma unroll
    for (int c = 0; c < 4; ++c)
      g.b[c] = bload16(c < 2 ? rw0 : rw1, ok ? b_voff[c] : kMaskedOffset, sb);
  };
  // Scales and biases of the lane's two weight rows come in windows of eight
  // groups split over the lane halves: half h loads groups 4h..4h+3 of the
  // window, one 8-byte load per row and matrix every eight groups (lanes l
  // and l + 32 own the same rows).  (One 2-byte load per k-step made as many
  // memory requests as the activation and weight loads together: each lane
  // reads a different row.)  At a window's first k-step the wavefront moves
  // the window, arrived in registers, to its rows' LDS as fp16 values, and
  // requests the next window into the same registers: it has the window's
  // eight groups of k-steps to arrive.
  u32x2 wcur[4];  // scale 0, bias 0, scale 1, bias 1
  // (A half's four groups are one 8-byte load when a row's groups are a
  // multiple of four: they then start on a dword and end inside their row.
  // Otherwise they are packed from 2-byte loads; groups past the row read
  // zeros.)
  const bool win8 = GPR % 4 == 0;
  auto issue_w = [&](u32x2 (&w)[4], int wi) {
    const int gh = 8 * wi + 4 * h;  // this half's first group
    const int so = __builtin_amdgcn_readfirstlane(16 * wi);
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const rsrc_t r = t ? (s ? rb1 : rb0) : (s ? rs1 : rs0);
        if (win8) {
          w[2 * s + t] = bload8(r, gh < GPR ? srow[s] + 8 * h : kMaskedOffset, so);
        } else {
          uint32_t v[4];
#pragma unroll
          for (int q = 0; q < 4; ++q)
            v[q] = bload2(r, gh + q < GPR ? srow[s] + 8 * h : kMaskedOffset, so + 2 * q) &
                   0xFFFFu;
          w[2 * s + t] = u32x2{v[0] | (v[1] << 16), v[2] | (v[3] << 16)};
        }
      }
  };
  int w_idx = 0;  // window of wcur
  issue_w(wcur, 0);
  auto store = [&](const Stage &g, int buf) {
    uint8_t *As = smem + buf * A_STAGE;
#pragma unroll
    for (int c = 0; c < 4; ++c)
      *(u32x4 *)(As + ((tid >> 3) + 32 * c) * A_PITCH + 16 * (tid & 7)) =
          (AH ? g.a[c] : act_to_h<DT>(g.a[c]));
  };
  auto store_b = [&](const PairB &g, int pbuf) {
    uint8_t *Bs = smem + 2 * A_STAGE + pbuf * B_STAGE;
#pragma unroll
    for (int c = 0; c < 4; ++c)
      *(u32x4 *)(Bs + ((tid >> 2) + 64 * c) * B_PITCH + 16 * ((tid & 3) ^ ((tid >> 4) & 3))) =
          g.b[c];
  };

  f32x16 acc[2][4];
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[s][i][r] = 0.f;

  // k-step ks's scale and bias of the lane's two weight rows, fp16 pairs
  // (k-step ks lies in group ks * 64 / gs; calls come in k-step order).  The
  // window in LDS: per row of the wavefront and group, the fp16 values
  // (scale 0, bias 0, scale 1, bias 1); only the wavefront itself writes and
  // reads its rows, in order.
  uint8_t *const w_lds = smem + 2 * A_STAGE + 2 * B_STAGE + wv * W_WAVE + l32 * W_PITCH;
  uint32_t sc[2], bi[2];
  auto take_sb = [&](int ks) {
    const int j = (ks * BK / a.gs) & 7;
    if ((ks * BK) % (8 * a.gs) == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {  // group 4h + i: value i of the half's four
        auto val = [&](const u32x2 &w) {
          const uint32_t d = (i & 2) ? w.y : w.x;
          return sb_h<DT>((i & 1) ? d >> 16 : d & 0xFFFFu);
        };
        *(u32x2 *)(w_lds + 8 * (4 * h + i)) =
            u32x2{val(wcur[0]) | (val(wcur[1]) << 16), val(wcur[2]) | (val(wcur[3]) << 16)};
      }
      issue_w(wcur, ++w_idx);
    }
    const u32x2 v = *(const u32x2 *)(w_lds + 8 * j);
    sc[0] = perm_b32(v.x, v.x, 0x01000100u);
    bi[0] = perm_b32(v.x, v.x, 0x03020302u);
    sc[1] = perm_b32(v.y, v.y, 0x01000100u);
    bi[1] = perm_b32(v.y, v.y, 0x03020302u);
  };
  // nibble-expansion constants in registers (one v_and_or_b32 per dword)
  const uint32_t nib_mask = sgpr_const(0x000F000Fu);
  const uint32_t magic = vgpr_const(0x64006400u);  // fp16 (1024, 1024)
  // Software-pipelined over the four 16-wide chunks: the A reads and the
  // dequantisation of chunk c + 1 are issued ahead of chunk c's MFMAs.
  // NA: the 32-row blocks of routed rows computed (the tile's rows lie in
  // the first NA; the others' A reads and MFMAs are left out).
  auto compute = [&](int ks, auto NA) {
    constexpr int na = decltype(NA)::value;
    const uint8_t *As = smem + (ks & 1) * A_STAGE;
    const uint8_t *Bs = smem + 2 * A_STAGE + ((ks >> 1) & 1) * B_STAGE;
    u32x4 bw[2];
#pragma unroll
    for (int s = 0; s < 2; ++s)
      bw[s] = *(const u32x4 *)(Bs + lrow[s] * B_PITCH +
                               16 * ((2 * (ks & 1) + h) ^ ((lrow[s] >> 2) & 3)));
    auto load_a = [&](int c, u32x4 (&af)[4]) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (i < na) af[i] = *(const u32x4 *)(As + (32 * i + l32) * A_PITCH + 16 * (4 * h + c));
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
        for (int i = 0; i < 4; ++i)
          if (i < na) acc[s][i] = mfma32_h(bf[s], af[i], acc[s][i]);
      if (c < 3) {
#pragma unroll
        for (int i = 0; i < 4; ++i) af[i] = afn[i];
        bf[0] = bfn[0];
        bf[1] = bfn[1];
      }
    }
  };

  // k-step ks computes activation stage ks & 1 and weight stage (ks / 2) & 1
  // while the activation loads of ks + 2 (and, ks even, the weights of the
  // pair ks + 2, ks + 3) are in flight in the register set that held ks;
  // then ks + 1 (issued a k-step earlier) is stored into the other stage,
  // and at the end of an odd k-step the next pair's weights.  Two k-steps per
  // loop trip keep the register sets static.
  // SH (tiles with shifted groups): before k-step ks, lane row block i's sums
  // are brought from the units of the previous group's shift to those of
  // ks's (2^(old - new), exact), and after the last k-step back to units of
  // one (2^shift); the shifts are read here, one byte per row and k-step.
  // (the current shift of each lane's row block i: s_cur[wave][i][lane], in
  // LDS so that no register is held across the k-loop for it)
  __shared__ uint8_t s_cur[4][4][64];
  auto k_loop = [&](auto NA, auto SH) {
    constexpr bool kSh = decltype(SH)::value;
    if constexpr (kSh) {
#pragma unroll
      for (int i = 0; i < 4; ++i) s_cur[wv][i][lane] = 0;
    }
    auto rescale = [&](int ks) {
      if constexpr (kSh) {
        for (int i = 0; i < 4; ++i) {
          const int r = s_arow[32 * i + l32];
          const int cs = s_cur[wv][i][lane];
          const int nsh = r >= 0 ? (int)a.act_sh[(int64_t)r * KSG + ks] : cs;
          if (nsh != cs) {
            const float f = pow2f(cs - nsh);
#pragma unroll
            for (int s = 0; s < 2; ++s)
#pragma unroll
              for (int q = 0; q < 16; ++q) acc[s][i][q] *= f;
            s_cur[wv][i][lane] = (uint8_t)nsh;
          }
        }
      }
    };
    auto step = [&](int ks) {
      if constexpr (kSh) {
        rescale(ks);
        // (the rescale stays apart from the k-step's operand reads, which
        // would otherwise be scheduled into it and raise register pressure)
        __builtin_amdgcn_sched_barrier(0);
      }
      compute(ks, NA);
    };
    Stage g0, g1;
    PairB gb;
    issue(g0, 0);
    issue_b(gb, 0);
    issue(g1, 1);
    store(g0, 0);
    store_b(gb, 0);
    take_sb(0);
    __syncthreads();
    int ks = 0;
    for (; ks + 1 < nk; ks += 2) {
      // even k-step
      issue(g0, ks + 2);
      issue_b(gb, ks + 2);
      step(ks);
      store(g1, 1);
      take_sb(ks + 1);
      __syncthreads();
      // odd k-step
      issue(g1, ks + 3);
      step(ks + 1);
      if (ks + 2 < nk) {
        store(g0, 0);
        store_b(gb, ((ks + 2) >> 1) & 1);
        take_sb(ks + 2);
      }
      __syncthreads();
    }
    if (ks < nk) step(ks);  // an odd count: the last k-step, already staged
    if constexpr (kSh) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float f = pow2f(s_cur[wv][i][lane]);
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
          for (int q = 0; q < 16; ++q) acc[s][i][q] *= f;
      }
    }
  };
  // A tile of at most 64 routed rows (an expert's last, short tile) runs the
  // k-steps with a half or a quarter of the MFMAs.
  using NoSh = std::false_type;
  if (shifted)
    k_loop(std::integral_constant<int, 4>{}, std::true_type{});
  else if (mcnt > 64)
    k_loop(std::integral_constant<int, 4>{}, NoSh{});
  else if (mcnt > 32)
    k_loop(std::integral_constant<int, 2>{}, NoSh{});
  else
    k_loop(std::integral_constant<int, 1>{}, NoSh{});

  // Epilogue through LDS.  The MFMAs take the weights as A and the routed
  // rows as B, so lane l holds routed row 32 i + l % 32 of every accumulator
  // and, in register 4 q + j, weight column 8 q + 4 (l / 32) + j of its 32:
  // four consecutive output columns, written to a [BM][OCOLS] tile over the
  // staging buffers with one 8-byte LDS store.  The block then writes each
  // routed row's OCOLS outputs with 16-byte stores (whole 128-byte lines of
  // the output row), where one 2-byte store per value and lane had covered
  // two rows' 64 bytes.
  constexpr int OCOLS = DUAL ? WROWS / 2 : WROWS;
  constexpr int O_PITCH = 2 * OCOLS + 16;  // bytes (+16: rows start 4 banks apart)
  static_assert(BM * O_PITCH <= kGemmLds, "output tile exceeds the staging LDS");
  __syncthreads();  // every wavefront is done with the stages
  uint8_t *Os = smem;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint8_t *orow = Os + (32 * i + l32) * O_PITCH;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (DUAL) {
        // silu(gate) * up of the act-rounded sums, op by op as silu_act
        uint32_t o[2];
#pragma unroll
        for (int j = 0; j < 4; j += 2) {
          float g0 = acc[0][i][4 * q + j], g1 = acc[0][i][4 * q + j + 1];
          float u0 = acc[1][i][4 * q + j], u1 = acc[1][i][4 * q + j + 1];
          round_act2<DT>(g0, g1);
          round_act2<DT>(u0, u1);
          o[j >> 1] = swiglu_act2<DT>(g0, g1, u0, u1);
        }
        *(u32x2 *)(orow + 2 * (32 * wv + 8 * q + 4 * h)) = u32x2{o[0], o[1]};
      } else {
#pragma unroll
        for (int s = 0; s < 2; ++s)
          *(u32x2 *)(orow + 2 * (64 * wv + 32 * s + 8 * q + 4 * h)) =
              u32x2{A::pack2(acc[s][i][4 * q], acc[s][i][4 * q + 1]),
                    A::pack2(acc[s][i][4 * q + 2], acc[s][i][4 * q + 3])};
      }
    }
  }
  __syncthreads();
  // 16-byte chunk c of rows tid / CPR + k * (256 / CPR); columns past R are
  // not written, and rows whose 16 bytes are not 16-byte aligned in `out`
  // are written a value at a time
  constexpr int CPR = OCOLS / 8;
  const int c = tid % CPR, col = n0 + 8 * c;
  const bool vec = (a.out_ld & 7) == 0 && ((uintptr_t)a.out & 15) == 0 && col + 8 <= R;
  for (int r = tid / CPR; r < mcnt; r += 256 / CPR) {
    u32x4 v = *(const u32x4 *)(Os + r * O_PITCH + 16 * c);
    if constexpr (DUAL && DT == DT_BF16) {
      if (a.out_h) {
        // out_h: the fp16 copy of h for the down product, each 64-column
        // group (eight consecutive lanes: CPR is a multiple of 8) shifted,
        // each 16-byte chunk in the pair order the down product stages
        const int sh = f16_shift_of(max8_lanes(bf16_absmax_bits(v)));
        v = bf16_to_f16_pairs(v, sh);
        if ((c & 7) == 0 && a.out_sh && col < R)
          a.out_sh[(int64_t)s_orow[r] * (R >> 6) + (col >> 6)] = (uint8_t)sh;
      }
    }
    uint16_t *op = a.out + (int64_t)s_orow[r] * a.out_ld + col;
    if (vec) {
      *(u32x4 *)op = v;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (col + e < R) op[e] = (uint16_t)(v[e >> 1] >> (16 * (e & 1)));
    }
  }
}

// ---------------------------------------------------------------------------
// The forward's GEMM (bf16 activations given as their fp16 copy, act_h): the
// tile, MFMA layout, arithmetic, scale/bias windows and epilogue are those of
// gemm_kernel, but nothing is staged through registers.
//  * The activation rows go from memory straight into LDS
//    (buffer_load_dwordx4 ... lds), four stages deep: k-step ks + 3 is
//    requested while ks is computed.  A stage holds 128 rows of 128 bytes;
//    the 16-byte chunk k of row r lies at slot k ^ (r & 7) ^ ((r >> 3) & 1),
//    so the chunk k of sixteen consecutive rows falls in sixteen distinct
//    16-byte bank groups of the 256-byte bank cycle (k ^ (r & 7) alone puts
//    rows r and r + 8 in the same one: a two-way conflict on every A read).
//    The lane-to-chunk assignment of each load instruction makes the
//    swizzle: LDS is written in lane order.
//  * A wavefront's packed weights are its own (no other wavefront reads its
//    rows), so they go from memory into a ring of registers a k-step pair at
//    a time (two 16-byte loads per row half and k-step pair: the pair's 64
//    bytes of a row in back-to-back requests), one pair ahead.
// The register staging of gemm_kernel held two k-steps of activations and a
// k-step pair of weights per thread; with the registers full, the compiler
// placed the next loads after the k-step's MFMAs, so they had a k-step to
// arrive.  Here nothing but the weight ring competes for registers.
//
// LDS waits: the compiler does not track the LDS written by these loads, so
// each k-step waits for its own stage by count before the block barrier:
// s_waitcnt vmcnt(8), the eight loads of the two later stages.  The count
// holds whatever order the register loads (weights, windows, shift scan)
// complete in, as long as the direct-to-LDS loads complete in order among
// themselves: while stage ks is in flight, so are stages ks + 1 and ks + 2,
// nine or more loads outstanding.  (Counting the register loads issued after
// stage ks as well, 12 to 20 by the step's position, would assume that every
// vector memory operation completes in issue order.)  The wait thus also
// drains the register loads issued before the later stages; exact counts
// measured the same.
constexpr int kDmaStages = 4;
// Keeps the loads on either side in program order (left free, the compiler
// groups the prologue's stage loads first, and its own waits for the window
// registers then assume them only eight loads old on every trip).
__device__ __forceinline__ void issue_order() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}
__device__ __forceinline__ void wait_stage() {
  static_assert(kDmaStages == 4, "two later stages of four loads each");
  asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
}
constexpr int D_STAGE = BM * 128;                          // 16 KB
constexpr int kGemmDmaLds = kDmaStages * D_STAGE + 4 * W_WAVE;  // 73 KB

__device__ __forceinline__ void dma16(rsrc_t r, void *lds, int voff, int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds, 16,
                                           voff, soff, 0, 0);
}
template <bool DUAL>
__global__ __launch_bounds__(256, 2) void gemm_dma_kernel(const GroupedArgs a, int n_tiles) {
  constexpr int DT = DT_BF16;
  using A = Act<DT>;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ int s_arow[BM];
  __shared__ int s_orow[BM];
  // the m-tile prefix and the expert offsets, in the first stage's LDS until
  // the tile's rows are known (the first stage loads come after the barrier
  // that follows)
  int *const s_tiles = (int *)smem;
  int *const s_offs = s_tiles + kMaxExperts + 1;
  static_assert(2 * (kMaxExperts + 1) * 4 <= D_STAGE, "m-tile list exceeds an activation stage");

  hoist_args(a.act, a.act_ld, a.act_rows, a.a_map, a.a_div, a.offsets, a.w0, a.s0, a.b0, a.w1,
             a.s1, a.b1, a.R, a.K, a.gs, a.E, a.out, a.o_map, a.out_ld, n_tiles);
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int l32 = lane & 31, h = lane >> 5;

  // m-tile list (as gemm_kernel); the offsets stay in LDS, so the tile's
  // rows need no second round trip to memory
  auto offs = [&](int i) { return a.offsets ? a.offsets[i] : (i == 0 ? 0 : (int)a.act_rows); };
  if (wv == 0) {
    int carry = 0;
    for (int c0 = 0; c0 < a.E; c0 += 64) {
      const int e = c0 + lane;
      const int o0 = e < a.E ? offs(e) : 0, o1 = e < a.E ? offs(e + 1) : 0;
      const int tv = e < a.E ? (o1 - o0 + BM - 1) / BM : 0;
      int inc = tv;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int u = __shfl_up(inc, o);
        if (lane >= o) inc += u;
      }
      if (e < a.E) {
        s_tiles[e] = carry + inc - tv;
        s_offs[e + 1] = o1;
        if (e == 0) s_offs[0] = o0;
      }
      carry += __shfl(inc, 63);
    }
    if (lane == 0) s_tiles[a.E] = carry;
  }
  __syncthreads();
  const int total = s_tiles[a.E] * n_tiles;
  const int per_xcd = (total + 7) >> 3;
  const int local = blockIdx.x >> 3;
  if (local >= per_xcd) return;
  const int t = (blockIdx.x & 7) * per_xcd + local;
  if (t >= total) return;
  const int mt = t / n_tiles, nt = t - mt * n_tiles;
  int lo = 0, hi = a.E - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (s_tiles[mid] <= mt)
      lo = mid;
    else
      hi = mid - 1;
  }
  const int e = lo;
  const int m0 = s_offs[e] + (mt - s_tiles[e]) * BM;
  const int mcnt = min(BM, s_offs[e + 1] - m0);
  const int R = a.R, KW = a.K >> 3, GPR = a.K / a.gs;
  const int n0 = nt * (DUAL ? WROWS / 2 : WROWS);

  for (int i = tid; i < BM; i += 256) {
    const int slot = m0 + i;
    s_arow[i] = i < mcnt ? (a.a_map ? a.a_map[slot] / a.a_div : slot) : -1;
    s_orow[i] = i < mcnt ? (a.o_map ? a.o_map[slot] : slot) : -1;
  }
  __syncthreads();

  const int KSG = a.K >> 6;
  const rsrc_t ra = make_rsrc(a.act, (uint32_t)(a.act_rows * a.act_ld * 2));
  const int64_t eoff = (int64_t)e * R;
  const rsrc_t rw0 = make_rsrc(a.w0 + eoff * KW, (uint32_t)R * KW * 4);
  const rsrc_t rw1 = make_rsrc((DUAL ? a.w1 : a.w0) + eoff * KW, (uint32_t)R * KW * 4);
  const rsrc_t rs0 = make_rsrc(a.s0 + eoff * GPR, (uint32_t)R * GPR * 2);
  const rsrc_t rb0 = make_rsrc(a.b0 + eoff * GPR, (uint32_t)R * GPR * 2);
  const rsrc_t rs1 = make_rsrc((DUAL ? a.s1 : a.s0) + eoff * GPR, (uint32_t)R * GPR * 2);
  const rsrc_t rb1 = make_rsrc((DUAL ? a.b1 : a.b0) + eoff * GPR, (uint32_t)R * GPR * 2);

  // Activation loads: instruction j of wavefront wv fills rows 32 wv + 8 j +
  // (lane >> 3) of a stage; lane (lane & 7) of a row loads chunk
  // (lane & 7) ^ (lane >> 3) ^ (j & 1) (row & 7 = lane >> 3, (row >> 3) & 1
  // = j & 1), which lands at slot lane & 7.
  int a_voff[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int ar = s_arow[32 * wv + 8 * j + (lane >> 3)];
    a_voff[j] = ar >= 0 ? (int)(((int64_t)ar * a.act_ld) * 2) +
                              16 * ((lane & 7) ^ (lane >> 3) ^ (j & 1))
                        : kMaskedOffset;
  }
  const int nk = a.K / BK;
  // k-step ks into stage ks % kDmaStages (k-steps past the end read zeros
  // into a stage nothing reads: every k-step issues the same loads, so the
  // wait counts below hold throughout)
  auto dma_stage = [&](int ks) {
    uint8_t *st = smem + (ks % kDmaStages) * D_STAGE + wv * 32 * 128;
    const bool ok = ks < nk;
    const int so = __builtin_amdgcn_readfirstlane(ok ? ks * BK * 2 : 0);
#pragma unroll
    for (int j = 0; j < 4; ++j) dma16(ra, st + j * 1024, ok ? a_voff[j] : kMaskedOffset, so);
  };
  // the lane's two weight rows (sub 0/1), for the weight ring and the
  // scale/bias windows
  int srow[2], b_voff[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int grow = DUAL ? n0 + 32 * wv + l32 : n0 + 64 * wv + 32 * s + l32;
    srow[s] = grow < R ? grow * GPR * 2 : kMaskedOffset;
    b_voff[s] = grow < R ? grow * KW * 4 + 16 * h : kMaskedOffset;
  }
  // weight ring: slot p & 1 holds k-step pair p, [sub][k-step of the pair]
  // (pairs past the end read zeros)
  u32x4 bq[2][2][2];
  const int np = (nk + 1) >> 1;
  auto issue_b = [&](u32x4 (&q)[2][2], int p) {
    const bool ok = p < np;
    const int sb = __builtin_amdgcn_readfirstlane(ok ? p * BK : 0);
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
        q[s][kk] = bload16(s ? rw1 : rw0, ok ? b_voff[s] : kMaskedOffset, sb + kk * (BK / 2));
  };
  // scale/bias windows of eight 64-wide groups, one a trip of eight k-steps
  // (group size 64; as gemm_kernel, one 8-byte load per row, matrix and half)
  u32x2 wcur[4];
  auto issue_w = [&](u32x2 (&w)[4], int wi) {
    const int gh = 8 * wi + 4 * h;
    const int so = __builtin_amdgcn_readfirstlane(16 * wi);
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int t2 = 0; t2 < 2; ++t2) {
        const rsrc_t r = t2 ? (s ? rb1 : rb0) : (s ? rs1 : rs0);
        w[2 * s + t2] = bload8(r, gh < GPR ? srow[s] + 8 * h : kMaskedOffset, so);
      }
  };

  f32x16 acc[2][4];
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[s][i][r] = 0.f;

  uint8_t *const w_lds = smem + kDmaStages * D_STAGE + wv * W_WAVE + l32 * W_PITCH;
  uint32_t sc[2], bi[2];
  // at a trip's first k-step: the arrived window to LDS, the next requested
  auto new_window = [&](int wi) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      auto val = [&](const u32x2 &w) {
        const uint32_t d = (i & 2) ? w.y : w.x;
        return sb_h<DT>((i & 1) ? d >> 16 : d & 0xFFFFu);
      };
      *(u32x2 *)(w_lds + 8 * (4 * h + i)) =
          u32x2{val(wcur[0]) | (val(wcur[1]) << 16), val(wcur[2]) | (val(wcur[3]) << 16)};
    }
    issue_w(wcur, wi + 1);
  };
  auto take_sb = [&](int j) {  // group j of the window
    const u32x2 v = *(const u32x2 *)(w_lds + 8 * j);
    sc[0] = perm_b32(v.x, v.x, 0x01000100u);
    bi[0] = perm_b32(v.x, v.x, 0x03020302u);
    sc[1] = perm_b32(v.y, v.y, 0x01000100u);
    bi[1] = perm_b32(v.y, v.y, 0x03020302u);
  };
  const uint32_t nib_mask = sgpr_const(0x000F000Fu);
  const uint32_t magic = vgpr_const(0x64006400u);
  // this lane's A read offsets within a stage: row l32 (+ 32 i), chunk
  // 4 h + c at slot (4 h + c) ^ (l32 & 7) ^ ((l32 >> 3) & 1)
  int a_rd[4];
#pragma unroll
  for (int c = 0; c < 4; ++c)
    a_rd[c] = l32 * 128 + 16 * ((4 * h + c) ^ (l32 & 7) ^ ((l32 >> 3) & 1));
  // k-step ks from stage ks % kDmaStages and the weights bw (as gemm_kernel)
  auto compute = [&](int ks, const u32x4 (&bw)[2], auto NA) {
    constexpr int na = decltype(NA)::value;
    const uint8_t *As = smem + (ks % kDmaStages) * D_STAGE;
    auto load_a = [&](int c, u32x4 (&af)[4]) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (i < na) af[i] = *(const u32x4 *)(As + a_rd[c] + 32 * 128 * i);
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
        for (int i = 0; i < 4; ++i)
          if (i < na) acc[s][i] = mfma32_h(bf[s], af[i], acc[s][i]);
      if (c < 3) {
#pragma unroll
        for (int i = 0; i < 4; ++i) af[i] = afn[i];
        bf[0] = bfn[0];
        bf[1] = bfn[1];
      }
    }
  };

  __shared__ uint8_t s_cur[4][4][64];
  auto k_loop = [&](auto NA, auto SH) {
    constexpr bool kSh = decltype(SH)::value;
    if constexpr (kSh) {
#pragma unroll
      for (int i = 0; i < 4; ++i) s_cur[wv][i][lane] = 0;
    }
    auto rescale = [&](int ks) {
      if constexpr (kSh) {
        for (int i = 0; i < 4; ++i) {
          const int r = s_arow[32 * i + l32];
          const int cs = s_cur[wv][i][lane];
          const int nsh = r >= 0 ? (int)a.act_sh[(int64_t)r * KSG + ks] : cs;
          if (nsh != cs) {
            const float f = pow2f(cs - nsh);
#pragma unroll
            for (int s = 0; s < 2; ++s)
#pragma unroll
              for (int q = 0; q < 16; ++q) acc[s][i][q] *= f;
            s_cur[wv][i][lane] = (uint8_t)nsh;
          }
        }
      }
    };
    // Trips of eight k-steps (one window).  k-step ks waits for this
    // wavefront's loads of stage ks (those of stages ks + 1 and ks + 2 may be
    // in flight), then meets the block: every wavefront's loads of ks have
    // landed, and every wavefront is done with ks - 1, whose stage the loads
    // of ks + 3 refill.  After an odd k-step its pair's slot takes the pair
    // two ahead.  Only the products are skipped past the end; the loads are
    // the same on every trip.
    for (int ks0 = 0; ks0 < nk; ks0 += 8) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int ks = ks0 + j;
        wait_stage();
        asm volatile("s_barrier" ::: "memory");
        dma_stage(ks + kDmaStages - 1);
        issue_order();
        if (j == 0) new_window(ks0 >> 3);
        take_sb(j);
        if (ks < nk) {
          if constexpr (kSh) {
            rescale(ks);
            __builtin_amdgcn_sched_barrier(0);
          }
          const u32x4 bw[2] = {bq[(j >> 1) & 1][0][j & 1], bq[(j >> 1) & 1][1][j & 1]};
          compute(ks, bw, NA);
        }
        if (j & 1) issue_b(bq[(j >> 1) & 1], (ks >> 1) + 2);
        issue_order();
      }
    }
    if constexpr (kSh) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float f = pow2f(s_cur[wv][i][lane]);
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
          for (int q = 0; q < 16; ++q) acc[s][i][q] *= f;
      }
    }
    // the zero-filling loads past the end land before LDS is reused
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  };
  // prologue: the first window, then stages 0..2 and weight pairs 0 and 1
  // in the order of steps -3 (stage 0, pair 0), -2 (stage 1) and -1
  // (stage 2, pair 1), as the trips issue them
  issue_w(wcur, 0);
  issue_order();
  dma_stage(0);
  issue_order();
  issue_b(bq[0], 0);
  issue_order();
  dma_stage(1);
  dma_stage(2);
  issue_order();
  issue_b(bq[1], 1);
  issue_order();
  // fp16 copies stored with group shifts (as gemm_kernel); scanned after the
  // first loads are out, so that its round trip overlaps theirs
  bool shifted = false;
  {
    uint32_t any = 0;
    if (a.act_sh) {
      if ((KSG & 3) == 0) {
        const int W = KSG >> 2;
        for (int j = tid; j < BM * W; j += 256) {
          const int r = s_arow[j / W];
          if (r >= 0) any |= *(const uint32_t *)(a.act_sh + (int64_t)r * KSG + 4 * (j % W));
        }
      } else {
        for (int j = tid; j < BM * KSG; j += 256) {
          const int r = s_arow[j / KSG];
          if (r >= 0) any |= a.act_sh[(int64_t)r * KSG + j % KSG];
        }
      }
    }
    shifted = __syncthreads_or(any != 0);
  }
  using NoSh = std::false_type;
  if (shifted)
    k_loop(std::integral_constant<int, 4>{}, std::true_type{});
  else if (mcnt > 64)
    k_loop(std::integral_constant<int, 4>{}, NoSh{});
  else if (mcnt > 32)
    k_loop(std::integral_constant<int, 2>{}, NoSh{});
  else
    k_loop(std::integral_constant<int, 1>{}, NoSh{});

  // Epilogue through LDS (as gemm_kernel), over the stages and windows
  constexpr int OCOLS = DUAL ? WROWS / 2 : WROWS;
  constexpr int O_PITCH = 2 * OCOLS + 16;
  static_assert(BM * O_PITCH <= kGemmDmaLds, "output tile exceeds the staging LDS");
  __syncthreads();
  uint8_t *Os = smem;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint8_t *orow = Os + (32 * i + l32) * O_PITCH;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (DUAL) {
        uint32_t o[2];
#pragma unroll
        for (int j = 0; j < 4; j += 2) {
          float g0 = acc[0][i][4 * q + j], g1 = acc[0][i][4 * q + j + 1];
          float u0 = acc[1][i][4 * q + j], u1 = acc[1][i][4 * q + j + 1];
          round_act2<DT>(g0, g1);
          round_act2<DT>(u0, u1);
          o[j >> 1] = swiglu_act2<DT>(g0, g1, u0, u1);
        }
        *(u32x2 *)(orow + 2 * (32 * wv + 8 * q + 4 * h)) = u32x2{o[0], o[1]};
      } else {
#pragma unroll
        for (int s = 0; s < 2; ++s)
          *(u32x2 *)(orow + 2 * (64 * wv + 32 * s + 8 * q + 4 * h)) =
              u32x2{A::pack2(acc[s][i][4 * q], acc[s][i][4 * q + 1]),
                    A::pack2(acc[s][i][4 * q + 2], acc[s][i][4 * q + 3])};
      }
    }
  }
  __syncthreads();
  constexpr int CPR = OCOLS / 8;
  const int c = tid % CPR, col = n0 + 8 * c;
  const bool vec = (a.out_ld & 7) == 0 && ((uintptr_t)a.out & 15) == 0 && col + 8 <= R;
  for (int r = tid / CPR; r < mcnt; r += 256 / CPR) {
    u32x4 v = *(const u32x4 *)(Os + r * O_PITCH + 16 * c);
    if constexpr (DUAL) {
      if (a.out_h) {
        const int sh = f16_shift_of(max8_lanes(bf16_absmax_bits(v)));
        v = bf16_to_f16_pairs(v, sh);
        if ((c & 7) == 0 && a.out_sh && col < R)
          a.out_sh[(int64_t)s_orow[r] * (R >> 6) + (col >> 6)] = (uint8_t)sh;
      }
    }
    uint16_t *op = a.out + (int64_t)s_orow[r] * a.out_ld + col;
    if (vec) {
      *(u32x4 *)op = v;
    } else {
#pragma unroll
      for (int e2 = 0; e2 < 8; ++e2)
        if (col + e2 < R) op[e2] = (uint16_t)(v[e2 >> 1] >> (16 * (e2 & 1)));
    }
  }
}

template <bool DUAL>
void allow_gemm_dma_lds() {
  static bool done[64] = {false};
  int dev = 0;
  if (hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64 && !done[dev]) {
    (void)hipFuncSetAttribute((const void *)&gemm_dma_kernel<DUAL>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, kGemmDmaLds);
    done[dev] = true;
  }
}

hipError_t launch_dma(bool dual, const GroupedArgs &a, int64_t max_m_tiles, hipStream_t st) {
  const int cols = dual ? WROWS / 2 : WROWS;
  const int n_tiles = (a.R + cols - 1) / cols;
  const int64_t total = max_m_tiles * n_tiles;
  const unsigned grid = (unsigned)(8 * ((total + 7) / 8));
  if (dual) {
    allow_gemm_dma_lds<true>();
    hipLaunchKernelGGL(gemm_dma_kernel<true>, dim3(grid), dim3(256), kGemmDmaLds, st, a, n_tiles);
  } else {
    allow_gemm_dma_lds<false>();
    hipLaunchKernelGGL(gemm_dma_kernel<false>, dim3(grid), dim3(256), kGemmDmaLds, st, a,
                       n_tiles);
  }
  return hipGetLastError();
}


// more than 64 KB of dynamic LDS: allowed once per device and instance (a
// failure shows up as a failed launch)
template <int DT, bool DUAL, bool AH>
void allow_gemm_lds() {
  static bool done[64] = {false};
  int dev = 0;
  if (hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64 && !done[dev]) {
    (void)hipFuncSetAttribute((const void *)&gemm_kernel<DT, DUAL, AH>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, kGemmLds);
    done[dev] = true;
  }
}

template <int DT, bool AH>
hipError_t launch_t(bool dual, const GroupedArgs &a, int64_t max_m_tiles, hipStream_t st) {
  const int cols = dual ? WROWS / 2 : WROWS;
  const int n_tiles = (a.R + cols - 1) / cols;
  const int64_t total = max_m_tiles * n_tiles;
  const unsigned grid = (unsigned)(8 * ((total + 7) / 8));
  if (dual)
    allow_gemm_lds<DT, true, AH>();
  else
    allow_gemm_lds<DT, false, AH>();
  if (dual)
    hipLaunchKernelGGL((gemm_kernel<DT, true, AH>), dim3(grid), dim3(256), kGemmLds, st, a,
                       n_tiles);
  else
    hipLaunchKernelGGL((gemm_kernel<DT, false, AH>), dim3(grid), dim3(256), kGemmLds, st, a,
                       n_tiles);
  return hipGetLastError();
}

// bf16 -> its fp16 copy for the prefill GEMMs, eight values a thread, stored
// in the pair order (x0,x4)(x1,x5)(x2,x6)(x3,x7): each group of 64 values
// (eight threads) shifted by bf16_to_f16_pairs, its shift in sh.  ALIGNED: x
// is 16-byte aligned (one 16-byte load a thread, else eight 2-byte loads).
template <bool ALIGNED>
__global__ __launch_bounds__(256) void act_to_f16_kernel(const uint16_t *__restrict__ x,
                                                        int64_t n8, uint16_t *__restrict__ out,
                                                        uint8_t *__restrict__ sh) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  // (n8 is a multiple of 8: a group's eight threads are all in range or all
  // out of it)
  const bool ok = i < n8;
  u32x4 v = {0u, 0u, 0u, 0u};
  if (ok) {
    if constexpr (ALIGNED) {
      v = ldg16(x + 8 * i);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        v[j] = (uint32_t)x[8 * i + 2 * j] | ((uint32_t)x[8 * i + 2 * j + 1] << 16);
    }
  }
  const int s = f16_shift_of(max8_lanes(bf16_absmax_bits(v)));
  if (!ok) return;
  *(u32x4 *)(out + 8 * i) = bf16_to_f16_pairs(v, s);
  if ((i & 7) == 0) sh[i >> 3] = (uint8_t)s;
}

}  // namespace

hipError_t launch_gemm(int dtype, bool dual, const GroupedArgs &a, int64_t max_m_tiles,
                       hipStream_t st) {
  if (dtype != DT_BF16) return launch_t<DT_F16, false>(dual, a, max_m_tiles, st);
  // (NVM_GEMM_NODMA=1, read at each launch, takes the register-staged
  // kernel of the same arithmetic: the tests compare the two bit for bit)
  const char *nodma = getenv("NVM_GEMM_NODMA");
  if (a.act_h && a.gs == 64 && a.K % 256 == 0 && !(nodma && nodma[0] == '1'))
    return launch_dma(dual, a, max_m_tiles, st);
  return a.act_h ? launch_t<DT_BF16, true>(dual, a, max_m_tiles, st)
                 : launch_t<DT_BF16, false>(dual, a, max_m_tiles, st);
}

hipError_t launch_act_to_f16(const void *x, int64_t n, void *out, uint8_t *sh, hipStream_t st) {
  if (n % 64 || (uintptr_t)out % 16 || (uintptr_t)x % 2 || !sh) return hipErrorInvalidValue;
  const int64_t n8 = n / 8;
  if (n8 == 0) return hipSuccess;
  const dim3 grid((unsigned)((n8 + 255) / 256));
  if ((uintptr_t)x % 16 == 0)
    hipLaunchKernelGGL(act_to_f16_kernel<true>, grid, dim3(256), 0, st, (const uint16_t *)x, n8,
                       (uint16_t *)out, sh);
  else
    hipLaunchKernelGGL(act_to_f16_kernel<false>, grid, dim3(256), 0, st, (const uint16_t *)x, n8,
                       (uint16_t *)out, sh);
  return hipGetLastError();
}

}  // namespace nvm
