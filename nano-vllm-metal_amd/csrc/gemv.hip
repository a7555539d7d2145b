// Decode-regime grouped W4A16 expert products (few routed rows per expert).
//
// Replaces `mx.gather_qmm` inside grouped_expert_linear (layers/moe.py:21-32)
// for decode-sized batches, fused with SwiGLU (layers/moe.py:84,
// layers/activation.py:21-24, op by op: silu_act) for the gate/up pair.
//
// Weight bytes dominate, so the kernel is shaped to stream them at HBM rate:
//
// * Work units are (expert, chunk of up to 16 routed rows, tile of 16*NT
//   weight rows).  The unit list of all active experts is derived on the
//   device from the expert offsets, and a persistent grid deals every block a
//   contiguous, equal share of it: every block moves the same number of
//   bytes, and consecutive units of a block share their routed rows.
// * Inside a block the wavefronts split the reduction dimension: wavefront w
//   owns k-slice w % KS (GPW 64-wide quantisation groups) of weight-row tile
//   w / KS, so all wavefronts move the same bytes per unit.  The KS partial
//   sums of a tile meet in LDS once per unit (double-buffered: one barrier per
//   unit) and are summed in k-slice order.
// * Each wavefront keeps DEPTH units of its weights (and their scales and
//   biases) in flight in a register ring that runs across unit boundaries, so
//   the memory pipe never drains between units.
//
// Exact inner products on the matrix cores.  A 4-bit code q becomes the exact
// 16-bit float M+q (M = 128 for bf16, code in mantissa bits 0-3; M = 64 for
// fp16, bits 4-7) by OR-ing it into a constant; v_mfma_f32_16x16x32 accumulates x.(M+q) over one 64-wide group,
// and the group is folded as
//   sum_i x_i w_i = s * sum_i x_i (M + q_i) + (b - M s) * sum_i x_i,
// the reference's w = q*s + b (metal/src/quantized_matmul.cpp:135) without
// ever rounding a weight.  The scale term is one FMA per accumulator and
// group; the bias terms of four groups are one v_mfma_f32_16x16x4_f32 whose A
// operand holds the 64-wide group sums of the routed rows.
//
// MFMA roles (16x16x32): A = routed rows [16 x 32 k], B = weights [32 k x 16
// weight rows], C[routed row][weight row].  Lane l = (c, G), c = l%16,
// G = l/16, supplies A row c and B column c for k-slots 8G..8G+7 and holds C
// rows 4G..4G+3 of column c.  Per pair of groups (64 bytes of a weight row),
// lane group G loads the 16 bytes at 16G: lane groups 0-1 hold the first
// group, 2-3 the second.  One v_permlane32_swap per two words trades words 2-3
// of the lower half-wave for words 0-1 of the upper one (swap_pairs), after
// which word j of every lane belongs to group j/2, so each MFMA step stays
// inside one group.  The A operand of the lane holds the matching activations,
// permuted once per chunk into the pair order that nibble_pairs() produces.
#include <algorithm>

#include "common.h"
#include "finalize.h"
#include "internal.h"
#include "sort.h"

namespace nvm {

namespace {

constexpr int kChunk = 16;  // routed rows per chunk (MFMA rows)
constexpr int kMaxNW = 8;   // wavefronts per block

// Register budget: resident wavefronts per SIMD (2 -> 256 VGPRs each) and the
// VGPRs of the weight ring.
#ifndef NVM_GEMV_WAVES_PER_SIMD
#define NVM_GEMV_WAVES_PER_SIMD 2
#endif
#ifndef NVM_GEMV_RING
#define NVM_GEMV_RING 48
#endif
constexpr int kWavesPerSimd = NVM_GEMV_WAVES_PER_SIMD;

// Scale or bias values of one weight row over the k-slice, read as an
// aligned window: the 16-bit value for group g of the slice is half
// sb_index(g) of the window (a few values on either side are read and unused).
template <int GPW>
struct SbVec {
  typedef u32x2 type;  // 4 values: enough for slices of up to 3 groups
};
template <>
struct SbVec<4> {
  typedef u32x2 type;  // 4 values, 8-byte aligned (see sb window below)
};
template <>
struct SbVec<6> {
  typedef u32x4 type;
};
template <>
struct SbVec<8> {
  typedef u32x4 type;
};

__device__ __forceinline__ void load_sb(rsrc_t r, int voff, u32x2 &v) { v = bload8(r, voff, 0); }
__device__ __forceinline__ void load_sb(rsrc_t r, int voff, u32x4 &v) { v = bload16(r, voff, 0); }

// 16-bit value `idx` of the window (idx may differ between lanes).
__device__ __forceinline__ uint32_t sb_at(const u32x2 &v, int idx) {
  const uint32_t d = (idx >> 1) ? v.y : v.x;
  return (idx & 1) ? (d >> 16) : (d & 0xFFFFu);
}
__device__ __forceinline__ uint32_t sb_at(const u32x4 &v, int idx) {
  const int w = idx >> 1;
  const uint32_t d = w == 0 ? v.x : w == 1 ? v.y : w == 2 ? v.z : v.w;
  return (idx & 1) ? (d >> 16) : (d & 0xFFFFu);
}
// The same as a select tree on the index bits: with aligned windows the
// equality chain above becomes a dynamic vector extract, which a per-lane
// index puts in scratch memory.
__device__ __forceinline__ uint32_t sb_at_tree(const u32x2 &v, int idx) { return sb_at(v, idx); }
__device__ __forceinline__ uint32_t sb_at_tree(const u32x4 &v, int idx) {
  const uint32_t d = (idx & 4) ? ((idx & 2) ? v.w : v.z) : ((idx & 2) ? v.y : v.x);
  return (idx & 1) ? (d >> 16) : (d & 0xFFFFu);
}

// Words (w0, w1, w2, w3) of a 16-byte load in lane group G hold codes
// 32G + 8j.. of a 128-code group pair.  Exchanging the lower half-wave's
// words 2-3 with the upper half-wave's words 0-1 leaves every lane with words
// 0-1 from the first group and words 2-3 from the second: lane group G then
// holds codes 32(G%2) + 16(G/2) + {0, 8} (first group) and 64 + the same
// (second group).
__device__ __forceinline__ u32x4 swap_pairs(u32x4 w) {
  // v_permlane32_swap: lanes 32-63 of the first operand trade places with
  // lanes 0-31 of the second
  const auto a = __builtin_amdgcn_permlane32_swap(w.x, w.z, false, false);
  const auto b = __builtin_amdgcn_permlane32_swap(w.y, w.w, false, false);
  return u32x4{a[0], b[0], a[1], b[1]};
}

template <bool DUAL, int GPW>
struct GemvCfg {
  static constexpr int NM = DUAL ? 2 : 1;  // weight matrices per unit
  static constexpr int SBW = sizeof(typename SbVec<GPW>::type) / 4;
  // VGPRs of one unit in the ring; DEPTH units make about RING
  static constexpr int UNIT_VGPRS = NM * (2 * GPW + 2 * SBW);  // GPW/2 16-byte loads
  static constexpr int RING = NVM_GEMV_RING;
  static constexpr int DEPTH =
      RING / UNIT_VGPRS < 2 ? 2 : (RING / UNIT_VGPRS > 8 ? 8 : RING / UNIT_VGPRS);
  static constexpr int NB = (GPW + 3) / 4;  // bias MFMAs (four groups each)
};

// SBA: group size 64 with an even number of groups per row, so every lane's
// scale window starts on a dword (sb_h = 0) and the group of a scale value is
// known at compile time.
template <int DT, bool DUAL, int GPW, bool SBA>
__global__ __launch_bounds__(64 * kMaxNW, kWavesPerSimd) void gemv_kernel(
    const GroupedArgs a, int KS, int NT) {
  using A = Act<DT>;
  using Cfg = GemvCfg<DUAL, GPW>;
  constexpr int NM = Cfg::NM, DEPTH = Cfg::DEPTH, NB = Cfg::NB;
  typedef typename SbVec<GPW>::type SB;

  __shared__ int s_off[kMaxExperts + 1];  // slot offsets of the experts
  __shared__ int s_cb[kMaxExperts + 1];   // first chunk index of each expert
  // Units per barrier: for the single product with an even ring the
  // reduction and the epilogue run once per two units (the epilogue items
  // then spread over more wavefronts), over four buffers of partials.  (The
  // gate/up product measured slower that way.)
  constexpr int UPB = !DUAL && DEPTH % 2 == 0 ? 2 : 1, NBUF = 2 * UPB;
  __shared__ int s_orow[NBUF][kChunk];  // output rows of the unit's routed rows
  __shared__ float s_red[NBUF][kMaxNW][NM][4][64];
  // routing finalised here (route_part): ids, scores and the sorted pairs
  __shared__ int s_rids[DUAL ? kFusedPairs : 1];
  __shared__ uint16_t s_rsc[DUAL ? kFusedPairs : 1];
  __shared__ int s_sorted[DUAL ? kFusedPairs : 1];
  __shared__ uint64_t s_mask[DUAL ? kRowExperts : 1];  // token set of each expert

  hoist_args(a.act, a.act_ld, a.act_rows, a.a_map, a.a_div, a.offsets, a.w0, a.s0, a.b0, a.w1,
             a.s1, a.b1, a.R, a.K, a.gs, a.E, a.out, a.o_map, a.out_ld, KS, NT);
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int NW = blockDim.x >> 6;
  const int col = lane & 15, G = lane >> 4;
  const int E = a.E, R = a.R, KW = a.K >> 3, GPR = a.K / a.gs;
  const int gsh = a.gs == 128 ? 1 : 0;
  // routing finalised in this prologue (uniform)
  const bool fused = DUAL && a.route_part != nullptr;

  if (fused) {
    // every block finalises every token (four per wavefront) and sorts the
    // pairs into expert order in LDS: offsets and chunk bases land in s_off
    // and s_cb
    const int T = (int)a.act_rows, k = a.a_div, n = T * k;
    route_in_block<DT>(a.route_part, a.route_splits, T, E, k, a.route_norm, kChunk, s_rids, s_rsc,
                       s_mask, s_off, s_cb, s_sorted);
    if (blockIdx.x == 0) {
      // the routing for the stages after this one (down product, combine)
      for (int i = tid; i < n; i += blockDim.x) {
        a.r_ids[i] = s_rids[i];
        a.r_scores[i] = s_rsc[i];
        a.r_sorted[i] = s_sorted[i];
      }
      for (int i = tid; i <= E; i += blockDim.x) a.r_offsets[i] = s_off[i];
    }
  } else if (wv == 0) {
    // every offset in flight at once (one round trip, not one per 64
    // experts), then the chunk counts from LDS
    // (no offsets: one expert over all act_rows rows, the dense product)
    constexpr int kOffRegs = kMaxExperts / 64 + 1;
    int ov[kOffRegs];
    if (a.offsets) {
      const rsrc_t off_r = make_rsrc(a.offsets, (uint32_t)(E + 1) * 4);
#pragma unroll
      for (int j = 0; j < kOffRegs; ++j)
        if (64 * j <= E) ov[j] = (int)bload4(off_r, (64 * j + lane) * 4, 0);
    } else {
      ov[0] = lane == 1 ? (int)a.act_rows : 0;
    }
#pragma unroll
    for (int j = 0; j < kOffRegs; ++j)
      if (64 * j <= E && 64 * j + lane <= E) s_off[64 * j + lane] = ov[j];
    __builtin_amdgcn_wave_barrier();
    int carry = 0;
    for (int e0 = 0; e0 < E; e0 += 64) {
      const int e = e0 + lane;
      int n = 0;
      if (e < E) n = (s_off[e + 1] - s_off[e] + kChunk - 1) / kChunk;
      int inc = n;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int u = __shfl_up(inc, o);
        if (lane >= o) inc += u;
      }
      if (e < E) s_cb[e] = carry + inc - n;
      carry += __shfl(inc, 63);
    }
    if (lane == 0) s_cb[E] = carry;
  }
  __syncthreads();

  const int rows_unit = 16 * NT;
  const int RT = (R + rows_unit - 1) / rows_unit;
  const int U = s_cb[E] * RT;
  // the block's share in 32-bit arithmetic where it fits (64-bit division is
  // a long software sequence)
  int u0, u1;
  if ((int64_t)U * gridDim.x < (1ll << 31)) {
    u0 = (int)((unsigned)(blockIdx.x * U) / gridDim.x);
    u1 = (int)((unsigned)((blockIdx.x + 1) * U) / gridDim.x);
  } else {
    u0 = (int)((int64_t)blockIdx.x * U / gridDim.x);
    u1 = (int)((int64_t)(blockIdx.x + 1) * U / gridDim.x);
  }
  const int nu = u1 - u0;
  if (nu <= 0) return;  // uniform over the block, before any further barrier

  const int ks = wv % KS, tile = wv / KS;

  // ---- unit iterator (uniform): chunk it_ci of expert it_e, row tile it_rt
  int it_ci = u0 / RT;
  int it_rt = u0 - it_ci * RT;
  int it_e = E - 1;
  // the non-empty expert holding chunk it_ci, found by all lanes at once
  for (int e0 = 0; e0 < E; e0 += 64) {
    const int e = e0 + lane;
    const uint64_t m = __ballot(e < E && s_cb[e] <= it_ci && it_ci < s_cb[e + 1]);
    if (m) {
      it_e = e0 + (int)__builtin_ctzll(m);
      break;
    }
  }
  auto advance = [&]() {
    if (++it_rt == RT) {
      it_rt = 0;
      ++it_ci;
      while (it_e + 1 < E && __builtin_amdgcn_readfirstlane(s_cb[it_e + 1]) <= it_ci) ++it_e;
    }
  };

  // ---- register ring: weights, scales and biases of DEPTH units
  constexpr int GP = GPW / 2;  // 16-byte loads (group pairs) per row and k-slice
  u32x4 wq[DEPTH][NM][GP];
  SB sv[DEPTH][NM], bv[DEPTH][NM];
  int m_e[DEPTH], m_ci[DEPTH], m_r0[DEPTH];

  const int kbyte = ks * GPW * 32;              // k-slice start within a row (bytes)
  const int sidx0 = (ks * GPW) >> gsh;          // first scale value of the k-slice
  const uint32_t mat_bytes = (uint32_t)R * KW * 4;
  const uint32_t sb_bytes = (uint32_t)R * GPR * 2;
  // Every ring refill issues the same loads: a unit past the block's range
  // reads through masked offsets (zeros, no memory traffic), so the number of
  // loads in flight after any ring slot is the same on every path and the
  // compiler's wait counts keep DEPTH - 1 units in flight.
  auto issue = [&](int d, bool valid) {
    const int e = it_e, r0 = it_rt * rows_unit;
    m_e[d] = e;
    m_ci[d] = it_ci;
    m_r0[d] = r0;
    const int row = r0 + 16 * tile + col;
    const bool ok = valid && row < R;
    const int wo = ok ? row * KW * 4 + kbyte + 16 * G : kMaskedOffset;
    const int sbyte = (row * GPR + sidx0) * 2;
    const int so = ok ? (sbyte & ~3) : kMaskedOffset;  // dword-aligned window
    const int64_t eo = (int64_t)e * R;
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      const rsrc_t wr = make_rsrc((m ? a.w1 : a.w0) + eo * KW, mat_bytes);
#pragma unroll
      for (int h = 0; h < GP; ++h) wq[d][m][h] = bload16(wr, wo + 64 * h, 0);
      load_sb(make_rsrc((m ? a.s1 : a.s0) + eo * GPR, sb_bytes), so, sv[d][m]);
      load_sb(make_rsrc((m ? a.b1 : a.b0) + eo * GPR, sb_bytes), so, bv[d][m]);
    }
    if (valid) advance();
  };

  // ---- activation operand of the current chunk
  u32x4 xa[GP][4];
  float xb[NB];
  int cur_ci = -1, cur_slot0 = 0, cur_cnt = 0, my_orow = 0;
  const rsrc_t act_r = make_rsrc(a.act, (uint32_t)(a.act_rows * a.act_ld * 2));
  // requests the chunk's activations into xa in load order (act_finish puts
  // them in MFMA order once they are needed)
  auto act_issue = [&](int e, int ci) {
    const int slot0 =
        __builtin_amdgcn_readfirstlane(s_off[e]) +
        (ci - __builtin_amdgcn_readfirstlane(s_cb[e])) * kChunk;
    const int cnt = min(kChunk, __builtin_amdgcn_readfirstlane(s_off[e + 1]) - slot0);
    cur_slot0 = slot0;
    cur_cnt = cnt;
    int arow = -1;
    if (col < cnt) {
      const int sl = slot0 + col;
      arow = fused ? s_sorted[sl] / a.a_div : a.a_map ? a.a_map[sl] / a.a_div : sl;
      my_orow = a.o_map ? a.o_map[sl] : sl;
    }
    // step s of group pair h covers codes 128h + 64(s/2) + 32(G%2) + 16(G/2)
    // + 8(s%2) + 0..7 of the k-slice in lane group G (see swap_pairs)
    const int ao = arow >= 0 ? (int)((int64_t)arow * a.act_ld * 2) +
                                   (ks * GPW * 64 + 32 * (G & 1) + 16 * (G >> 1)) * 2
                             : kMaskedOffset;
#pragma unroll
    for (int h = 0; h < GP; ++h)
#pragma unroll
      for (int st = 0; st < 4; ++st)
        xa[h][st] = bload16(act_r, ao + (128 * h + 64 * (st >> 1) + 8 * (st & 1)) * 2, 0);
  };
  // group sums (bias operand) and MFMA order of the requested activations
  auto act_finish = [&]() {
    float ps[GPW];
#pragma unroll
    for (int h = 0; h < GP; ++h) {
      ps[2 * h] = 0.f;
      ps[2 * h + 1] = 0.f;
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const u32x4 v = xa[h][st];
#pragma unroll
        for (int i = 0; i < 4; ++i) ps[2 * h + (st >> 1)] = A::dot2(v[i], A::kOne2, ps[2 * h + (st >> 1)]);
        xa[h][st] = pair_order(v);
      }
    }
    // 64-wide group sums of routed row c, in every lane of column c
#pragma unroll
    for (int g = 0; g < GPW; ++g) {
      ps[g] += __shfl_xor(ps[g], 16);
      ps[g] += __shfl_xor(ps[g], 32);
    }
    // bias-MFMA A operand: lane (c, G) holds the sum of group 4b + G of row c
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      float v = 0.f;
#pragma unroll
      for (int g = 0; g < 4; ++g)
        if (4 * b + g < GPW && G == g) v = ps[4 * b + g];
      xb[b] = v;
    }
  };

  // window position of group g of the slice: the window starts at the dword
  // holding value sidx0, which is its half `sb_h` (odd rows of an odd number
  // of scale values start mid-dword)
  const int sb_h = SBA ? 0 : ((tile * 16 + col) * GPR + sidx0) & 1;
  auto sb_index = [&](int g) { return SBA ? g : ((ks * GPW + g) >> gsh) - sidx0 + sb_h; };
  // nibble-expansion constants in registers (one v_and_or_b32 per dword)
  const uint32_t nib_mask = sgpr_const(0x000F000Fu << A::kCodeShift);
  const uint32_t magic = vgpr_const(A::kMagic2);
  auto expand = [&](uint32_t w) { return nibble_pairs_v<A::kCodeShift>(w, nib_mask, magic); };
  auto scale_f = [&](const SB &v, int g) { return A::to_f32(sb_at(v, sb_index(g))); };

  // The first chunk's activations are requested before the ring fill: loads
  // return in order, so they are in registers while the ring still streams.
  // The wider slices leave no registers for them beside the filling ring and
  // load them at the first unit instead.
  constexpr bool kActFirst = GPW <= 4 || (!DUAL && GPW == 6);
  if (kActFirst) {
    cur_ci = it_ci;
    act_issue(it_e, it_ci);
  }
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) issue(d, d < nu);
  if (kActFirst) act_finish();

  // epilogue metadata of the units since the last barrier
  int ep_r0[UPB], ep_cnt[UPB], ep_slot0[UPB], ep_buf[UPB];
  // outputs of the last nun units: items (unit, tile, routed row < cnt,
  // weight row), one per thread and pass
  auto epilogue = [&](int nun) {
    const int n0 = NT * ep_cnt[0] * 16;
    const int ntot = n0 + (nun > 1 ? NT * ep_cnt[UPB - 1] * 16 : 0);
    for (int item0 = tid; item0 < ntot; item0 += 64 * NW) {
      const bool second = UPB > 1 && item0 >= n0;
      const int item = second ? item0 - n0 : item0;
      const int cnt = second ? ep_cnt[UPB - 1] : ep_cnt[0];
      const int ub = second ? ep_buf[UPB - 1] : ep_buf[0];
      const int c = item & 15, rest = item >> 4;
      const int t = rest / cnt, tok = rest - t * cnt;
      const int row = (second ? ep_r0[UPB - 1] : ep_r0[0]) + 16 * t + c;
      if (row < R) {
        const int pl = c + 16 * (tok >> 2), pv = tok & 3;
        float sum[NM];
#pragma unroll
        for (int m = 0; m < NM; ++m) {
          // four partials per LDS round trip (reads past KS land on other
          // entries of s_red and are not added), summed in k-slice order
          float acc = 0.f;
          for (int k0 = 0; k0 < KS; k0 += 4) {
            float part[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) part[j] = s_red[ub][min(t * KS + k0 + j, NW - 1)][m][pv][pl];
#pragma unroll
            for (int j = 0; j < 4; ++j)
              if (k0 + j < KS) acc = (k0 + j == 0) ? part[0] : acc + part[j];
          }
          sum[m] = acc;
        }
        uint16_t r;
        int64_t orow;
        if constexpr (DUAL) {
          // reference rounding points: gate and up outputs are act tensors,
          // silu's ops each round (silu_act), and silu(gate) * up rounds once
          // more (its float32 product is exact)
          const float gv = round_act<DT>(sum[0]);
          const float uv = round_act<DT>(sum[NM - 1]);
          r = A::from_f32(silu_act<DT>(gv) * uv);
          orow = (second ? ep_slot0[UPB - 1] : ep_slot0[0]) + tok;
        } else {
          r = A::from_f32(sum[0]);
          orow = s_orow[ub][tok];
        }
        a.out[orow * a.out_ld + row] = r;
      }
    }
  };

  // one unit: ring slot d holds unit i of the block's range
  auto step = [&](int d, int i) {
    if (m_ci[d] != cur_ci) {
      cur_ci = m_ci[d];
      act_issue(m_e[d], m_ci[d]);
      act_finish();
    }
    // ---- partial products of this wavefront's k-slice.  Narrow slices: all
    // codes are expanded into operands of their own, then the MFMAs issue as
    // independent chains (two per group), then the group scales apply in
    // group order (expanding into one reused operand serialises expansion,
    // MFMA and the next expansion).  Wider slices keep the per-pair order,
    // which needs fewer registers.  Both sum in the same order.
    f32x4 o[NM];
#pragma unroll
    for (int m = 0; m < NM; ++m) o[m] = f32x4{0.f, 0.f, 0.f, 0.f};
    if constexpr (GPW <= 4) {
      constexpr int HB = GP, h0 = 0;
      u32x4 bop[HB][NM][4];
      f32x4 acc[HB][NM][2];
#pragma unroll
      for (int hh = 0; hh < HB; ++hh)
#pragma unroll
        for (int m = 0; m < NM; ++m)
          if (h0 + hh < GP) {
            const u32x4 w = swap_pairs(wq[d][m][h0 + hh]);
#pragma unroll
            for (int j = 0; j < 4; ++j) bop[hh][m][j] = expand(w[j]);
          }
#pragma unroll
      for (int step2 = 0; step2 < 2; ++step2)
#pragma unroll
        for (int hh = 0; hh < HB; ++hh)
#pragma unroll
          for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int q = 0; q < 2; ++q)
              if (h0 + hh < GP)
                acc[hh][m][q] = A::mfma16(xa[h0 + hh][2 * q + step2], bop[hh][m][2 * q + step2],
                                          step2 ? acc[hh][m][q] : f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
      for (int hh = 0; hh < HB; ++hh)
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
          for (int q = 0; q < 2; ++q)
            if (h0 + hh < GP) {
              const float s = scale_f(sv[d][m], 2 * (h0 + hh) + q);
#pragma unroll
              for (int v = 0; v < 4; ++v) o[m][v] = fmaf(s, acc[hh][m][q][v], o[m][v]);
            }
    } else {
#pragma unroll
      for (int h = 0; h < GP; ++h) {
#pragma unroll
        for (int m = 0; m < NM; ++m) {
          const u32x4 w = swap_pairs(wq[d][m][h]);
#pragma unroll
          for (int q = 0; q < 2; ++q) {
            f32x4 acc = A::mfma16(xa[h][2 * q], expand(w[2 * q]),
                                  f32x4{0.f, 0.f, 0.f, 0.f});
            acc = A::mfma16(xa[h][2 * q + 1], expand(w[2 * q + 1]), acc);
            const float s = scale_f(sv[d][m], 2 * h + q);
#pragma unroll
            for (int v = 0; v < 4; ++v) o[m][v] = fmaf(s, acc[v], o[m][v]);
          }
        }
      }
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const int gg = 4 * b + G;
#pragma unroll
      for (int m = 0; m < NM; ++m) {
        float bp = 0.f;
        if (gg < GPW) {
          const int si = sb_index(gg);
          const float s = A::to_f32(SBA ? sb_at_tree(sv[d][m], si) : sb_at(sv[d][m], si));
          const float bb = A::to_f32(SBA ? sb_at_tree(bv[d][m], si) : sb_at(bv[d][m], si));
          bp = fmaf(-A::kMagic, s, bb);
        }
        o[m] = __builtin_amdgcn_mfma_f32_16x16x4f32(xb[b], bp, o[m], 0, 0, 0);
      }
    }
    const int r0 = m_r0[d];
    // refill this ring slot DEPTH units ahead before the reduction
    issue(d, i + DEPTH < nu);

    // ---- partial tiles of the unit into LDS; every UPB units one barrier,
    // then the KS partials of each output are summed in k-slice order
    const int buf = i % NBUF;
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
      for (int v = 0; v < 4; ++v) s_red[buf][wv][m][v][lane] = o[m][v];
    if (!DUAL && wv == 0 && G == 0) s_orow[buf][col] = my_orow;
    const int u = d % UPB;
    ep_r0[u] = r0;
    ep_cnt[u] = cur_cnt;
    ep_slot0[u] = cur_slot0;
    ep_buf[u] = buf;
    if (u == UPB - 1) {
      __syncthreads();
      epilogue(UPB);
    }
  };

  // Full passes over the ring, then the remainder: the loop body has no exit
  // in the middle, so at every compute the ring holds DEPTH - 1 younger units
  // of loads and the wait counts say so.
  const int nfull = nu / DEPTH;
  for (int it = 0; it < nfull; ++it) {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) step(d, it * DEPTH + d);
  }
  const int rem = nu - nfull * DEPTH;
#pragma unroll
  for (int d = 0; d < DEPTH - 1; ++d)
    if (d < rem) step(d, nfull * DEPTH + d);
  // a last unit still waiting for its barrier (uniform)
  if (UPB > 1 && (nu % UPB) != 0) {
    __syncthreads();
    epilogue(1);
  }
}

struct GemvShape {
  int gpw, ks, nt;
};

// Groups per wavefront k-slice (GPW) and k-slices per tile (KS): the block
// is KS x NT <= 8 wavefronts, preferably exactly 8 (KS dividing 8).
bool gemv_shape(int K, int R, GemvShape &s) {
  if (K <= 0 || K % 64) return false;
  const int g = K / 64;
  static const int cand[] = {4, 6, 8, 2};  // even: 16-byte loads cover group pairs
  s.gpw = 0;
  for (int pass = 0; pass < 2 && !s.gpw; ++pass)
    for (int c : cand)
      if (g % c == 0 && g / c <= kMaxNW && (pass == 1 || kMaxNW % (g / c) == 0)) {
        s.gpw = c;
        break;
      }
  if (!s.gpw) return false;
  s.ks = g / s.gpw;
  s.nt = std::max(1, std::min(kMaxNW / s.ks, (R + 15) / 16));
  return true;
}

template <int DT, bool DUAL, int GPW, bool SBA>
hipError_t launch_cfg(const GroupedArgs &a, const GemvShape &s, hipStream_t st) {
  // as many blocks as the register budget keeps resident on every CU
  const int nw = s.ks * s.nt;
  const int blocks = std::max(1, 4 * kWavesPerSimd / nw) * cu_count();
  hipLaunchKernelGGL((gemv_kernel<DT, DUAL, GPW, SBA>), dim3(blocks), dim3(64 * s.ks * s.nt), 0, st,
                     a, s.ks, s.nt);
  return hipGetLastError();
}

template <int DT, bool DUAL>
hipError_t launch_t(const GroupedArgs &a, const GemvShape &s, hipStream_t st) {
  // aligned scale windows for the common slice widths
  const bool sba = a.gs == 64 && (a.K / 64) % 2 == 0;
  switch (s.gpw) {
    case 8: return launch_cfg<DT, DUAL, 8, false>(a, s, st);
    case 6:
      return sba ? launch_cfg<DT, DUAL, 6, true>(a, s, st) : launch_cfg<DT, DUAL, 6, false>(a, s, st);
    case 4:
      return sba ? launch_cfg<DT, DUAL, 4, true>(a, s, st) : launch_cfg<DT, DUAL, 4, false>(a, s, st);
    default: return launch_cfg<DT, DUAL, 2, false>(a, s, st);
  }
}

}  // namespace

// Compute units of the current device (cached per device).
int cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

bool gemv_supports(int K) {
  GemvShape s;
  return gemv_shape(K, 16, s);
}

hipError_t launch_gemv(int dtype, bool dual, const GroupedArgs &a, hipStream_t st) {
  // The expert products run on gemv3.  A dense product (one expert, no
  // offsets) does only when its unit list (16-row chunks x weight-row tiles
  // of 16 for gate/up, 32 otherwise) gives every wavefront of the grid at
  // least four units, as the lm head at 32 rows does.  With fewer units this
  // kernel's split of the reduction over a block's wavefronts keeps more
  // loads in flight: q_proj (2048 -> 4096) at one row takes 5.7 us here and
  // 9.4 us on gemv3.
  GemvShape s;
  const bool old_ok = gemv_shape(a.K, a.R, s);
  if (gemv3_supports(a.K, a.R, a.E, a.gs)) {
    const int RU = dual ? 16 : 32;
    const int64_t units = (a.act_rows + 15) / 16 * ((a.R + RU - 1) / RU);
    if (a.offsets || !old_ok || units >= 4 * 8 * (int64_t)cu_count())
      return launch_gemv3(dtype, dual, a, st);
  }
  if (!old_ok) return hipErrorInvalidValue;
  if (dtype == DT_BF16)
    return dual ? launch_t<DT_BF16, true>(a, s, st) : launch_t<DT_BF16, false>(a, s, st);
  return dual ? launch_t<DT_F16, true>(a, s, st) : launch_t<DT_F16, false>(a, s, st);
}

}  // namespace nvm
