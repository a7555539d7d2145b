// Decode-regime grouped W4A16 expert products for the common reduction
// widths (K = 256 NS, NS in {3, 6, 8, 16}: 768, 1536, 2048, 4096).
//
// Replaces `mx.gather_qmm` inside grouped_expert_linear (layers/moe.py:21-32)
// for decode-sized batches, fused with SwiGLU (layers/moe.py:84,
// layers/activation.py:21-24, op by op: silu_act) for the gate/up pair.  The
// arithmetic is gemv.hip's (exact M+q codes on v_mfma_f32_16x16x32, groups
// folded as s * sum x(M+q) + (b - M s) * sum x); what differs is the shape of
// the work, chosen so that every instruction of the inner loop is weight
// streaming or its arithmetic:
//
// * A work unit is (chunk of up to 16 routed rows of one expert, tile of
//   weight rows) over the whole reduction dimension, owned by one wavefront:
//   no partial sums cross wavefronts and the epilogue reads the MFMA
//   accumulators.  Gate/up units are 16 rows of both matrices; down units
//   are two 16-row tiles of the one matrix (the same bytes per unit).
// * The unit's NS steps of 256 reduction columns are unrolled at compile
//   time, and a register ring of D slots (D | NS) streams the weights, scales
//   and biases D steps ahead, across unit boundaries (the next unit's
//   addresses are known when its first slots are requested).  Every slot
//   issues the same loads (a missing unit reads through masked offsets:
//   zeros, no traffic), so the compiler's wait counts keep D - 1 slots in
//   flight.  Step, ring slot and LDS offsets are compile-time constants: the
//   loop body holds no index arithmetic.
// * The routed rows are staged in LDS once per block, already in the lane
//   order of the MFMA A operand, with their 64-wide group sums (the bias
//   MFMA's A operand).  A block's contiguous unit range spans few chunks;
//   they are staged together when they fit ("phase"), else in several
//   phases.  Lanes past a chunk's row count read its last row: an A row
//   only reaches the same C row, which the epilogue does not store.
// * A persistent grid (one block of 8 wavefronts per CU) deals the unit list
//   evenly: block b owns units [bU/n, (b+1)U/n), its wavefronts take them in
//   turn.
#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "common.h"
#include "finalize.h"
#include "internal.h"
#include "sort.h"

namespace nvm {

namespace {

constexpr int kW = 8;           // wavefronts per block
constexpr int kRows = 16;       // routed rows per chunk (MFMA rows)
constexpr int kMaxRounds = 64;  // chunks per staging phase
// dynamic LDS for the staged chunks; with the static LDS of the fused-routing
// gate/up kernel (about 17 KB) within the 160 KB of a CU
constexpr int kActLds = 136 * 1024;
// offset of a masked row: with the 4 KB of step offsets added it stays below
// 2^31 and at or beyond the end of every tensor (gemv3_supports)
constexpr int kMasked = 0x7FFF0000;
// FDOWN: rows of the h stage (a routed row per token at most: the fused
// routing's token limit)
constexpr int kFdRows = 64;

// Bytes per staged routed row: the A operands (2K) and the group sums (K/16),
// padded to an odd multiple of 16 bytes, so that the 16 rows one lane group
// reads in an MFMA step fall in distinct 16-byte bank groups.
constexpr int row_bytes(int K) { return ((2 * K + K / 16 + 31) / 32) * 32 + 16; }

// Exchange of the lower half-wave's words 2-3 with the upper half-wave's
// words 0-1: afterwards words 0-1 of every lane belong to the first group of
// the pair and words 2-3 to the second (see gemv.hip).
__device__ __forceinline__ u32x4 swap_pairs3(u32x4 w) {
  const auto a = __builtin_amdgcn_permlane32_swap(w.x, w.z, false, false);
  const auto b = __builtin_amdgcn_permlane32_swap(w.y, w.w, false, false);
  return u32x4{a[0], b[0], a[1], b[1]};
}

// Position of an A operand inside a staged row: for MFMA step st (0..3) of
// group pair h (0..1) of slot s, lane group G reads the 16 bytes at
// (((s * 2 + h) * 4 + st) * 4 + G) * 16.
__device__ __forceinline__ constexpr int a_offset(int s, int h, int st, int G) {
  return (((s * 2 + h) * 4 + st) * 4 + G) * 16;
}

// Byte offset of column k's 16-bit value inside a staged row: stage_store's
// placement (group g = k / 64 of half-step g / 2, chunk i = k % 64 / 8 at
// MFMA step 2 (g % 2) + i % 2 and lane group G_i, each chunk in pair order).
__device__ __forceinline__ int h_pos(int k) {
  const int g = k >> 6, i = (k >> 3) & 7, e = k & 7;
  const int Gi = ((i >> 2) & 1) | (((i >> 1) & 1) << 1);
  return a_offset(g >> 2, (g >> 1) & 1, 2 * (g & 1) + (i & 1), Gi) + 4 * (e & 3) + 2 * (e >> 2);
}

// Value j (0..3) of a step's scale or bias window (four 16-bit values).
__device__ __forceinline__ uint32_t sb_val(const u32x2 &v, int j) {
  const uint32_t d = (j & 2) ? v.y : v.x;
  return (j & 1) ? (d >> 16) : (d & 0xFFFFu);
}

// One 128-column half-step h (0, 1) of a unit's step: the codes of the
// NM weight-row tiles (wh: this lane's 16 bytes of each) expanded to exact
// M+q values, their MFMAs against the four A operands af, and the scale
// FMAs of the half-step's two groups (values 2h and 2h + 1 of the step's
// scale window sv) into o.
template <int DT, int NM>
__device__ __forceinline__ void halfstep_products(const u32x4 (&wh)[NM], const u32x2 (&sv)[NM],
                                                  const u32x4 (&af)[4], int h, uint32_t nib_mask,
                                                  uint32_t magic, f32x4 (&o)[NM]) {
  using A = Act<DT>;
  u32x4 bop[NM][4];
#pragma unroll
  for (int m = 0; m < NM; ++m) {
    const u32x4 w = swap_pairs3(wh[m]);
#pragma unroll
    for (int j = 0; j < 4; ++j) bop[m][j] = nibble_pairs_v<A::kCodeShift>(w[j], nib_mask, magic);
  }
  f32x4 acc[NM][2];
#pragma unroll
  for (int step2 = 0; step2 < 2; ++step2)
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
      for (int q = 0; q < 2; ++q)
        acc[m][q] = A::mfma16(af[2 * q + step2], bop[m][2 * q + step2],
                              step2 ? acc[m][q] : f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const float sc = A::to_f32(sb_val(sv[m], 2 * h + q));
#pragma unroll
      for (int v = 0; v < 4; ++v) o[m][v] = fmaf(sc, acc[m][q][v], o[m][v]);
    }
}

// The bias terms of half-step h's two groups: lane (c, G) with G < 2
// supplies the group sum xg of routed row c (group 2h + G of the step) and
// (b - M s) of weight row c; lanes with G >= 2 supply zeros.
template <int DT, int NM>
__device__ __forceinline__ void halfstep_bias(const u32x2 (&sv)[NM], const u32x2 (&bv)[NM],
                                              float xg, int h, int G, f32x4 (&o)[NM]) {
  using A = Act<DT>;
  const bool gl = G < 2;
  const int j = 2 * h + (G & 1);
#pragma unroll
  for (int m = 0; m < NM; ++m) {
    const float scv = A::to_f32(sb_val(sv[m], j));
    const float bvv = A::to_f32(sb_val(bv[m], j));
    o[m] = __builtin_amdgcn_mfma_f32_16x16x4f32(gl ? xg : 0.f, gl ? fmaf(-A::kMagic, scv, bvv) : 0.f,
                                                o[m], 0, 0, 0);
  }
}

// FUSED: the gate/up product that finalises the routing in its prologue
// (a distinct instance, so that profiles tell the two apart).
//
// STATIC: expert-major blocks for batches that touch most experts.  Block b
// owns expert b / SPE and its weight-row tiles [p RT / SPE, (p + 1) RT / SPE),
// p = b % SPE, and each wavefront a fixed eighth of those tiles, so a
// wavefront knows its first tile's weights before the routing does: its ring
// and scale/bias window are requested at the very start (behind the partial
// logits when the routing is finalised here, behind the expert offsets
// otherwise) and stream in while the routing and the staging run.  A block
// whose expert no token chose ends there.  Its units are the (tile, chunk)
// pairs of its tiles and its expert's chunks, tile-major, so that an expert
// of more than 16 rows reads a tile's weights again from the cache.
//
// TILE: the down product with the combine in its epilogue (decode batches of
// at most kTilePairs pairs).  Block b owns the 16 weight rows [16 b, 16 b +
// 16), i.e. 16 columns of y, and every chunk of every expert the batch
// touches: its units are (chunk, its tile), in chunk order, dealt over its
// wavefronts phase by phase.  A unit's outputs are the ones the dealt down
// product computes for those rows (the same steps in the same order), and
// go, rounded to the act dtype, into LDS by sorted slot; after the last
// phase the block sums each token's k slots for its 16 columns as
// combine_kernel does (act-rounded terms rnd(down * score), float32, slot
// order, rounded once) and stores y.  No partial result leaves the block.
//
// FDOWN (NSD > 0, with FUSED and STATIC, two blocks per expert): the down
// product of the block's expert follows its gate/up product in the same
// launch.  Block part p's gate/up tiles are h's columns [p KH, (p + 1) KH),
// KH = 128 NSD = I / 2: its wavefronts write their SwiGLU outputs into LDS
// (as staged rows of K = KH) instead of memory, and after a barrier the
// block computes the down product over that half of the reduction for all
// of the expert's rows and every down row: the sum the single product forms
// from zero over the same half-steps (o = lo + hi), stored in float32 to
// d_part[p][pair][row].  The combine adds the halves (lo + hi, rounded to
// the act dtype as the down product's output) before weighting them, so y
// is bit-identical to the separate down product and combine.  The
// block's down units are (32-row tile, chunk of the expert's rows): each
// wavefront's first one is requested before the barrier, and the rest are
// taken from a block counter as the wavefronts finish theirs.
template <int DT, bool DUAL, int NS, bool FUSED, bool STATIC, bool TILE = false, int NSD = 0>
__global__ __launch_bounds__(64 * kW, 2) void gemv3_kernel(const GroupedArgs a, int RT, int SPE) {
  using A = Act<DT>;
  constexpr int D = NS % 4 == 0 ? 4 : 3;  // ring slots
  static_assert(NS % D == 0, "the ring must divide the steps of a unit");
  static_assert(!TILE || (!DUAL && !FUSED && !STATIC), "TILE is a mode of the down product");
  constexpr int K = 256 * NS, KW = K / 8, G64 = K / 64;
  constexpr int ROWB = row_bytes(K);
  constexpr int NM = TILE ? 1 : 2;         // gate and up, or one or two row tiles
  constexpr int RU = DUAL ? kRows : NM * kRows;  // weight rows per unit
  // 16-byte windows per lane of a weight row's scales (or biases): lane
  // group G holds groups 8G..8G+7 of window j, 32j + 8G.. of the row
  constexpr int SBW = (G64 + 31) / 32;
  constexpr bool FDOWN = NSD > 0;
  static_assert(!FDOWN || (DUAL && FUSED && STATIC), "FDOWN follows the expert-major gate/up");
  constexpr int KH = 128 * NSD;                     // reduction columns of a down half
  constexpr int HROWB = FDOWN ? row_bytes(KH) : 0;  // bytes per h row in LDS
  constexpr int HST = FDOWN ? kFdRows * HROWB : 0;  // the h rows, at the top of the LDS
  // staged rows per phase
  constexpr int kMaxStagedRows = (kActLds - HST) / ROWB;
  static_assert(kMaxStagedRows >= kRows, "one chunk must fit the staging LDS");

  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ int s_off[kMaxExperts + 1];  // slot offsets of the experts
  __shared__ int s_cb[kMaxExperts + 1];   // first chunk index of each expert
  __shared__ int s_round[kMaxRounds][4];  // expert, first slot, rows, first staged row
  __shared__ int s_nph, s_nrows;          // chunks and staged rows of the current phase
  __shared__ int s_orow[DUAL || TILE ? 1 : kMaxRounds][kRows];  // output rows (single product)
  static_assert(!FUSED || DUAL, "only the gate/up product finalises the routing");
  // routing finalised here (route_part): ids, scores and the sorted pairs
  __shared__ int s_rids[FUSED ? kFusedPairs : 1];
  __shared__ uint16_t s_rsc[FUSED ? kFusedPairs : 1];
  __shared__ int s_sorted[FUSED ? kFusedPairs : 1];
  __shared__ uint64_t s_mask[FUSED ? kRowExperts : 1];  // token set of each expert
  // TILE: the tile's down outputs [slot][16] (act bits), the slot of each
  // pair and each pair's score (act bits)
  __shared__ uint16_t s_y[TILE ? kTilePairs * kRows : 1];
  __shared__ int s_inv[TILE ? kTilePairs : 1];
  __shared__ uint16_t s_csc[TILE ? kTilePairs : 1];
  __shared__ int s_dctr;  // FDOWN: the next down unit

  hoist_args(a.act, a.act_ld, a.act_rows, a.a_map, a.a_div, a.offsets, a.w0, a.s0, a.b0, a.w1,
             a.s1, a.b1, a.R, a.gs, a.E, a.out, a.o_map, a.out_ld, RT, SPE);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, G = lane >> 4;
  const int E = a.E, R = a.R;
  constexpr bool fused = FUSED;
  // The wavefronts w and w + 4 of a block share a SIMD: they take ranges 2w
  // and 2w + 1 of the eight, so that every SIMD gets a quarter of the units
  // (to one unit).
  const int ri = (wv & 3) * 2 + (wv >> 2);

  // STATIC: the block's expert and this wavefront's tiles [tw0, tw1)
  int e_s = 0, tw0 = 0, tw1 = 0, part = 0, b0 = 0;
  if constexpr (STATIC) {
    e_s = blockIdx.x / SPE;
    part = blockIdx.x - e_s * SPE;
    if (FDOWN && E % 8 == 0) {
      // the two blocks of an expert on one XCD (blocks are dealt to the
      // eight XCDs round-robin by id), so that the 128-byte line of each
      // down row that both halves read comes from its L2 the second time
      const int b = blockIdx.x;
      e_s = (b >> 4) * 8 + (b & 7);
      part = (b >> 3) & 1;
    }
    b0 = part * RT / SPE;
    const int b1 = (part + 1) * RT / SPE;
    tw0 = b0 + ri * (b1 - b0) / kW;
    tw1 = b0 + (ri + 1) * (b1 - b0) / kW;
  }

  // whole-tensor descriptors: every expert's rows are reached through 32-bit
  // offsets (the host keeps E * R * K / 2 below 2 GiB)
  const int64_t ER = (int64_t)E * R;
  rsrc_t w_r[NM], s_r[NM], b_r[NM];
  w_r[0] = make_rsrc(a.w0, (uint32_t)(ER * KW * 4));
  s_r[0] = make_rsrc(a.s0, (uint32_t)(ER * G64 * 2));
  b_r[0] = make_rsrc(a.b0, (uint32_t)(ER * G64 * 2));
  if constexpr (NM > 1) {
    w_r[NM - 1] = make_rsrc(DUAL ? a.w1 : a.w0, (uint32_t)(ER * KW * 4));
    s_r[NM - 1] = make_rsrc(DUAL ? a.s1 : a.s0, (uint32_t)(ER * G64 * 2));
    b_r[NM - 1] = make_rsrc(DUAL ? a.b1 : a.b0, (uint32_t)(ER * G64 * 2));
  }
  const rsrc_t act_r = make_rsrc(a.act, (uint32_t)(a.act_rows * a.act_ld * 2));

  // ring: the weights, two 16-byte loads per matrix and step
  u32x4 wq[D][NM][2];
  // per-lane byte offsets of a unit's rows: weights and scale/bias rows
  struct Addr {
    int w[NM], sb[NM];
  };
  auto issue = [&](int d, int s, const Addr &ad) {
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      wq[d][m][0] = bload16(w_r[m], ad.w[m] + s * 128, 0);
      wq[d][m][1] = bload16(w_r[m], ad.w[m] + s * 128 + 64, 0);
    }
  };
  // A unit's scales and biases come in whole: one 16-byte load per lane,
  // matrix and window (each row's values are read once, by its four lane
  // groups, in full 64-byte segments), one unit ahead of their use.  (Read
  // per step, the 8-byte values every lane group repeats would take as many
  // memory requests as the weights.)  Step s reads its four groups from lane
  // group (s % 8) / 2 of window s / 8 with ds_bpermute.
  typedef u32x4 SbUnit[NM][SBW];
  SbUnit su_cur, bu_cur, su_nxt, bu_nxt;
  auto sb_issue = [&](SbUnit &su, SbUnit &bu, const Addr &ad) {
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
      for (int j = 0; j < SBW; ++j) {
        su[m][j] = bload16(s_r[m], ad.sb[m] + 16 * G + 64 * j, 0);
        bu[m][j] = bload16(b_r[m], ad.sb[m] + 16 * G + 64 * j, 0);
      }
  };
  // row offsets of weight-row tile rt of expert e (masked when !ok or past R)
  auto setup_tile = [&](bool ok, int e, int rt, Addr &ad) {
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      const int row = rt * RU + (DUAL ? 0 : kRows * m) + col;
      const bool rok = ok && row < R;
      const int er = e * R + row;
      ad.w[m] = rok ? er * (KW * 4) + 16 * G : kMasked;
      ad.sb[m] = rok ? er * (G64 * 2) : kMasked;
    }
  };
  Addr cur, nxt;
  // STATIC: the first tile's scale/bias window and ring, before the routing
  auto prefetch = [&]() {
    if constexpr (STATIC) {
      setup_tile(tw0 < tw1, e_s, tw0, cur);
      sb_issue(su_cur, bu_cur, cur);
#pragma unroll
      for (int d = 0; d < D; ++d) issue(d, d, cur);
    }
  };

  const uint32_t nib_mask = sgpr_const(0x000F000Fu << A::kCodeShift);
  const uint32_t magic = vgpr_const(A::kMagic2);

  // ---- routing: finalised and sorted here, or the offsets of dispatch
  if constexpr (fused) {
    const int T = (int)a.act_rows, k = a.a_div, n = T * k;
    route_in_block<DT>(a.route_part, a.route_splits, T, E, k, a.route_norm, kRows, s_rids, s_rsc,
                       s_mask, s_off, s_cb, s_sorted, prefetch);
    if (blockIdx.x == 0) {
      // the routing for the stages after this one (down product, combine)
      for (int i = tid; i < n; i += 64 * kW) {
        a.r_ids[i] = s_rids[i];
        a.r_scores[i] = s_rsc[i];
        a.r_sorted[i] = s_sorted[i];
      }
      for (int i = tid; i <= E; i += 64 * kW) a.r_offsets[i] = s_off[i];
    }
  } else if constexpr (STATIC) {
    // the expert's two offsets first, then the ring behind them
    int o = 0;
    if (tid < 2) o = a.offsets[e_s + tid];
    __builtin_amdgcn_sched_barrier(0);
    prefetch();
    __builtin_amdgcn_sched_barrier(0);
    if (tid < 2) s_off[e_s + tid] = o;
    __syncthreads();
  } else {
    // (no offsets: one expert over all act_rows rows, the dense product)
    for (int i = tid; i <= E; i += 64 * kW)
      s_off[i] = a.offsets ? a.offsets[i] : (i == 0 ? 0 : (int)a.act_rows);
    if constexpr (TILE) {
      // the slot of every pair (inverse of o_map) and its score, for the
      // combine after the last phase
      for (int i = tid; i < (int)a.act_rows; i += 64 * kW) s_inv[i] = 0;
      __syncthreads();
      for (int i = tid; i < (int)a.act_rows; i += 64 * kW) {
        const int p = a.o_map[i];
        if ((unsigned)p < (unsigned)a.act_rows) s_inv[p] = i;
        s_csc[i] = a.c_scores[i];
      }
    }
    __syncthreads();
    if (wv == 0) {
      // chunk bases: exclusive prefix over experts of ceil(rows / 16)
      int carry = 0;
      for (int e0 = 0; e0 < E; e0 += 64) {
        const int e = e0 + lane;
        const int n = e < E ? (s_off[e + 1] - s_off[e] + kRows - 1) / kRows : 0;
        const int inc = wave_incl_scan(n, lane);
        if (e < E) s_cb[e] = carry + inc - n;
        carry += __shfl(inc, 63);
      }
      if (lane == 0) s_cb[E] = carry;
    }
    __syncthreads();
  }

  // ---- the block's chunks [c_first, c_last] and, dynamic, its share of
  // units [u0, u1); unit u = (chunk u / RT, tile u % RT).  STATIC chunk
  // indices are the expert's own (0 .. its chunk count - 1).
  int u0 = 0, u1 = 0, c_first, c_last, n_e = 0;
  if constexpr (STATIC) {
    n_e = s_off[e_s + 1] - s_off[e_s];
    if (n_e == 0) {
      // no token chose this expert: the prefetched ring is not used (its
      // requests complete before the wavefront ends)
      __builtin_amdgcn_s_waitcnt(0);
      return;  // uniform over the block, before any further barrier
    }
    c_first = 0;
    c_last = (n_e + kRows - 1) / kRows - 1;
  } else if constexpr (TILE) {
    // every chunk, for this block's tile
    u0 = 0;
    u1 = s_cb[E];
    if (u1 <= u0) return;  // uniform over the block, before any further barrier
    c_first = 0;
    c_last = u1 - 1;
  } else {
    const int U = s_cb[E] * RT;
    if ((int64_t)U * gridDim.x < (1ll << 31)) {
      u0 = (int)((unsigned)(blockIdx.x * U) / gridDim.x);
      u1 = (int)((unsigned)((blockIdx.x + 1) * U) / gridDim.x);
    } else {
      u0 = (int)((int64_t)blockIdx.x * U / gridDim.x);
      u1 = (int)((int64_t)(blockIdx.x + 1) * U / gridDim.x);
    }
    if (u1 <= u0) return;  // uniform over the block, before any further barrier
    c_first = u0 / RT;
    c_last = (u1 - 1) / RT;
  }

  // ---- FDOWN: the down product's state (used after the gate/up phases)
  [[maybe_unused]] uint8_t *const hst = smem + (kActLds - HST);
  constexpr int NSDR = FDOWN ? NSD : 1;
  constexpr int KWD = 2 * KH / 8, G64D = 2 * KH / 64;  // down row: words, groups
  constexpr int SBWD = FDOWN ? (G64D + 31) / 32 : 1;
  // a down unit: NMD 16-row tiles of the down weights; the ring holds one
  constexpr int NMD = 2;
  struct DAddr {
    int w[NMD], sb[NMD];
  };
  const int Rd = FDOWN ? a.d_R : 0;
  const int64_t ERd = (int64_t)E * Rd;
  const rsrc_t dw_r = make_rsrc(a.d_w, (uint32_t)(ERd * KWD * 4));
  const rsrc_t ds_r = make_rsrc(a.d_s, (uint32_t)(ERd * G64D * 2));
  const rsrc_t db_r = make_rsrc(a.d_b, (uint32_t)(ERd * G64D * 2));
  u32x4 dq[NSDR][NMD];                      // down ring: a half-step (16 bytes a tile) a slot
  u32x4 dsu[NMD][SBWD], dbu[NMD][SBWD];    // the current unit's scale/bias windows
  u32x4 dsu_n[NMD][SBWD], dbu_n[NMD][SBWD];  // the next unit's
  // the block's down units: (tile, chunk of the expert's rows), tile-major
  int dnch = 1, dnu = 0;
  if constexpr (FDOWN) {
    dnch = (n_e + kRows - 1) / kRows;
    dnu = Rd / (NMD * kRows) * dnch;
  }
  // down unit u: row offsets of its tiles (masked past the block's units)
  auto setup_d = [&](int u, DAddr &ad) {
    const bool ok = u < dnu;
    const int tile = ok ? u / dnch : 0;
#pragma unroll
    for (int m = 0; m < NMD; ++m) {
      const int er = e_s * Rd + tile * NMD * kRows + kRows * m + col;
      ad.w[m] = ok ? er * (KWD * 4) + NSD * 64 * part + 16 * G : kMasked;
      ad.sb[m] = ok ? er * (G64D * 2) : kMasked;
    }
  };
  auto issue_d = [&](int slot, int hsl, const DAddr &ad) {
#pragma unroll
    for (int m = 0; m < NMD; ++m) dq[slot][m] = bload16(dw_r, ad.w[m] + 64 * hsl, 0);
  };
  // (a lane group's window of groups 32j + 8G .. + 7 is requested only where
  // it meets the half's groups [2 NSD part, 2 NSD (part + 1)))
  auto sb_issue_d = [&](u32x4 (&su)[NMD][SBWD], u32x4 (&bu)[NMD][SBWD], const DAddr &ad) {
#pragma unroll
    for (int m = 0; m < NMD; ++m)
#pragma unroll
      for (int j = 0; j < SBWD; ++j) {
        const int g0 = 32 * j + 8 * G;
        const bool need = g0 < 2 * NSD * (part + 1) && g0 + 8 > 2 * NSD * part;
        const int off = need ? ad.sb[m] + 16 * G + 64 * j : kMasked;
        su[m][j] = bload16(ds_r, off, 0);
        bu[m][j] = bload16(db_r, off, 0);
      }
  };

  // the staged rows' activation rows (and, single product, output rows)
  auto act_row = [&](int sl) {
    return fused ? s_sorted[sl] / a.a_div : a.a_map ? a.a_map[sl] / a.a_div : sl;
  };
  // staging item (staged row gr, 64-wide group g): its 128 bytes, requested
  // into registers, then written in A-operand order with the group sum.  The
  // rows of the phase's n chunks are staged one after another.
  auto stage_load = [&](int item, int tot, int n, u32x4 (&v)[8]) {
    const bool ok = item < tot;
    const int gr = ok ? item / G64 : 0, g = item - gr * G64;
    int r = 0;
    while (r + 1 < n && s_round[r + 1][3] <= gr) ++r;
    const int arow = act_row(s_round[r][1] + gr - s_round[r][3]);
    const int ao = ok ? (int)((int64_t)arow * a.act_ld * 2) + g * 128 : kMasked;
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = bload16(act_r, ao + 16 * i, 0);
  };
  auto stage_store = [&](int item, int tot, const u32x4 (&v)[8]) {
    if (item >= tot) return;
    const int gr = item / G64, g = item - gr * G64;
    uint8_t *row = smem + gr * ROWB;
    const int s = g >> 2, h = (g >> 1) & 1, q = g & 1;
    float gs = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#pragma unroll
      for (int j = 0; j < 4; ++j) gs = A::dot2(v[i][j], A::kOne2, gs);
      // codes 8i..8i+7 of the group go to lane group
      // Gi = ((i >> 2) & 1) | (((i >> 1) & 1) << 1), MFMA step 2q + (i & 1)
      const int Gi = ((i >> 2) & 1) | (((i >> 1) & 1) << 1);
      *(u32x4 *)(row + a_offset(s, h, 2 * q + (i & 1), Gi)) = pair_order(v[i]);
    }
    *(float *)(row + 2 * K + 4 * g) = gs;
  };

  for (int cb = c_first; cb <= c_last;) {
    const bool prefetched = STATIC && cb == c_first;
    // ---- phase: chunks cb .. cb + n - 1, as many as fit the LDS (at least
    // one); their rows are staged one after another
    if (wv == 0) {
      // the chunks cb .. cb + 63 (within the block's range): expert, first
      // slot and rows of each
      const int c_end = min(c_last + 1, cb + kMaxRounds);
      if constexpr (STATIC) {
        const int ci = cb + lane;
        if (ci < c_end) {
          const int slot0 = s_off[e_s] + ci * kRows;
          s_round[lane][0] = e_s;
          s_round[lane][1] = slot0;
          s_round[lane][2] = min(kRows, s_off[e_s + 1] - slot0);
        }
      } else {
        // expert e owns chunks s_cb[e] .. s_cb[e + 1] - 1
        for (int e0 = 0; e0 < E; e0 += 64) {
          const int e = e0 + lane;
          if (e < E) {
            const int c0 = max(s_cb[e], cb), c1 = min(s_cb[e + 1], c_end);
            for (int ci = c0; ci < c1; ++ci) {
              const int slot0 = s_off[e] + (ci - s_cb[e]) * kRows;
              s_round[ci - cb][0] = e;
              s_round[ci - cb][1] = slot0;
              s_round[ci - cb][2] = min(kRows, s_off[e + 1] - slot0);
            }
          }
        }
      }
      __builtin_amdgcn_wave_barrier();
      const int ci = cb + lane;
      const int cnt = ci < c_end ? s_round[lane][2] : 0;
      const int incl = wave_incl_scan(cnt, lane);
      const bool fits = ci < c_end && (lane == 0 || incl <= kMaxStagedRows);
      const int n = __popcll(__ballot(fits));
      if (fits) s_round[lane][3] = incl - cnt;  // first staged row
      // (every lane takes part in the shuffle: it reads lane n - 1)
      const int rows = __shfl(incl, n - 1);
      if (lane == 0) {
        s_nph = n;
        s_nrows = rows;
      }
    }
    __syncthreads();
    const int n = s_nph, tot = s_nrows * G64;
    if constexpr (!DUAL && !TILE) {
      // output rows of the phase's routed rows (single product)
      for (int i = tid; i < n * kRows; i += 64 * kW) {
        const int r = i / kRows, c = i - r * kRows;
        const int sl = s_round[r][1] + c;
        s_orow[r][c] = c < s_round[r][2] ? (a.o_map ? a.o_map[sl] : sl) : 0;
      }
    }

    // ---- this wavefront's units of the phase: a contiguous range [p0, p1)
    // of the phase's units (dynamic) or its tiles times the phase's chunks,
    // tile-major (STATIC)
    int ua = 0, p0, p1;
    if constexpr (STATIC) {
      p0 = 0;
      p1 = (tw1 - tw0) * n;
    } else {
      const int upc = TILE ? 1 : RT;  // units per chunk (TILE: the block's tile only)
      ua = max(u0, cb * upc);
      const int ub = min(u1, (cb + n) * upc);
      const int P = ub - ua;
      auto range_start = [&](int i) { return ua + (int)((unsigned)(i * P) / kW); };
      p0 = range_start(ri);
      p1 = range_start(ri + 1);
    }
    // unit u -> its chunk r within the phase and its tile rt
    auto unit_of = [&](int u, int &r, int &rt) {
      if constexpr (STATIC) {
        const int q = n == 1 ? u : u / n;
        r = u - q * n;
        rt = tw0 + q;
      } else if constexpr (TILE) {
        r = u - cb;
        rt = blockIdx.x;
      } else {
        const int ci = u / RT;
        r = ci - cb;
        rt = u - ci * RT;
      }
    };
    // unit u: row offsets of its rows (uniform except the lane's rows; a unit
    // past the range is masked)
    auto setup = [&](int u, Addr &ad) {
      const bool ok = u < p1;
      int r, rt;
      unit_of(ok ? u : (STATIC ? 0 : ua), r, rt);
      const int e = STATIC ? e_s : __builtin_amdgcn_readfirstlane(s_round[r][0]);
      setup_tile(ok, e, rt, ad);
    };

    // The first two staging reads, then the first unit's scale/bias window and
    // ring slot 0 (queued behind those reads, so they do not delay them), the
    // staging stores and a barrier, then ring slots 1..D-1.  (All D slots
    // requested ahead of the stores measure no better: later staging reads
    // would wait behind the ring's whole first burst.)  The first phase of a
    // STATIC block has its ring and window in flight already.
    if (!prefetched) setup(p0, cur);
    setup(p0 + 1, nxt);
    {
      u32x4 v0[8], v1[8];
      stage_load(tid, tot, n, v0);
      stage_load(tid + 64 * kW, tot, n, v1);
      if (!prefetched) {
        sb_issue(su_cur, bu_cur, cur);
        issue(0, 0, cur);
      }
      stage_store(tid, tot, v0);
      stage_store(tid + 64 * kW, tot, v1);
      for (int item = tid + 128 * kW; item < tot; item += 64 * kW) {
        stage_load(item, tot, n, v0);
        stage_store(item, tot, v0);
      }
    }
    __syncthreads();
    if (!prefetched) {
#pragma unroll
      for (int d = 1; d < D; ++d) issue(d, d, cur);
    }

    // unit u's epilogue: lane (c, G) holds routed rows 4G..4G+3 of weight row c
    auto epilogue = [&](int u, const f32x4 (&o)[NM]) {
      int r, rt;
      unit_of(u, r, rt);
      const int slot0 = __builtin_amdgcn_readfirstlane(s_round[r][1]);
      const int cnt = __builtin_amdgcn_readfirstlane(s_round[r][2]);
#pragma unroll
      for (int m = 0; m < (DUAL ? 1 : NM); ++m) {
        const int row = rt * RU + (DUAL ? 0 : kRows * m) + col;
        if (row < R) {
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int t = 4 * G + v;
            if (t < cnt) {
              if constexpr (TILE) {
                s_y[(slot0 + t) * kRows + col] = A::from_f32(o[0][v]);
              } else if constexpr (DUAL) {
                // reference rounding points: gate and up outputs are act
                // tensors, silu's ops each round (silu_act), and silu(gate) *
                // up rounds once more (its float32 product is exact)
                const float gv = round_act<DT>(o[0][v]);
                const float uv = round_act<DT>(o[1][v]);
                const uint16_t hv = A::from_f32(silu_act<DT>(gv) * uv);
                if constexpr (FDOWN)
                  *(uint16_t *)(hst + (slot0 - s_off[e_s] + t) * HROWB +
                                h_pos(row - b0 * kRows)) = hv;
                else
                  a.out[(int64_t)(slot0 + t) * a.out_ld + row] = hv;
              } else {
                a.out[(int64_t)s_orow[r][t] * a.out_ld + row] = A::from_f32(o[m][v]);
              }
            }
          }
        }
      }
    };

    for (int u = p0; u < p1; ++u) {
      int r, rt_unused;
      unit_of(u, r, rt_unused);
      const int cnt = __builtin_amdgcn_readfirstlane(s_round[r][2]);
      const uint8_t *arow =
          smem + (__builtin_amdgcn_readfirstlane(s_round[r][3]) + min(col, cnt - 1)) * ROWB;
      const uint8_t *ab = arow + G * 16;
      const float *gsum = (const float *)(arow + 2 * K);
      // the next unit's scales and biases, ahead of its first ring slots
      sb_issue(su_nxt, bu_nxt, nxt);
      // The single product sums its reduction in two halves, half-steps
      // [0, NS) and [NS, 2 NS) (128 columns each), each from zero, and adds
      // them at the end: the order a block that owns one half of the
      // reduction also follows (FDOWN).  Per half-step: its MFMAs, the scale
      // FMAs of its two groups, then the bias MFMA of its two groups.
      constexpr int NP = DUAL ? 1 : 2;
      f32x4 op[NP][NM];
#pragma unroll
      for (int P = 0; P < NP; ++P)
#pragma unroll
        for (int m = 0; m < NM; ++m) op[P][m] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const int d = s % D;
        // the step's scale and bias windows (groups 4s..4s+3) from lane group
        // (s % 8) / 2: dwords 2 (s % 2) and 2 (s % 2) + 1 of window s / 8
        u32x2 sv[NM], bv[NM];
#pragma unroll
        for (int m = 0; m < NM; ++m) {
          const int j = s / 8, Gp = (s % 8) / 2, w0 = 2 * (s % 2);
          const int src = (Gp * 16 + col) * 4;
          sv[m] = u32x2{(uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)su_cur[m][j][w0]),
                        (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)su_cur[m][j][w0 + 1])};
          bv[m] = u32x2{(uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)bu_cur[m][j][w0]),
                        (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)bu_cur[m][j][w0 + 1])};
        }
        // A operands of the step's eight MFMA steps and the group sums of its
        // four groups, requested before the expansion
        u32x4 af[2][4];
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int st = 0; st < 4; ++st) af[h][st] = *(const u32x4 *)(ab + a_offset(s, h, st, 0));
        // group sums: the step's four groups (lane group G: group 4s + G),
        // or per half-step its two (lane groups 0 and 1)
        const float xb = gsum[4 * s + (DUAL ? G : (G & 1))];
        const float xb2 = DUAL ? 0.f : gsum[4 * s + 2 + (G & 1)];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int P = !DUAL && 2 * s + h >= NS ? 1 : 0;
          u32x4 wh[NM];
#pragma unroll
          for (int m = 0; m < NM; ++m) wh[m] = wq[d][m][h];
          halfstep_products<DT, NM>(wh, sv, af[h], h, nib_mask, magic, op[P]);
          if constexpr (!DUAL) halfstep_bias<DT, NM>(sv, bv, h ? xb2 : xb, h, G, op[P]);
        }
        if constexpr (DUAL) {
          // bias terms of the step's four groups: lane (c, G) supplies the
          // group sum of routed row c and (b - M s) of weight row c, group
          // 4s + G
#pragma unroll
          for (int m = 0; m < NM; ++m) {
            const float scv = A::to_f32(sb_val(sv[m], G));
            const float bvv = A::to_f32(sb_val(bv[m], G));
            op[0][m] = __builtin_amdgcn_mfma_f32_16x16x4f32(xb, fmaf(-A::kMagic, scv, bvv),
                                                            op[0][m], 0, 0, 0);
          }
        }
        // refill the slot D steps ahead: this unit, or the next one.  The
        // scheduling barrier keeps each step's requests in that step (the
        // scheduler would otherwise sink them towards their use and drain
        // the ring).
        if (s + D < NS) issue(d, s + D, cur);
        else issue(d, s + D - NS, nxt);
        __builtin_amdgcn_sched_barrier(0);
      }
      f32x4 o[NM];
#pragma unroll
      for (int m = 0; m < NM; ++m) o[m] = DUAL ? op[0][m] : op[0][m] + op[NP - 1][m];
      epilogue(u, o);
      cur = nxt;
      setup(u + 2, nxt);
#pragma unroll
      for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int j = 0; j < SBW; ++j) {
          su_cur[m][j] = su_nxt[m][j];
          bu_cur[m][j] = bu_nxt[m][j];
        }
    }

    // every wavefront is done with the staged rows (FDOWN: the last phase's
    // barrier follows the first down requests, below)
    if (!FDOWN || cb + n <= c_last) __syncthreads();
    cb += n;
  }

  if constexpr (FDOWN) {
    // the first down unit's ring and windows, requested before the barrier
    // that ends the gate/up product
    {
      // (the wavefronts' first units are units 0 .. 7; the rest are taken
      // from a block counter as the wavefronts finish, so that the younger
      // wavefront of each SIMD, which the SIMD serves second, takes fewer)
      DAddr d0;
      setup_d(ri, d0);
      sb_issue_d(dsu, dbu, d0);
#pragma unroll
      for (int hsl = 0; hsl < NSDR; ++hsl) issue_d(hsl, hsl, d0);
      if (tid == 0) s_dctr = kW;
    }
    __syncthreads();
    // group sums of the h rows, formed as stage_store forms them for the
    // down product's staged rows (eight 16-byte chunks in column order, each
    // dword's pair in column order)
    for (int it = tid; it < n_e * (KH / 64); it += 64 * kW) {
      const int er = it / (KH / 64), lg = it - er * (KH / 64);
      uint8_t *hrow = hst + er * HROWB;
      float gs = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int Gi = ((i >> 2) & 1) | (((i >> 1) & 1) << 1);
        const u32x4 pv = *(const u32x4 *)(hrow + a_offset(lg >> 2, (lg >> 1) & 1,
                                                           2 * (lg & 1) + (i & 1), Gi));
        // undo pair_order: (x0,x4)(x1,x5)(x2,x6)(x3,x7) -> (x0,x1)(x2,x3)(x4,x5)(x6,x7)
        const u32x4 v = {perm_b32(pv.y, pv.x, 0x05040100u), perm_b32(pv.w, pv.z, 0x05040100u),
                         perm_b32(pv.y, pv.x, 0x07060302u), perm_b32(pv.w, pv.z, 0x07060302u)};
#pragma unroll
        for (int j = 0; j < 4; ++j) gs = A::dot2(v[j], A::kOne2, gs);
      }
      *(float *)(hrow + 2 * KH + 4 * lg) = gs;
    }
    __syncthreads();
    const int TK = (int)a.act_rows * a.a_div;
    // half P of the reduction: half-steps NSD P .. NSD P + NSD - 1 of the
    // single product's unit (compile-time, so are the window picks)
    auto down_phase = [&](auto pc) {
      constexpr int P = decltype(pc)::value;
      // the next unit from the block counter (one lane's LDS atomic)
      auto grab = [&]() {
        int v = 0;
        if (lane == 0)
          v = __hip_atomic_fetch_add(&s_dctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        return __builtin_amdgcn_readfirstlane(v);
      };
      int u = ri;        // in the ring
      int un = grab();   // requested into the ring during unit u
      while (u < dnu) {  // uniform over the wavefront
        const int q = u / dnch, c = u - q * dnch;
        const int cnt = min(kRows, n_e - kRows * c);
        const uint8_t *arow = hst + (kRows * c + min(col, cnt - 1)) * HROWB;
        const uint8_t *ab = arow + G * 16;
        const float *gsum = (const float *)(arow + 2 * KH);
        // the next unit's scales and biases, ahead of its first use
        DAddr an;
        setup_d(un, an);
        sb_issue_d(dsu_n, dbu_n, an);
        f32x4 o[NMD];
#pragma unroll
        for (int m = 0; m < NMD; ++m) o[m] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int hsl = 0; hsl < NSDR; ++hsl) {
          const int hsg = NSDR * P + hsl, sg = hsg >> 1, h = hsg & 1;
          u32x2 sv[NMD], bv[NMD];
#pragma unroll
          for (int m = 0; m < NMD; ++m) {
            const int j = sg / 8, Gp = (sg % 8) / 2, w0 = 2 * (sg % 2);
            const int src = (Gp * 16 + col) * 4;
            sv[m] = u32x2{(uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)dsu[m][j][w0]),
                          (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)dsu[m][j][w0 + 1])};
            bv[m] = u32x2{(uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)dbu[m][j][w0]),
                          (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)dbu[m][j][w0 + 1])};
          }
          u32x4 af[4];
#pragma unroll
          for (int st = 0; st < 4; ++st)
            af[st] = *(const u32x4 *)(ab + a_offset(hsl >> 1, hsl & 1, st, 0));
          const float xg = gsum[2 * hsl + (G & 1)];
          halfstep_products<DT, NMD>(dq[hsl], sv, af, h, nib_mask, magic, o);
          halfstep_bias<DT, NMD>(sv, bv, xg, h, G, o);
          // refill the slot with the next unit's half-step
          issue_d(hsl, hsl, an);
          __builtin_amdgcn_sched_barrier(0);
        }
        // this half's float32 sums, by pair
#pragma unroll
        for (int m = 0; m < NMD; ++m) {
          const int row = q * NMD * kRows + kRows * m + col;
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int t = 4 * G + v;
            if (t < cnt) {
              const int pair = s_sorted[s_off[e_s] + kRows * c + t];
              a.d_part[((int64_t)P * TK + pair) * Rd + row] = o[m][v];
            }
          }
        }
#pragma unroll
        for (int m = 0; m < NMD; ++m)
#pragma unroll
          for (int j = 0; j < SBWD; ++j) {
            dsu[m][j] = dsu_n[m][j];
            dbu[m][j] = dbu_n[m][j];
          }
        u = un;
        un = grab();
      }
    };
    if (part == 0)
      down_phase(std::integral_constant<int, 0>{});
    else
      down_phase(std::integral_constant<int, 1>{});
  }

  if constexpr (TILE) {
    // y[t][16 b + c] = rnd(sum over slots j in order of rnd(down * score)),
    // combine_kernel's arithmetic (the last phase's barrier has passed)
    const int k = a.c_k, T = (int)a.act_rows / k;
    for (int i = tid; i < T * kRows; i += 64 * kW) {
      const int t = i / kRows, c = i - t * kRows;
      const int row = (int)blockIdx.x * kRows + c;
      float acc = 0.f;
      for (int j = 0; j < k; ++j) {
        const int p = t * k + j;
        const float s = A::to_f32(s_csc[p]);
        // (a slot outside the batch, from sorted pairs that are not a
        // permutation, reads slot 0 rather than past the array)
        const int sl = s_inv[p];
        const int slc = (unsigned)sl < (unsigned)a.act_rows ? sl : 0;
        acc += round_act<DT>(A::to_f32(s_y[slc * kRows + c]) * s);
      }
      if (row < R) a.c_y[(int64_t)t * a.out_ld + row] = A::from_f32(acc);
    }
  }
}

}  // namespace

bool gemv3_supports(int K, int R, int E, int gs) {
  const int NS = K / 256;
  if (K % 256 || gs != 64 || R <= 0 || E <= 0 || E > kMaxExperts) return false;
  if (NS != 3 && NS != 6 && NS != 8 && NS != 16) return false;
  // one chunk of 16 rows fits the staging LDS; 32-bit weight offsets
  if (kRows * row_bytes(K) > kActLds) return false;
  return (int64_t)E * R * (K / 2) <= kMasked;
}

// Expert-major (STATIC) blocks pay when most experts have rows: a block
// whose expert has none ends at once, and the weights stream on the others.
// Taken when the batch has at least two routed rows per expert (with
// uniform routing about 86 % of the experts are then touched) and there are
// offsets (expert products).  NVM_GEMV_STATIC=0/1 overrides the choice.
bool use_static(const GroupedArgs &a) {
  if (!a.offsets && !a.route_part) return false;
  const char *v = getenv("NVM_GEMV_STATIC");
  if (v && (v[0] == '0' || v[0] == '1')) return v[0] == '1';
  return a.act_rows * a.a_div >= 2 * (int64_t)a.E;
}

template <int DT, bool DUAL, int NS, bool FUSED, bool STATIC, bool TILE = false, int NSD = 0>
hipError_t launch_v3(const GroupedArgs &a, hipStream_t st) {
  const int RU = DUAL || TILE ? kRows : 2 * kRows;
  const int RT = (a.R + RU - 1) / RU;
  auto *const kern = &gemv3_kernel<DT, DUAL, NS, FUSED, STATIC, TILE, NSD>;
  // more than 64 KB of dynamic LDS (once per device; a failure here shows up
  // as a failed launch below)
  static bool attr_set[64] = {false};
  int dev = 0;
  if (hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64 && !attr_set[dev]) {
    (void)hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                              kActLds);
    attr_set[dev] = true;
  }
  // STATIC: SPE blocks per expert, about one block per compute unit in all
  // (and at least one tile a block); FDOWN: two, one per half of the down
  // reduction
  // TILE: one block per 16-row tile
  const int spe =
      NSD > 0 ? 2 : STATIC ? std::max(1, std::min(cu_count() / a.E, RT)) : 1;
  const int grid = TILE ? RT : STATIC ? a.E * spe : cu_count();
  hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * kW), kActLds, st, a, RT, spe);
  return hipGetLastError();
}

template <int DT, bool DUAL, int NS>
hipError_t launch_v3_f(const GroupedArgs &a, hipStream_t st) {
  const bool stat = use_static(a);
  if constexpr (DUAL) {
    if (a.route_part)
      return stat ? launch_v3<DT, true, NS, true, true>(a, st)
                  : launch_v3<DT, true, NS, true, false>(a, st);
    return launch_v3<DT, true, NS, false, false>(a, st);
  } else {
    return stat ? launch_v3<DT, false, NS, false, true>(a, st)
                : launch_v3<DT, false, NS, false, false>(a, st);
  }
}

template <int DT, bool DUAL>
hipError_t launch_v3_ns(const GroupedArgs &a, hipStream_t st) {
  switch (a.K / 256) {
    case 3: return launch_v3_f<DT, DUAL, 3>(a, st);
    case 6: return launch_v3_f<DT, DUAL, 6>(a, st);
    case 8: return launch_v3_f<DT, DUAL, 8>(a, st);
    case 16: return launch_v3_f<DT, DUAL, 16>(a, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_gemv3(int dtype, bool dual, const GroupedArgs &a, hipStream_t st) {
  if (!gemv3_supports(a.K, a.R, a.E, a.gs)) return hipErrorInvalidValue;
  if (dtype == DT_BF16)
    return dual ? launch_v3_ns<DT_BF16, true>(a, st) : launch_v3_ns<DT_BF16, false>(a, st);
  return dual ? launch_v3_ns<DT_F16, true>(a, st) : launch_v3_ns<DT_F16, false>(a, st);
}

// The fused gate/up + down launch: the 30B-A3B decode shape (K 2048, I 768:
// a down half of three half-steps), down rows in 32-row tiles (d_R a
// multiple of 256: a whole number a wavefront), at most
// kFdRows tokens (one h row each per expert) and the fused routing's limits.
bool gemv3_fused_down_supports(int K, int R, int dR, int E, int gs, int64_t T, int k) {
  return K == 2048 && R == 2 * 128 * 3 && gemv3_supports(K, R, E, gs) &&
         gemv3_supports(R, dR, E, gs) && dR % 256 == 0 && T >= 1 && T <= kFdRows &&
         T * k <= kFusedPairs && E <= kRowExperts && k <= kRowTopK;
}

hipError_t launch_gemv3_fused_down(int dtype, const GroupedArgs &a, hipStream_t st) {
  if (!gemv3_fused_down_supports(a.K, a.R, a.d_R, a.E, a.gs, a.act_rows, a.a_div) ||
      !a.route_part || !a.d_w || !a.d_s || !a.d_b || !a.d_part)
    return hipErrorInvalidValue;
  return dtype == DT_BF16 ? launch_v3<DT_BF16, true, 8, true, true, false, 3>(a, st)
                          : launch_v3<DT_F16, true, 8, true, true, false, 3>(a, st);
}

bool gemv3_down_combine_supports(int K, int R, int E, int gs, int64_t pairs, int k) {
  return gemv3_supports(K, R, E, gs) && k >= 1 && pairs >= 1 && pairs <= kTilePairs &&
         pairs % k == 0;
}

hipError_t launch_gemv3_down_combine(int dtype, const GroupedArgs &a, hipStream_t st) {
  if (!gemv3_down_combine_supports(a.K, a.R, a.E, a.gs, a.act_rows, a.c_k) || !a.offsets ||
      !a.o_map || !a.c_scores || !a.c_y || a.route_part)
    return hipErrorInvalidValue;
  auto go = [&](auto dt) -> hipError_t {
    constexpr int D = decltype(dt)::value;
    switch (a.K / 256) {
      case 3: return launch_v3<D, false, 3, false, false, true>(a, st);
      case 6: return launch_v3<D, false, 6, false, false, true>(a, st);
      case 8: return launch_v3<D, false, 8, false, false, true>(a, st);
      case 16: return launch_v3<D, false, 16, false, false, true>(a, st);
      default: return hipErrorInvalidValue;
    }
  };
  return dtype == DT_BF16 ? go(std::integral_constant<int, DT_BF16>{})
                          : go(std::integral_constant<int, DT_F16>{});
}

}  // namespace nvm
