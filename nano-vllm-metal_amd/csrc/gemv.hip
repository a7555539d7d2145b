// Decode-regime grouped W4A16 expert products (few routed rows per expert).
//
// Replaces `mx.gather_qmm` inside grouped_expert_linear (layers/moe.py:21-32)
// for decode-sized batches, fused with SwiGLU (layers/moe.py:84,
// layers/activation.py:21-24) for the gate/up pair.
//
// Weight bytes dominate, so each expert's rows are streamed from HBM once and
// applied to every row routed to that expert (up to 16 per pass).  The inner
// product runs on the matrix cores without rounding the weights: a 4-bit code
// q becomes the exact 16-bit float M+q (M = 128 for bf16, 1024 for fp16) by
// OR-ing it into a constant, v_mfma_f32_16x16x32 accumulates x.(M+q) over one
// 64-wide quantisation group, and the group is folded in float32 as
//   sum_i x_i w_i = s * sum_i x_i (M + q_i) + (b - M s) * sum_i x_i,
// which is the reference's w = q*s + b (metal/src/quantized_matmul.cpp:135).
//
// MFMA roles (16x16x32): A = activations [16 rows x 32 k], B = weights
// [32 k x 16 output features], C[row][feature].  Lane l = (c, G), c = l%16,
// G = l/16, supplies A row c and B column c for k-slots 8G..8G+7 and holds C
// rows 4G..4G+3 of column c.
//
// Memory shape: lane (c, G) loads 16 contiguous bytes (4 packed words) of
// weight row c per load, so the four lane groups read 64 contiguous bytes of
// each of 16 rows -- two quantisation groups.  Lane groups 0-1 then hold the
// first group and 2-3 the second, so each word position feeds two MFMAs, one
// whose activation operand is zero in lane groups 2-3 (first group) and one
// zero in lane groups 0-1 (second group).  The activations of the block's
// routed rows are staged once per block in LDS, already in the pair order of
// nibble_pairs(), together with their 64-wide group sums; masked lanes read a
// row of zeros, so the masking costs no arithmetic.
#include "common.h"
#include "internal.h"

namespace nvm {

namespace {

constexpr int GI = 4;  // 64-wide groups per pipeline stage: one 128-byte line per row

// Scales and biases.  SB_ROW: each lane loads 16 bytes (8 values) of its
// row's scales and biases once per tile -- lane group G holds scale groups
// 8G..8G+7 -- and the stage fetches the value it needs from the holding lane
// with ds_bpermute.  Needs rows of an even number of scale groups (4-byte
// aligned rows) and at most 32 of them.  SB_PER_GROUP: 16-bit loads per group
// and stage, for the remaining shapes.
enum { SB_PER_GROUP = 0, SB_ROW = 1 };

// Routed rows staged per pass (MFMA rows CH..15 stay zero).  Experts with
// more routed rows take further passes over their weights.
constexpr int CH = 8;

// LDS bytes of a block: CH+1 activation rows (CH routed rows + one of zeros)
// of K/8+1 sixteen-byte chunks (the extra chunk staggers the banks of
// consecutive rows), CH group sums per 64-wide group, and 512 bytes of slack
// that a short last stage (K not a multiple of 256) may read past the end.
__host__ __device__ constexpr int gemv_lds_bytes(int K) {
  return (CH + 1) * (K / 8 + 1) * 16 + (K / 64) * CH * 4 + 512;
}
// LDS per workgroup on gfx950 is 160 KiB; 4 KiB stay for static LDS
constexpr int kMaxLds = 156 * 1024;

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

// Persistent grid: block b walks a contiguous share of the work items
// (active expert, 64*NT-row block) in expert order, so the activation rows of
// an expert are staged once per block and the grid drains evenly.
template <int DT, bool DUAL, int NT, int SB>
__global__ __launch_bounds__(256, 3) void gemv_kernel(const GroupedArgs a) {
  using A = Act<DT>;
  constexpr int NM = DUAL ? 2 : 1;
  constexpr int ROWS = 4 * 16 * NT;  // output rows of one work item
  extern __shared__ __attribute__((aligned(16))) u32x4 xl[];
  __shared__ int s_act[kMaxExperts];  // active experts, ascending
  __shared__ int s_nact;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;

  const int col = lane & 15, G = lane >> 4;
  const int KW = a.K >> 3, KG = a.K >> 6, GPR = a.K / a.gs;
  const int gsh = a.gs == 128 ? 1 : 0;
  const int pitch = KW + 1;  // LDS row pitch in 16-byte chunks
  const int zero_row = CH * pitch;
  float *sxl = (float *)(xl + (CH + 1) * pitch);  // [KG][CH]

  for (int i = tid; i < pitch; i += blockDim.x) xl[zero_row + i] = u32x4{0, 0, 0, 0};
  if (wv == 0) {
    int base = 0;
    for (int c0 = 0; c0 < a.E; c0 += 64) {
      const int e = c0 + lane;
      const bool act = e < a.E && a.offsets[e + 1] > a.offsets[e];
      const uint64_t m = __ballot(act);
      if (act) s_act[base + __popcll(m & ((1ull << lane) - 1ull))] = e;
      base += __popcll(m);
    }
    if (lane == 0) s_nact = base;
  }
  __syncthreads();
  const int RBPE = (a.R + ROWS - 1) / ROWS;
  const int W = s_nact * RBPE;
  const int i0 = (int)((int64_t)blockIdx.x * W / gridDim.x);
  const int i1 = (int)((int64_t)(blockIdx.x + 1) * W / gridDim.x);
  const int NS = (KG + GI - 1) / GI;
  int staged_e = -1, staged_nc = -1;

  for (int item = i0; item < i1; ++item) {
  const int e = s_act[item / RBPE];
  const int r0 = (item % RBPE) * ROWS + wv * 16 * NT;
  const bool wave_rows = r0 < a.R;
  const int nb = a.offsets[e], ne = a.offsets[e + 1];

  rsrc_t wr[NM], sr[NM], br[NM];
#pragma unroll
  for (int m = 0; m < NM; ++m) {
    const int64_t eo = (int64_t)e * a.R;
    wr[m] = make_rsrc((m ? a.w1 : a.w0) + eo * KW, (uint32_t)(a.R * KW * 4));
    sr[m] = make_rsrc((m ? a.s1 : a.s0) + eo * GPR, (uint32_t)(a.R * GPR * 2));
    br[m] = make_rsrc((m ? a.b1 : a.b0) + eo * GPR, (uint32_t)(a.R * GPR * 2));
  }
  int wo[NT], so[NT];
  bool tv[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    tv[t] = r0 + 16 * t < a.R;
    const int row = r0 + 16 * t + col;
    wo[t] = tv[t] ? (row * KW + 4 * G) * 4 : kMaskedOffset;
    so[t] = tv[t] ? row * GPR * 2 : kMaskedOffset;
  }

  // one pipeline stage = 4 groups: two 16-byte loads per (matrix, row tile);
  // with SB_PER_GROUP also the stage's scales/biases, packed (value of group
  // gi in half (gi & 1) of dword gi >> 1)
  struct Stage {
    u32x4 q[NM][NT][2];
    u32x2 s[NM][NT], b[NM][NT];
  };
  auto load = [&](int st_idx, Stage &st) {
    const int ws = __builtin_amdgcn_readfirstlane(128 * st_idx);
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        st.q[m][t][0] = bload16(wr[m], wo[t], ws);
        st.q[m][t][1] = bload16(wr[m], wo[t] + 64, ws);
        if constexpr (SB == SB_PER_GROUP) {
          uint32_t sv[GI], bv[GI];
#pragma unroll
          for (int gi = 0; gi < GI; ++gi) {
            sv[gi] = bload2(sr[m], so[t] + 2 * ((GI * st_idx + gi) >> gsh), 0);
            bv[gi] = bload2(br[m], so[t] + 2 * ((GI * st_idx + gi) >> gsh), 0);
          }
          st.s[m][t] = u32x2{sv[0] | (sv[1] << 16), sv[2] | (sv[3] << 16)};
          st.b[m][t] = u32x2{bv[0] | (bv[1] << 16), bv[2] | (bv[3] << 16)};
        }
      }
  };
  // SB_ROW: the tile's scales/biases, resident for the whole wavefront
  u32x4 srow[NM][NT], brow[NM][NT];
  if constexpr (SB == SB_ROW) {
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        srow[m][t] = bload16(sr[m], so[t] + 16 * G, 0);
        brow[m][t] = bload16(br[m], so[t] + 16 * G, 0);
      }
  }
  // dword holding the scale/bias values of 64-wide groups (g, g + 1), g even:
  // both share one 32-bit word of the resident row (group 64) or are the same
  // value (group 128, duplicated into both halves)
  auto sb_pair = [&](const u32x4 &row, int g) -> uint32_t {
    const int sg = g >> gsh;  // scale group of g
    const int src = col + 16 * (sg >> 3);
    const int w = (sg & 7) >> 1;
    const uint32_t mine = w == 0 ? row.x : w == 1 ? row.y : w == 2 ? row.z : row.w;
    const uint32_t d = (uint32_t)__builtin_amdgcn_ds_bpermute(src << 2, (int)mine);
    if (gsh == 0) return d;
    const uint32_t h = (sg & 1) ? (d >> 16) : (d & 0xFFFFu);
    return h * 0x10001u;
  };

  const int rot = __builtin_amdgcn_readfirstlane(
      (int)((item * 4u + wv + 3u * e) % (unsigned)NS));
  auto st_at = [&](int i) {
    const int st = rot + i;
    return st >= NS ? st - NS : st;
  };

  for (int nc = nb; nc < ne; nc += CH) {
    const int cnt = min(CH, ne - nc);
    // the first two weight stages do not depend on the activations: issue
    // them before staging so their latency overlaps the staging
    Stage sa, sb, sc;
    if (wave_rows) {
      load(st_at(0), sa);
      if (NS > 1) load(st_at(1), sb);
    }
    if (e != staged_e || nc != staged_nc) {
    staged_e = e;
    staged_nc = nc;
    __syncthreads();  // every wavefront is done with the previous rows
    // stage the routed activation rows (pair order) and their group sums
    for (int it = tid; it < cnt * KW; it += blockDim.x) {
      const int c = it / KW, ch = it - c * KW;
      const int arow = a.a_map ? a.a_map[nc + c] / a.a_div : nc + c;
      const u32x4 v = ldg16(a.act + (int64_t)arow * a.act_ld + 8 * ch);
      xl[c * pitch + ch] = pair_order(v);
      float sx = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) sx = A::dot2(v[i], A::kOne2, sx);
      // 8 consecutive items (lanes) form one 64-wide group
      sx += __shfl_xor(sx, 1);
      sx += __shfl_xor(sx, 2);
      sx += __shfl_xor(sx, 4);
      if ((ch & 7) == 0) sxl[(ch >> 3) * CH + c] = sx;
    }
    __syncthreads();
    }
    if (!wave_rows) continue;

    const bool tok_ok = col < cnt;
    const int lo_base = (tok_ok && G < 2) ? col * pitch + 4 * G : zero_row + 4 * G;
    const int hi_base = (tok_ok && G >= 2) ? col * pitch + 4 * G : zero_row + 4 * G;

    f32x4 o[NM][NT];
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
      for (int t = 0; t < NT; ++t) o[m][t] = f32x4{0.f, 0.f, 0.f, 0.f};

    // ng = valid groups of the stage (GI except in a short last stage)
    auto compute = [&](int st_idx, const Stage &st, int ng) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        if (2 * j >= ng) break;
        const bool has_b = 2 * j + 1 < ng;
        const int cbase = 32 * st_idx + 16 * j;
        f32x4 acc_a[NM][NT], acc_b[NM][NT];
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
          for (int t = 0; t < NT; ++t) {
            acc_a[m][t] = f32x4{0.f, 0.f, 0.f, 0.f};
            acc_b[m][t] = f32x4{0.f, 0.f, 0.f, 0.f};
          }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const u32x4 alo = xl[lo_base + cbase + k];
          const u32x4 ahi = xl[hi_base + cbase + k];
#pragma unroll
          for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int t = 0; t < NT; ++t) {
              if (!tv[t]) continue;
              const u32x4 bq = nibble_pairs<DT>(st.q[m][t][j][k]);
              acc_a[m][t] = A::mfma16(alo, bq, acc_a[m][t]);
              acc_b[m][t] = A::mfma16(ahi, bq, acc_b[m][t]);
            }
        }
        // group sums of the lane's C rows 4G..4G+3 (rows >= CH are never stored)
        const int ga = GI * st_idx + 2 * j;
        const int gq = min(4 * G, CH - 4);
        const f32x4 sxa = *(const f32x4 *)(sxl + ga * CH + gq);
        const f32x4 sxb = *(const f32x4 *)(sxl + (ga + 1) * CH + gq);
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
          for (int t = 0; t < NT; ++t) {
            if (!tv[t]) continue;
            uint32_t sd, bd;
            if constexpr (SB == SB_ROW) {
              sd = sb_pair(srow[m][t], ga);
              bd = sb_pair(brow[m][t], ga);
            } else {
              sd = st.s[m][t][j];
              bd = st.b[m][t][j];
            }
            const float s0 = A::lo(sd), b0 = A::lo(bd);
            const float bp0 = fmaf(-A::kMagic, s0, b0);
#pragma unroll
            for (int v = 0; v < 4; ++v) o[m][t][v] = fmaf(s0, acc_a[m][t][v], fmaf(bp0, sxa[v], o[m][t][v]));
            if (has_b) {
              const float s1 = A::hi(sd), b1 = A::hi(bd);
              const float bp1 = fmaf(-A::kMagic, s1, b1);
#pragma unroll
              for (int v = 0; v < 4; ++v)
                o[m][t][v] = fmaf(s1, acc_b[m][t][v], fmaf(bp1, sxb[v], o[m][t][v]));
            }
          }
      }
    };

    // Three stage buffers in rotation keep two stages of weights in flight
    // while one is multiplied; nothing is copied between buffers.  Every pass
    // of the main loop issues the same loads, which lets the compiler wait
    // only for the stage about to be used.  Wavefronts start at different
    // stages of their rows so that concurrent wavefronts do not sweep the
    // same column offsets (and memory channels) in lockstep.
    auto run = [&](int i, const Stage &st) { compute(st_at(i), st, min(GI, KG - GI * st_at(i))); };
    int i = 0;
    for (; i + 4 < NS; i += 3) {
      load(st_at(i + 2), sc);
      run(i, sa);
      load(st_at(i + 3), sa);
      run(i + 1, sb);
      load(st_at(i + 4), sb);
      run(i + 2, sc);
    }
    // 1 to 4 stages remain: sa holds stage i, sb stage i + 1
    if (i + 2 < NS) load(st_at(i + 2), sc);
    run(i, sa);
    if (i + 1 < NS) {
      if (i + 3 < NS) load(st_at(i + 3), sa);
      run(i + 1, sb);
      if (i + 2 < NS) run(i + 2, sc);
      if (i + 3 < NS) run(i + 3, sa);
    }

#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (!tv[t]) continue;
      const int rowc = r0 + 16 * t + col;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int tok = 4 * G + v;
        if (tok >= cnt) continue;
        const int n = nc + tok;
        const int64_t orow = a.o_map ? a.o_map[n] : n;
        uint16_t r;
        if (DUAL) {
          // reference rounding points: gate and up outputs are act tensors,
          // silu(gate) * up is rounded once more
          const float gv = round_act<DT>(o[0][t][v]);
          const float uv = round_act<DT>(o[NM - 1][t][v]);
          r = A::from_f32(gv / (1.0f + __expf(-gv)) * uv);
        } else {
          r = A::from_f32(o[0][t][v]);
        }
        a.out[orow * a.out_ld + rowc] = r;
      }
    }
  }
  }
}

template <int DT, bool DUAL, int NT>
hipError_t launch_nt(const GroupedArgs &a, int sb_mode, hipStream_t st) {
  constexpr int WAVES = 4;
  const int rows_per_block = 16 * NT * WAVES;
  // work items can number at most E * ceil(R / rows); three blocks per CU
  // are resident at once (register-limited), so launch no more than that
  const int64_t items = (int64_t)a.E * ((a.R + rows_per_block - 1) / rows_per_block);
  dim3 grid((unsigned)std::min<int64_t>(items, 3 * (int64_t)cu_count()));
  const size_t lds = gemv_lds_bytes(a.K);
  if (lds > (size_t)kMaxLds) return hipErrorInvalidValue;
  // allow dynamic LDS beyond the 64 KiB default (once per instantiation)
  static const hipError_t attr[2] = {
      hipFuncSetAttribute((const void *)gemv_kernel<DT, DUAL, NT, SB_PER_GROUP>,
                          hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds),
      hipFuncSetAttribute((const void *)gemv_kernel<DT, DUAL, NT, SB_ROW>,
                          hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds)};
  for (hipError_t e : attr)
    if (e != hipSuccess) return e;
  if (sb_mode == SB_ROW)
    hipLaunchKernelGGL((gemv_kernel<DT, DUAL, NT, SB_ROW>), grid, dim3(64 * WAVES), lds, st, a);
  else
    hipLaunchKernelGGL((gemv_kernel<DT, DUAL, NT, SB_PER_GROUP>), grid, dim3(64 * WAVES), lds,
                       st, a);
  return hipGetLastError();
}

template <int DT>
hipError_t launch_t(bool dual, const GroupedArgs &a, hipStream_t st) {
  const int gpr = a.K / a.gs;
  const int sb_mode = (gpr % 2 == 0 && gpr <= 32) ? SB_ROW : SB_PER_GROUP;
  // gate/up: one 16-row tile of both matrices per wavefront; down: two tiles
  return dual ? launch_nt<DT, true, 1>(a, sb_mode, st) : launch_nt<DT, false, 2>(a, sb_mode, st);
}

}  // namespace

hipError_t launch_gemv(int dtype, bool dual, const GroupedArgs &a, hipStream_t st) {
  return dtype == DT_BF16 ? launch_t<DT_BF16>(dual, a, st) : launch_t<DT_F16>(dual, a, st);
}

}  // namespace nvm
