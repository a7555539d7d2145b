// Paged attention over a paged KV cache (declared in include/nvm_attention.h).
//
// Restates the reference's op metal/src/paged_attention.cpp (CPU loop
// :122-296, int8 decode loop :298-410, decode split-K kernel
// paged_attention.metal:277-409): per query row, an online softmax in float32
// over the key positions j < min(context_len, max_pages * page_size) whose
// page id (block_table[b, j / page_size]) is not negative, causal rows seeing
// j <= i + context_len - L, then the probability-weighted sum of the values.
// Pages are [P, num_kv_heads, page_size, D] (cache/paged.py).
//
// Decode kernel (L = 1, f16/bf16 pages, D = 64 or 128).  A block owns one
// (request, kv head, group of up to RP query heads, context split): the query
// heads that share a kv head read each key and value row once (grouped-query
// sharing; the reference reads them once per query head).  Its eight
// wavefronts take 64-position tiles of the split in turn, each with its
// tile's keys and values in registers (one memory round trip a tile; eight
// wavefronts keep twice the tiles in flight that four did).
//   * Scores on the matrix cores, S^T = K . Q^T with v_mfma_f32_16x16x32 in
//     the page dtype: the key rows are the A operand straight from memory
//     (lane (c, G) loads 16 bytes: position c of a 16-row subtile, dims
//     32k + 8G .. +7), and the float32 query is split into three page-dtype
//     parts q = q1 + q2 + q3 (exact for bf16; for f16 to the f16 subnormal
//     range), so every product is exact and the sums are float32 as in the
//     reference.  C holds head c, positions 4G..4G+3 of each subtile.
//   * Softmax in base 2 (scores pre-scaled by scale * log2 e): the tile's
//     row maximum is two lane swaps, the row sums stay lane-partial.
//   * P . V on the matrix cores as well, O^T += V^T . P^T per 32-position
//     chunk: the S^T layout leaves each lane holding exactly its B operand
//     (its head's probabilities at the chunk's k-slots), split into three
//     page-dtype parts like q; the value rows (16-byte loads issued with the
//     key loads) are staged in LDS and read back transposed as the A operand.
//   * The wavefronts' (max, sum, output) partials meet in LDS; with more
//     than one split per row they go to the workspace and a second launch
//     combines them.
// Other shapes (L > 1, f32 or int8 pages, other head dims) run one wavefront
// per query row over the context, with the reference's formula per element.
#include <math.h>

#include <algorithm>

#include "common.h"
#include "internal.h"
#include "nvm_attention.h"

namespace nvm {

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kTile = 64;           // context positions per wavefront step
constexpr int kTargetBlocks = 256;  // decode: split the context until about this many blocks
constexpr int kDecodeWaves = 8;     // decode: wavefronts per block (tiles in flight per block)
constexpr int kMaxRowDim = 256;     // head dim of the row kernel (4 values per lane)
constexpr int kMaxSplits = 64;      // context splits of a decode row

struct PagedArgs {
  const float *q;
  const void *kp, *vp;
  const float *ks, *vs;
  const int32_t *bt, *lens;
  void *out;
  float *part_o, *part_ml;
  int out_dt;  // NVM_KV_F32, NVM_KV_BF16 or NVM_KV_F16
  int P, L, D, page_size, max_pages, Hkv, Hq, R, HG, S, span, causal;
  float scale2;  // scale * log2(e): scores are kept in base 2
};

// Output element i: float32, or rounded to bf16/f16 (the model's
// `.astype(x.dtype)` after the op, models/qwen3.py:150-161).
__device__ __forceinline__ void store_out(void *out, int dt, int64_t i, float v) {
  if (dt == NVM_KV_F32)
    ((float *)out)[i] = v;
  else if (dt == NVM_KV_BF16)
    ((uint16_t *)out)[i] = Act<DT_BF16>::from_f32(v);
  else
    ((uint16_t *)out)[i] = Act<DT_F16>::from_f32(v);
}

// Hand-over of LDS data between the lanes of one wavefront: its LDS
// operations execute in program order, so only the compiler must not move
// loads or stores across this point.
__device__ __forceinline__ void wave_lds_sync() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_wave_barrier();
  asm volatile("" ::: "memory");
}

// q = p0 + p1 + p2 in the page dtype, for four pairs of values.
template <int DT>
__device__ __forceinline__ void split3(const float (&x)[8], u32x4 &p0, u32x4 &p1, u32x4 &p2) {
  using A = Act<DT>;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float a0 = x[2 * i], a1 = x[2 * i + 1];
    const uint32_t h = A::pack2(a0, a1);
    a0 -= A::lo(h);
    a1 -= A::hi(h);
    const uint32_t m = A::pack2(a0, a1);
    a0 -= A::lo(m);
    a1 -= A::hi(m);
    p0[i] = h;
    p1[i] = m;
    p2[i] = A::pack2(a0, a1);
  }
}

template <int DT, int DH, int RP, int NW>
__global__ __launch_bounds__(64 * NW) void paged_decode_kernel(PagedArgs a) {
  using A = Act<DT>;
  constexpr int NC = DH / 32;        // 32-dim chunks of a score MFMA
  constexpr int NT = DH / 16;        // 16-dim output tiles of a P.V MFMA
  constexpr int LPD = DH / 8;        // lanes per value row in the V loads, 8 dims each
  constexpr int PG = 64 / LPD;       // position groups of the V loads
  constexpr int PPG = kTile / PG;    // positions per lane per tile
  constexpr int VP = DH + 8;         // LDS pitch of a staged value row (16-bit elements)
  // one 32-position chunk of values per wavefront during the tile loop; the
  // wavefronts' output partials afterwards (the same LDS)
  constexpr int kVBytes = NW * 32 * VP * 2, kOBytes = NW * RP * DH * 4;
  __shared__ __attribute__((aligned(16))) char s_buf[kVBytes > kOBytes ? kVBytes : kOBytes];
  auto s_v = reinterpret_cast<uint16_t(*)[32][VP]>(s_buf);
  auto s_o = reinterpret_cast<float(*)[RP][DH]>(s_buf);
  __shared__ u32x4 s_q[NC][3][64];  // the score MFMAs' B operand, per lane
  __shared__ int s_row[NW][kTile];
  __shared__ float s_m[NW][RP], s_l[NW][RP];

  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int c16 = lane & 15, G = lane >> 4;
  int blk = blockIdx.x;
  const int s = blk % a.S;
  blk /= a.S;
  const int hg = blk % a.HG;
  blk /= a.HG;
  const int kvh = blk % a.Hkv;
  const int b = blk / a.Hkv;
  const int nh = min(RP, a.R - hg * RP);
  const int64_t n0 = (int64_t)b * a.Hq + (int64_t)kvh * a.R + hg * RP;
  const int ctx = min(a.lens[b], a.max_pages * a.page_size);
  const int p0 = s * a.span;
  const int p1 = min(p0 + a.span, ctx);

  // B operand of the score MFMAs (query head c16, dims 32k + 8G .. +7), the
  // same for every wavefront: built once into LDS, read back per tile (it
  // would hold 12 * NC VGPRs for the whole loop)
  if (wv == 0) {
    const bool ok = c16 < nh;
    const float *qp = a.q + (n0 + (ok ? c16 : 0)) * DH;
#pragma unroll
    for (int k = 0; k < NC; ++k) {
      const int d0 = 32 * k + 8 * G;
      const f32x4 x0 = ok ? *(const f32x4 *)(qp + d0) : f32x4{0.f, 0.f, 0.f, 0.f};
      const f32x4 x1 = ok ? *(const f32x4 *)(qp + d0 + 4) : f32x4{0.f, 0.f, 0.f, 0.f};
      const float x[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
      u32x4 q0, q1, q2;
      split3<DT>(x, q0, q1, q2);
      s_q[k][0][lane] = q0;
      s_q[k][1][lane] = q1;
      s_q[k][2][lane] = q2;
    }
  }
  __syncthreads();

  const uint32_t kv_bytes = (uint32_t)((int64_t)a.P * a.Hkv * a.page_size * DH * 2);
  const rsrc_t kr = make_rsrc(a.kp, kv_bytes), vr = make_rsrc(a.vp, kv_bytes);
  const int64_t bt_row = (int64_t)b * a.max_pages;
  const int dd = 8 * (lane % LPD), pgrp = lane / LPD;

  float m_run = -INFINITY, l_run = 0.f;  // head c16; l_run is this lane's share
  // O^T tiles: lane (c16, G) holds head c16, dims 16t + 4G + i
  f32x4 oacc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) oacc[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  // page ids of positions t0 + 16u + c16, one tile ahead of their use
  auto page_ids = [&](int t0, int (&pg)[4]) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int pos = t0 + 16 * u + c16;
      pg[u] = pos < p1 ? a.bt[bt_row + pos / a.page_size] : -1;
    }
  };
  int pg_next[4];
  page_ids(p0 + kTile * wv, pg_next);
  for (int t0 = p0 + kTile * wv; t0 < p1; t0 += NW * kTile) {
    // element offsets of the key/value rows of positions t0 + 16u + c16
    int rowoff[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int pos = t0 + 16 * u + c16;
      const int pg = pg_next[u];
      rowoff[u] = (pg >= 0 && pg < a.P)
                      ? ((pg * a.Hkv + kvh) * a.page_size + pos % a.page_size) * DH
                      : -1;
    }
    page_ids(t0 + NW * kTile, pg_next);
    u32x4 kop[4][NC];
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int k = 0; k < NC; ++k)
        kop[u][k] = bload16(kr, rowoff[u] >= 0 ? (rowoff[u] + 32 * k + 8 * G) * 2 : kMaskedOffset, 0);
    uint32_t vmask[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      vmask[u] = (uint32_t)__builtin_amdgcn_ballot_w64(rowoff[u] >= 0) & 0xFFFFu;
      if (G == 0) s_row[wv][16 * u + c16] = rowoff[u];
    }
    wave_lds_sync();
    // the value rows, loaded with the keys (one memory round trip per tile):
    // lane group pgrp holds dims dd..dd+7 of positions pgrp + PG*mm
    u32x4 vv[PPG];
#pragma unroll
    for (int mm = 0; mm < PPG; ++mm) {
      const int ro = s_row[wv][pgrp + PG * mm];
      vv[mm] = bload16(vr, ro >= 0 ? (ro + dd) * 2 : kMaskedOffset, 0);
    }

    // S^T: lane (c16, G) holds head c16 at positions 16u + 4G + i
    f32x4 acc[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      acc[u] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < NC; ++k)
#pragma unroll
        for (int part = 0; part < 3; ++part)
          acc[u] = A::mfma16(kop[u][k], s_q[k][part][lane], acc[u]);
    }
    float sc[4][4];
    float tmax = -INFINITY;
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bool valid = (vmask[u] >> (4 * G + i)) & 1u;
        sc[u][i] = valid ? acc[u][i] * a.scale2 : -INFINITY;
        tmax = fmaxf(tmax, sc[u][i]);
      }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
    const float m_new = fmaxf(m_run, tmax);
    const bool any = m_new != -INFINITY;
    const float alpha = any ? exp2f(m_run - m_new) : 1.f;
    float psum = 0.f;
    float pv[4][4];
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pv[u][i] = any ? exp2f(sc[u][i] - m_new) : 0.f;
        psum += pv[u][i];
      }
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int t = 0; t < NT; ++t) oacc[t] *= alpha;

    // P . V on the matrix cores, one 32-position chunk at a time: O^T += V^T P^T.
    // k-slot 8G + j of the chunk is position 4G + j (j < 4) or 16 + 4G + j - 4,
    // so the B operand (P^T, head c16) is this lane's own probabilities of
    // subtiles 2kc and 2kc+1, and the A operand (V^T, dim 16t + c16) is read
    // from the chunk staged in LDS (pitch VP keeps the four lane groups on
    // disjoint banks).
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
#pragma unroll
      for (int mm = kc * (32 / PG); mm < (kc + 1) * (32 / PG); ++mm)
        *(u32x4 *)&s_v[wv][pgrp + PG * mm - 32 * kc][dd] = vv[mm];
      wave_lds_sync();
      const float x[8] = {pv[2 * kc][0], pv[2 * kc][1], pv[2 * kc][2], pv[2 * kc][3],
                          pv[2 * kc + 1][0], pv[2 * kc + 1][1], pv[2 * kc + 1][2],
                          pv[2 * kc + 1][3]};
      u32x4 pb[3];
      split3<DT>(x, pb[0], pb[1], pb[2]);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int d = 16 * t + c16;
        u32x4 va;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int r0 = jj < 2 ? 4 * G + 2 * jj : 16 + 4 * G + 2 * jj - 4;
          va[jj] = (uint32_t)s_v[wv][r0][d] | ((uint32_t)s_v[wv][r0 + 1][d] << 16);
        }
#pragma unroll
        for (int part = 0; part < 3; ++part) oacc[t] = A::mfma16(va, pb[part], oacc[t]);
      }
      wave_lds_sync();
    }
  }

  // the lane shares of the row sums; the outputs are whole in oacc
  l_run += __shfl_xor(l_run, 16);
  l_run += __shfl_xor(l_run, 32);
  __syncthreads();  // every wavefront is past its last use of s_v
  if (c16 < RP) {
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) s_o[wv][c16][16 * t + 4 * G + i] = oacc[t][i];
  }
  if (G == 0 && c16 < RP) {
    s_m[wv][c16] = m_run;
    s_l[wv][c16] = l_run;
  }
  __syncthreads();

  for (int e = threadIdx.x; e < RP * DH; e += 64 * NW) {
    const int r = e / DH, d = e % DH;
    if (r >= nh) continue;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, s_m[w][r]);
    float Ls = 0.f, Os = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float mw = s_m[w][r];
      if (mw != -INFINITY) {
        const float f = exp2f(mw - M);
        Ls += f * s_l[w][r];
        Os += f * s_o[w][r][d];
      }
    }
    const int64_t n = n0 + r;
    if (a.S == 1) {
      store_out(a.out, a.out_dt, n * DH + d, Ls > 0.f ? Os / Ls : 0.f);
    } else {
      a.part_o[(n * a.S + s) * DH + d] = Os;
      if (d == 0) {
        a.part_ml[(n * a.S + s) * 2] = M;
        a.part_ml[(n * a.S + s) * 2 + 1] = Ls;
      }
    }
  }
}

// Splits of a row: out = sum_s 2^(M_s - M) O_s / sum_s 2^(M_s - M) L_s.
// One block per row: the splits' (M_s, L_s) are read in parallel into LDS,
// then thread d sums its dim over the splits with the loads of eight splits
// in flight at a time.
__global__ __launch_bounds__(256) void paged_combine_kernel(const float *__restrict__ part_o,
                                                            const float *__restrict__ part_ml,
                                                            int S, int D, void *out,
                                                            int out_dt) {
  __shared__ float s_w[kMaxSplits];
  __shared__ float s_inv;
  const int64_t n = blockIdx.x;
  const float *ml = part_ml + n * S * 2;
  const int t = threadIdx.x;
  if (t < 64) {
    // wavefront 0: the row maximum and the weighted sum of the L_s
    float M = -INFINITY;
    for (int s = t; s < S; s += 64) M = fmaxf(M, ml[2 * s]);
#pragma unroll
    for (int x = 32; x > 0; x >>= 1) M = fmaxf(M, __shfl_xor(M, x));
    float Ls = 0.f;
    for (int s = t; s < S; s += 64) {
      const float ms = ml[2 * s];
      const float w = ms != -INFINITY ? exp2f(ms - M) : 0.f;
      s_w[s] = w;
      Ls += w * ml[2 * s + 1];
    }
#pragma unroll
    for (int x = 32; x > 0; x >>= 1) Ls += __shfl_xor(Ls, x);
    if (t == 0) s_inv = Ls > 0.f ? 1.f / Ls : 0.f;
  }
  __syncthreads();
  for (int d = t; d < D; d += 256) {
    const float *po = part_o + n * S * D + d;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    int s = 0;
    for (; s + 8 <= S; s += 8) {
#pragma unroll
      for (int u = 0; u < 8; ++u) acc[u] += s_w[s + u] * po[(int64_t)(s + u) * D];
    }
    for (; s < S; ++s) acc[0] += s_w[s] * po[(int64_t)s * D];
    const float o = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
    store_out(out, out_dt, n * D + d, o * s_inv);
  }
}

template <int KVT>
__device__ __forceinline__ float kv_at(const void *base, int64_t i) {
  if constexpr (KVT == NVM_KV_F32) return ((const float *)base)[i];
  if constexpr (KVT == NVM_KV_I8) return (float)((const int8_t *)base)[i];
  if constexpr (KVT == NVM_KV_BF16) return Act<DT_BF16>::to_f32(((const uint16_t *)base)[i]);
  return Act<DT_F16>::to_f32(((const uint16_t *)base)[i]);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int x = 32; x > 0; x >>= 1) v += __shfl_xor(v, x);
  return v;  // the same in every lane: each step adds the same two operands
}

// One wavefront per query row (n, i): lanes hold dims lane + 64k; positions
// in order, the score reduced across the wavefront, online softmax.
template <int KVT>
__global__ __launch_bounds__(256) void paged_rows_kernel(PagedArgs a, int64_t rows) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  const int64_t n = row / a.L;
  const int i = (int)(row - n * a.L);
  const int b = (int)(n / a.Hq);
  const int kvh = (int)(n % a.Hq) / a.R;
  const int ctx_len = a.lens[b];
  const int ctx = min(ctx_len, a.max_pages * a.page_size);
  const int last = a.causal ? min(ctx, i + ctx_len - a.L + 1) : ctx;
  constexpr int KD = kMaxRowDim / 64;
  float qv[KD], ov[KD];
#pragma unroll
  for (int k = 0; k < KD; ++k) {
    const int d = lane + 64 * k;
    qv[k] = d < a.D ? a.q[row * a.D + d] : 0.f;
    ov[k] = 0.f;
  }
  float m = -INFINITY, l = 0.f;
  for (int j = 0; j < last; ++j) {
    const int pg = a.bt[(int64_t)b * a.max_pages + j / a.page_size];
    if (pg < 0 || pg >= a.P) continue;
    const int64_t slot = ((int64_t)pg * a.Hkv + kvh) * a.page_size + j % a.page_size;
    const float ksc = KVT == NVM_KV_I8 ? a.ks[slot] : 1.f;
    const float vsc = KVT == NVM_KV_I8 ? a.vs[slot] : 1.f;
    float dot = 0.f;
#pragma unroll
    for (int k = 0; k < KD; ++k) {
      const int d = lane + 64 * k;
      if (d < a.D) {
        const float kx = kv_at<KVT>(a.kp, slot * a.D + d);
        dot += qv[k] * (KVT == NVM_KV_I8 ? kx * ksc : kx);
      }
    }
    const float sc = wave_sum(dot) * a.scale2;
    const float m_new = fmaxf(m, sc);
    const float alpha = exp2f(m - m_new);
    const float p = exp2f(sc - m_new);
    l = l * alpha + p;
#pragma unroll
    for (int k = 0; k < KD; ++k) {
      const int d = lane + 64 * k;
      if (d < a.D) {
        const float vx = kv_at<KVT>(a.vp, slot * a.D + d);
        ov[k] = ov[k] * alpha + p * (KVT == NVM_KV_I8 ? vx * vsc : vx);
      }
    }
    m = m_new;
  }
#pragma unroll
  for (int k = 0; k < KD; ++k) {
    const int d = lane + 64 * k;
    if (d < a.D) store_out(a.out, a.out_dt, row * a.D + d, l > 0.f ? ov[k] / l : 0.f);
  }
}

struct AttnPlan {
  bool decode;  // the split-context decode kernel
  int RP, HG, S, span;
};

AttnPlan attn_plan(int64_t N, int64_t L, int64_t D, int64_t max_pages, int64_t page_size,
                   int kv_dtype, int Hkv, int Hq) {
  AttnPlan p{false, 0, 1, 1, 0};
  p.decode = L == 1 && (kv_dtype == NVM_KV_F16 || kv_dtype == NVM_KV_BF16) && (D == 64 || D == 128);
  if (!p.decode) return p;
  const int R = Hq / Hkv;
  p.RP = R <= 8 ? 8 : 16;
  p.HG = (R + p.RP - 1) / p.RP;
  const int64_t tiles = (max_pages * page_size + kTile - 1) / kTile;
  const int64_t base = N / Hq * Hkv * p.HG;
  const int64_t s0 = std::max<int64_t>(1, (kTargetBlocks + base - 1) / base);
  int64_t tps = std::max<int64_t>(1, (tiles + s0 - 1) / s0);
  tps = std::max<int64_t>(tps, (tiles + kMaxSplits - 1) / kMaxSplits);
  p.S = (int)std::max<int64_t>(1, (tiles + tps - 1) / tps);
  p.span = (int)(tps * kTile);
  return p;
}

size_t attn_workspace(const AttnPlan &p, int64_t N, int64_t D) {
  if (!p.decode || p.S == 1) return 0;
  const size_t o = ((size_t)N * p.S * D * sizeof(float) + 255) & ~(size_t)255;
  return o + (((size_t)N * p.S * 2 * sizeof(float) + 255) & ~(size_t)255);
}

template <int DT>
void launch_decode(const PagedArgs &a, int RP, int D, unsigned grid, hipStream_t st) {
  if (D == 128) {
    if (RP == 8)
      hipLaunchKernelGGL((paged_decode_kernel<DT, 128, 8, kDecodeWaves>), dim3(grid),
                         dim3(64 * kDecodeWaves), 0, st, a);
    else
      hipLaunchKernelGGL((paged_decode_kernel<DT, 128, 16, kDecodeWaves>), dim3(grid),
                         dim3(64 * kDecodeWaves), 0, st, a);
  } else {
    if (RP == 8)
      hipLaunchKernelGGL((paged_decode_kernel<DT, 64, 8, kDecodeWaves>), dim3(grid),
                         dim3(64 * kDecodeWaves), 0, st, a);
    else
      hipLaunchKernelGGL((paged_decode_kernel<DT, 64, 16, kDecodeWaves>), dim3(grid),
                         dim3(64 * kDecodeWaves), 0, st, a);
  }
}

#define ATTN_REQUIRE(cond, ...)                                              \
  do {                                                                       \
    if (!(cond)) return set_error(NVM_ERR_INVALID, __VA_ARGS__);             \
  } while (0)
#define ATTN_SUPPORTED(cond, ...)                                            \
  do {                                                                       \
    if (!(cond)) return set_error(NVM_ERR_UNSUPPORTED, __VA_ARGS__);         \
  } while (0)

int check_attention(int64_t N, int64_t L, int64_t D, int64_t max_pages, int64_t page_size,
                    int kv_dtype, int num_kv_heads, int num_heads) {
  ATTN_REQUIRE(num_heads > 0 && num_kv_heads > 0 && num_heads % num_kv_heads == 0,
               "paged_attention: num_heads must be divisible by num_kv_heads");
  ATTN_REQUIRE(N >= 0 && N % num_heads == 0,
               "paged_attention: q.shape[0] must be divisible by num_heads");
  ATTN_REQUIRE(L >= 1 && D >= 1 && page_size >= 1 && max_pages >= 0,
               "paged_attention: bad shape L=%lld D=%lld page_size=%lld max_pages=%lld",
               (long long)L, (long long)D, (long long)page_size, (long long)max_pages);
  ATTN_REQUIRE(kv_dtype >= NVM_KV_F16 && kv_dtype <= NVM_KV_I8, "paged_attention: bad kv dtype %d",
               kv_dtype);
  ATTN_SUPPORTED(D <= kMaxRowDim, "paged_attention: head dimension at most %d", kMaxRowDim);
  ATTN_SUPPORTED(max_pages * page_size <= 0x7FFFFFFFll, "paged_attention: context capacity too large");
  return NVM_OK;
}

}  // namespace

}  // namespace nvm

extern "C" {

int nvm_paged_attention_workspace_size(int64_t N, int64_t L, int64_t D, int64_t max_pages,
                                       int64_t page_size, int kv_dtype, int num_kv_heads,
                                       int num_heads, size_t *bytes) {
  using namespace nvm;
  if (int r = check_attention(N, L, D, max_pages, page_size, kv_dtype, num_kv_heads, num_heads))
    return r;
  if (!bytes) return set_error(NVM_ERR_INVALID, "paged_attention: null bytes");
  *bytes = attn_workspace(attn_plan(N, L, D, max_pages, page_size, kv_dtype, num_kv_heads,
                                    num_heads),
                          N, D);
  return NVM_OK;
}

int nvm_paged_attention(const float *q, int64_t N, int64_t L, int64_t D, const void *key_pages,
                        const void *value_pages, int64_t P, int64_t page_size, int kv_dtype,
                        const float *key_scales, const float *value_scales,
                        const int32_t *block_table, int64_t B, int64_t max_pages,
                        const int32_t *context_lens, float scale, int is_causal,
                        int num_kv_heads, int num_heads, int out_dtype, void *out,
                        void *workspace,
                        size_t workspace_bytes, nvm_stream_t stream) {
  using namespace nvm;
  if (int r = check_attention(N, L, D, max_pages, page_size, kv_dtype, num_kv_heads, num_heads))
    return r;
  ATTN_REQUIRE(out_dtype == NVM_KV_F32 || out_dtype == NVM_KV_BF16 || out_dtype == NVM_KV_F16,
               "paged_attention: out dtype must be f32, bf16 or f16");
  ATTN_REQUIRE(B >= 0 && N / num_heads == B,
               "paged_attention: q batch size must match block_table batch size");
  ATTN_REQUIRE(P >= 0 && P <= 0x7FFFFFFFll, "paged_attention: bad page count %lld", (long long)P);
  const int elt = kv_dtype == NVM_KV_F32 ? 4 : kv_dtype == NVM_KV_I8 ? 1 : 2;
  // (the kernels address pages through 32-bit buffer offsets, and a masked
  // lane reads at kMaskedOffset, which must lie beyond every page tensor)
  ATTN_SUPPORTED(P * num_kv_heads * page_size * D * elt <= 0x7FFF0000ll,
                 "paged_attention: page tensors of %lld bytes; at most 2 GiB each",
                 (long long)(P * num_kv_heads * page_size * D * elt));
  if (N == 0) return NVM_OK;
  ATTN_REQUIRE(q && out && block_table && context_lens, "paged_attention: null pointer");
  ATTN_REQUIRE(P == 0 || (key_pages && value_pages), "paged_attention: null page pointer");
  ATTN_REQUIRE(kv_dtype != NVM_KV_I8 || P == 0 || (key_scales && value_scales),
               "paged_attention_int8: key_scales and value_scales are required");

  const AttnPlan plan = attn_plan(N, L, D, max_pages, page_size, kv_dtype, num_kv_heads,
                                  num_heads);
  const size_t need = attn_workspace(plan, N, D);
  if (need && (!workspace || workspace_bytes < need))
    return set_error(NVM_ERR_WORKSPACE, "paged_attention: workspace of %zu bytes needed", need);

  PagedArgs a{};
  a.q = q;
  a.kp = key_pages;
  a.vp = value_pages;
  a.ks = key_scales;
  a.vs = value_scales;
  a.bt = block_table;
  a.lens = context_lens;
  a.out = out;
  a.out_dt = out_dtype;
  a.P = (int)P;
  a.L = (int)L;
  a.D = (int)D;
  a.page_size = (int)page_size;
  a.max_pages = (int)max_pages;
  a.Hkv = num_kv_heads;
  a.Hq = num_heads;
  a.R = num_heads / num_kv_heads;
  a.HG = plan.HG;
  a.S = plan.S;
  a.span = plan.span;
  a.causal = is_causal ? 1 : 0;
  a.scale2 = scale * kLog2e;
  hipStream_t st = (hipStream_t)stream;

  if (plan.decode) {
    if (plan.S > 1) {
      a.part_o = (float *)workspace;
      a.part_ml = (float *)((char *)workspace + (((size_t)N * plan.S * D * sizeof(float) + 255) &
                                                 ~(size_t)255));
    }
    const unsigned grid = (unsigned)(B * num_kv_heads * plan.HG * plan.S);
    if (grid == 0) return NVM_OK;
    if (kv_dtype == NVM_KV_BF16)
      launch_decode<DT_BF16>(a, plan.RP, (int)D, grid, st);
    else
      launch_decode<DT_F16>(a, plan.RP, (int)D, grid, st);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(NVM_ERR_HIP, "paged_attention: %s", hipGetErrorString(e));
    if (plan.S > 1) {
      hipLaunchKernelGGL(paged_combine_kernel, dim3((unsigned)N), dim3(256), 0, st, a.part_o,
                         a.part_ml, plan.S, (int)D, out, out_dtype);
      e = hipGetLastError();
      if (e != hipSuccess)
        return set_error(NVM_ERR_HIP, "paged_attention combine: %s", hipGetErrorString(e));
    }
    return NVM_OK;
  }

  if (paged_prefill_supports(L, D, kv_dtype, num_kv_heads, num_heads)) {
    const hipError_t e = launch_paged_prefill(q, B, L, D, key_pages, value_pages, P, page_size,
                                              kv_dtype, block_table, max_pages, context_lens,
                                              scale, is_causal, num_kv_heads, num_heads,
                                              out_dtype, out, st);
    if (e != hipSuccess) return set_error(NVM_ERR_HIP, "paged_attention: %s", hipGetErrorString(e));
    return NVM_OK;
  }
  const int64_t rows = N * L;
  const unsigned grid = (unsigned)((rows + 3) / 4);
  switch (kv_dtype) {
    case NVM_KV_F32:
      hipLaunchKernelGGL((paged_rows_kernel<NVM_KV_F32>), dim3(grid), dim3(256), 0, st, a, rows);
      break;
    case NVM_KV_I8:
      hipLaunchKernelGGL((paged_rows_kernel<NVM_KV_I8>), dim3(grid), dim3(256), 0, st, a, rows);
      break;
    case NVM_KV_BF16:
      hipLaunchKernelGGL((paged_rows_kernel<NVM_KV_BF16>), dim3(grid), dim3(256), 0, st, a, rows);
      break;
    default:
      hipLaunchKernelGGL((paged_rows_kernel<NVM_KV_F16>), dim3(grid), dim3(256), 0, st, a, rows);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(NVM_ERR_HIP, "paged_attention: %s", hipGetErrorString(e));
  return NVM_OK;
}

}  // extern "C"
