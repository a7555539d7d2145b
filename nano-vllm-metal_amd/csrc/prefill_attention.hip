// Causal attention of an initial prefill (declared in include/nvm_attention.h).
//
// Replaces the float32 `mx.fast.scaled_dot_product_attention(q, k, v,
// scale, mask="causal")` of the model's initial prefill
// (models/qwen3.py:134-141): every request attends over its own new tokens,
// query i seeing keys j <= i, with float32 sums.  q, k and v arrive as float32
// tensors holding activation-dtype values (the q/k norm, RoPE and store step
// rounds them like the reference), so each product of two of them is exact in
// float32.
//
// A block owns (request b, kv head h, two 16-column tiles per wavefront): a
// column is one (query position, query head) of the heads that share kv
// head h, so the grouped-query heads read each key and value row once, from
// LDS.  A column tile is 16 / R positions x the R = Hq / Hkv heads; the
// block's eight wavefronts take consecutive positions.  Every key or value
// operand a wavefront reads from LDS feeds the MFMAs of both its column
// tiles (with one tile per wavefront, the LDS reads per tile took as many
// cycles as the MFMAs).  Per 64-key tile:
//   * the tile's keys (act dtype, key-major) and values (act dtype,
//     transposed: dim-major, key pairs per dword) are staged in LDS by the
//     whole block, double-buffered, the next tile's rows loaded into
//     registers during the current tile's products;
//   * S^T = K . Q^T on the matrix cores (v_mfma_f32_16x16x32 in the act
//     dtype): lane (c, G) holds column c at keys 16u + 4G + i; scores are
//     kept in base 2 (scaled by scale * log2 e) for an online softmax whose
//     column maximum is two lane swaps;
//   * O^T += V^T . P^T per 32-key chunk, P split into three act-dtype parts
//     (exact for bf16; for f16 down to its subnormal range) so the products
//     stay exact: the S^T layout leaves each lane its own B operand (k-slot
//     8G + j is key 4G + j, j < 4, or 16 + 4G + j - 4), and the A operand is
//     two 8-byte reads of the transposed values.
// Heavy blocks (late query positions, more key tiles) are launched first.
#include <math.h>

#include <algorithm>
#include <type_traits>

#include "common.h"
#include "internal.h"
#include "nvm_attention.h"

namespace nvm {

namespace {

constexpr float kLog2eC = 1.4426950408889634f;
constexpr int kCW = 8;      // wavefronts per block
constexpr int kCT = 2;      // 16-column tiles per wavefront
constexpr int kKT = 64;     // keys per tile

struct CausalArgs {
  const float *q, *k, *v;
  void *out;
  int out_dt;
  int B, L, Hq, Hkv, n_qb;
  float scale2;  // scale * log2(e)
};

__device__ __forceinline__ void store_out_c(void *out, int dt, int64_t i, float v) {
  if (dt == NVM_KV_F32)
    ((float *)out)[i] = v;
  else if (dt == NVM_KV_BF16)
    ((uint16_t *)out)[i] = Act<DT_BF16>::from_f32(v);
  else
    ((uint16_t *)out)[i] = Act<DT_F16>::from_f32(v);
}

// x = p0 + p1 + p2 in the act dtype, for four pairs of values (x >= 0 and
// normal or zero, as the probabilities are).  bf16: each part is the upper
// half of what is left (truncation: x - trunc(x) is exact and has at most 16
// significant bits, its remainder at most 8, a bf16 value), the pairs packed
// with one v_perm_b32 a part.  f16: each part rounded to nearest, the packed
// word pinned so that the compiler takes its halves back instead of
// converting again.
template <int DT>
__device__ __forceinline__ void split3c(const float (&x)[8], u32x4 &p0, u32x4 &p1, u32x4 &p2) {
  using A = Act<DT>;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float a0 = x[2 * i], a1 = x[2 * i + 1];
    if constexpr (DT == DT_BF16) {
      const uint32_t h0 = __float_as_uint(a0), h1 = __float_as_uint(a1);
      a0 -= __uint_as_float(h0 & 0xFFFF0000u);
      a1 -= __uint_as_float(h1 & 0xFFFF0000u);
      const uint32_t m0 = __float_as_uint(a0), m1 = __float_as_uint(a1);
      a0 -= __uint_as_float(m0 & 0xFFFF0000u);
      a1 -= __uint_as_float(m1 & 0xFFFF0000u);
      // upper halves of (lo, hi) into one word, lo first
      p0[i] = perm_b32(h1, h0, 0x07060302u);
      p1[i] = perm_b32(m1, m0, 0x07060302u);
      p2[i] = perm_b32(__float_as_uint(a1), __float_as_uint(a0), 0x07060302u);
    } else {
      uint32_t h = A::pack2(a0, a1);
      asm volatile("" : "+v"(h));
      a0 -= A::lo(h);
      a1 -= A::hi(h);
      uint32_t m = A::pack2(a0, a1);
      asm volatile("" : "+v"(m));
      a0 -= A::lo(m);
      a1 -= A::hi(m);
      p0[i] = h;
      p1[i] = m;
      p2[i] = A::pack2(a0, a1);
    }
  }
}

// Column of key pair kp in row r of the transposed values in LDS.  A lane's
// P.V operand is key pairs kp0 = 16 kc + 2 G, kp0 + 1, kp0 + 8, kp0 + 9:
// they sit in columns 16 kc + 4 G .. + 3, one 16-byte read (the two 8-byte
// reads it replaces collided on banks).  Rows in groups of 16 XOR the column
// with vt_swz of the group (bits 1, 3 and 4), which spreads the staging
// stores (16 lanes on 16 rows 8 apart, one key pair) over 8 columns instead
// of 1; bit 1 swaps the two pairs inside a read, which the read undoes.
__device__ __forceinline__ constexpr int vt_swz(int g) { return ((g & 1) << 1) | ((g & 6) << 2); }
__device__ __forceinline__ int vt_col(int r, int kp) {
  const int pc = (kp & 16) | (((kp >> 1) & 3) << 2) | (((kp >> 3) & 1) << 1) | (kp & 1);
  return pc ^ vt_swz((r >> 4) & 7);
}

template <int DT, int DH, int R, int CT>
__global__ __launch_bounds__(64 * kCW) void causal_prefill_kernel(CausalArgs a) {
  using A = Act<DT>;
  constexpr int NC = DH / 32;       // 32-dim steps of a score MFMA
  constexpr int NT = DH / 16;       // 16-dim tiles of the output
  constexpr int PPC = 16 / R;       // query positions per column tile
  constexpr int PPW = CT * PPC;     // query positions per wavefront
  constexpr int QB = kCW * PPW;     // query positions per block
  // LDS pitches (the LDS serves a 16-byte access 32 lanes at a time over
  // 128 banks): key rows of DH + 16 elements (72 or 40 dwords) and value
  // rows of 40 dwords put the 32 lanes of a score or P.V read on distinct
  // banks (pitches of 68 or 36 dwords collide on one bank pair)
  constexpr int KP = DH + 16;       // LDS pitch of a key row (16-bit elements)
  constexpr int VP = kKT / 2 + 8;   // LDS pitch of a transposed value row (dwords)
  constexpr int DG = DH / 8;        // 8-dim groups of a row
  // staging items of a tile: keys (key, 8 dims), values (key pair, 8 dims),
  // and per thread
  constexpr int KN = kKT * DG, VN = (kKT / 2) * DG;
  constexpr int KI = (KN + 64 * kCW - 1) / (64 * kCW), VI = (VN + 64 * kCW - 1) / (64 * kCW);
  __shared__ __attribute__((aligned(16))) uint16_t s_k[2][kKT][KP];
  __shared__ __attribute__((aligned(16))) uint32_t s_vt[2][DH][VP];

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int c16 = lane & 15, G = lane >> 4;
  // heavy query blocks first
  const int bh = blockIdx.x % (a.B * a.Hkv);
  const int qb = a.n_qb - 1 - blockIdx.x / (a.B * a.Hkv);
  const int b = bh / a.Hkv, kvh = bh - b * a.Hkv;
  const int q0 = qb * QB;
  const int wp0 = q0 + wv * PPW;  // the wavefront's first query position
  // this lane's columns: positions (one per column tile) and query head
  int pos[CT];
  bool col_ok[CT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    pos[ct] = wp0 + ct * PPC + c16 / R;
    col_ok[ct] = pos[ct] < a.L;
  }
  const int head = kvh * R + c16 % R;
  const int64_t tok0 = (int64_t)b * a.L;  // the request's first token row

  // B operands of the score MFMAs: query (pos, head), dims 32kk + 8G .. +7
  u32x4 qop[CT][NC];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    const float *qp = a.q + ((tok0 + (col_ok[ct] ? pos[ct] : 0)) * a.Hq + head) * DH;
#pragma unroll
    for (int kk = 0; kk < NC; ++kk) {
      const int d0 = 32 * kk + 8 * G;
      const f32x4 x0 = col_ok[ct] ? *(const f32x4 *)(qp + d0) : f32x4{0.f, 0.f, 0.f, 0.f};
      const f32x4 x1 = col_ok[ct] ? *(const f32x4 *)(qp + d0 + 4) : f32x4{0.f, 0.f, 0.f, 0.f};
      qop[ct][kk] = u32x4{A::pack2(x0[0], x0[1]), A::pack2(x0[2], x0[3]),
                          A::pack2(x1[0], x1[1]), A::pack2(x1[2], x1[3])};
    }
  }

  // keys of the block: every position below q0 + QB (and below L)
  const int kend = min(q0 + QB, a.L);
  const int ntile = (kend + kKT - 1) / kKT;
  // the wavefront's columns all exist and see every key below wp0 + 1
  const bool all_cols = wp0 + PPW <= a.L;

  // staging loads of tile kt into registers (rows past kend read as zeros)
  f32x4 kreg[KI][2], vreg[VI][4];
  auto stage_load = [&](int kt) {
#pragma unroll
    for (int i = 0; i < KI; ++i) {
      const int item = tid + 64 * kCW * i;
      const int key = item / DG, dg = item - key * DG;
      const int j = kt * kKT + key;
      const bool ok = item < KN && j < kend;
      const float *kp = a.k + ((tok0 + (ok ? j : 0)) * a.Hkv + kvh) * DH + 8 * dg;
      kreg[i][0] = ok ? *(const f32x4 *)kp : f32x4{0.f, 0.f, 0.f, 0.f};
      kreg[i][1] = ok ? *(const f32x4 *)(kp + 4) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int i = 0; i < VI; ++i) {
      const int item = tid + 64 * kCW * i;
      const int kp2 = item / DG, dg = item - kp2 * DG;
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int j = kt * kKT + 2 * kp2 + r;
        const bool ok = item < VN && j < kend;
        const float *vp = a.v + ((tok0 + (ok ? j : 0)) * a.Hkv + kvh) * DH + 8 * dg;
        vreg[i][2 * r] = ok ? *(const f32x4 *)vp : f32x4{0.f, 0.f, 0.f, 0.f};
        vreg[i][2 * r + 1] = ok ? *(const f32x4 *)(vp + 4) : f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
  };
  auto stage_store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < KI; ++i) {
      const int item = tid + 64 * kCW * i;
      if (item >= KN) continue;
      const int key = item / DG, dg = item - key * DG;
      const f32x4 x0 = kreg[i][0], x1 = kreg[i][1];
      *(u32x4 *)&s_k[buf][key][8 * dg] =
          u32x4{A::pack2(x0[0], x0[1]), A::pack2(x0[2], x0[3]), A::pack2(x1[0], x1[1]),
                A::pack2(x1[2], x1[3])};
    }
#pragma unroll
    for (int i = 0; i < VI; ++i) {
      const int item = tid + 64 * kCW * i;
      if (item >= VN) continue;
      const int kp2 = item / DG, dg = item - kp2 * DG;
#pragma unroll
      for (int d = 0; d < 8; ++d) {
        const float lo = vreg[i][d >> 2][d & 3], hi = vreg[i][2 + (d >> 2)][d & 3];
        s_vt[buf][8 * dg + d][vt_col(8 * dg + d, kp2)] = A::pack2(lo, hi);
      }
    }
  };

  // per column tile: running maximum (base 2, scaled) and this lane's share
  // of the column's sum; O^T: column c16, dims 16t + 4G + i
  float m_run[CT], l_run[CT];
  f32x4 oacc[CT][NT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    m_run[ct] = -INFINITY;
    l_run[ct] = 0.f;
#pragma unroll
    for (int t = 0; t < NT; ++t) oacc[ct][t] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  stage_load(0);
  stage_store(0);
  __syncthreads();
  for (int kt = 0; kt < ntile; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < ntile) stage_load(kt + 1);  // uniform

    // S^T: keys 16u + c16 as the A operand (dims 32kk + 8G .. +7), each key
    // operand read once for the column tiles
    f32x4 acc[CT][4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) acc[ct][u] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < NC; ++kk) {
        const u32x4 kop = *(const u32x4 *)&s_k[buf][16 * u + c16][32 * kk + 8 * G];
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) acc[ct][u] = A::mfma16(kop, qop[ct][kk], acc[ct][u]);
      }
    }
    // Causal mask (key j <= position, j < L), base-2 scores, online softmax.
    // Interior tiles (every key of the tile visible to every column of the
    // wavefront, all columns real: uniform) take a path without the mask and
    // without the guard for a column that has seen no key yet.  scale2 > 0:
    // the maximum of the raw scores scaled is the maximum of the scaled
    // scores, and exp2(s * scale2 - m) is one fma into v_exp_f32, whose
    // results below 2^-126 (terms that far below the column maximum) flush to
    // zero, which the float32 sum cannot tell.
    float pv[CT][4][4];
    bool rescale = false;
    float alpha[CT];
    auto softmax = [&](auto interior) {
      constexpr bool kIn = decltype(interior)::value;
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        float tmax = -INFINITY;
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int j = kt * kKT + 16 * u + 4 * G + i;
            pv[ct][u][i] = kIn || (col_ok[ct] && j <= pos[ct]) ? acc[ct][u][i] : -INFINITY;
            tmax = fmaxf(tmax, pv[ct][u][i]);
          }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
        const float m_new = fmaxf(m_run[ct], tmax * a.scale2);
        const bool any = kIn || m_new != -INFINITY;
        alpha[ct] = any ? __builtin_amdgcn_exp2f(m_run[ct] - m_new) : 1.f;
        rescale |= alpha[ct] != 1.f;
        float psum = 0.f;
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            pv[ct][u][i] =
                any ? __builtin_amdgcn_exp2f(__builtin_fmaf(pv[ct][u][i], a.scale2, -m_new)) : 0.f;
            psum += pv[ct][u][i];
          }
        l_run[ct] = l_run[ct] * alpha[ct] + psum;
        m_run[ct] = m_new;
      }
    };
    if (all_cols && kt * kKT + kKT - 1 <= wp0)
      softmax(std::true_type{});
    else
      softmax(std::false_type{});
    // O^T *= alpha, skipped when no column's maximum moved (the factors are
    // then all 1)
    if (__builtin_amdgcn_ballot_w64(rescale)) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int t = 0; t < NT; ++t) oacc[ct][t] *= alpha[ct];
    }

    // O^T += V^T . P^T per 32-key chunk, each value operand read once for the
    // column tiles
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
      u32x4 pb[CT][3];
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        const float x[8] = {pv[ct][2 * kc][0],     pv[ct][2 * kc][1],     pv[ct][2 * kc][2],
                            pv[ct][2 * kc][3],     pv[ct][2 * kc + 1][0], pv[ct][2 * kc + 1][1],
                            pv[ct][2 * kc + 1][2], pv[ct][2 * kc + 1][3]};
        split3c<DT>(x, pb[ct][0], pb[ct][1], pb[ct][2]);
      }
      // key pairs 2G, 2G + 1 and 2G + 8, 2G + 9 of the chunk (keys 4G .. 4G + 3 and
      // the same + 16): the 16 bytes at vt_col
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const uint32_t *row = s_vt[buf][16 * t + c16];
        const int sw = vt_swz(t & 7);
        u32x4 va = *(const u32x4 *)&row[(16 * kc + 4 * G) ^ (sw & ~3)];
        if (sw & 2) va = u32x4{va[2], va[3], va[0], va[1]};  // (t unrolled: no branch)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
          for (int part = 0; part < 3; ++part)
            oacc[ct][t] = A::mfma16(va, pb[ct][part], oacc[ct][t]);
      }
    }
    // the next tile's rows into the other buffer (every wavefront passed the
    // previous tile's barrier: no one reads it any more)
    if (kt + 1 < ntile) stage_store(buf ^ 1);
    __syncthreads();
  }

  // each column's sum (four lane shares), then O = O^T / l
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    float l = l_run[ct];
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    if (col_ok[ct]) {
      const int64_t o0 = ((tok0 + pos[ct]) * a.Hq + head) * DH;
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          store_out_c(a.out, a.out_dt, o0 + 16 * t + 4 * G + i,
                      l > 0.f ? oacc[ct][t][i] / l : 0.f);
    }
  }
}

template <int DT, int DH>
hipError_t launch_causal_r(const CausalArgs &a0, int R, hipStream_t st) {
  CausalArgs a = a0;
  auto go = [&](auto kern, int QB) {
    a.n_qb = (a.L + QB - 1) / QB;
    hipLaunchKernelGGL(kern, dim3((unsigned)((int64_t)a.n_qb * a.B * a.Hkv)), dim3(64 * kCW), 0, st,
                       a);
    return hipGetLastError();
  };
  switch (R) {
    case 1: return go(causal_prefill_kernel<DT, DH, 1, kCT>, kCW * kCT * 16);
    case 2: return go(causal_prefill_kernel<DT, DH, 2, kCT>, kCW * kCT * 8);
    case 4: return go(causal_prefill_kernel<DT, DH, 4, kCT>, kCW * kCT * 4);
    case 8: return go(causal_prefill_kernel<DT, DH, 8, kCT>, kCW * kCT * 2);
    case 16: return go(causal_prefill_kernel<DT, DH, 16, kCT>, kCW * kCT);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

}  // namespace nvm

extern "C" int nvm_causal_attention(const float *q, const float *k, const float *v, int64_t B,
                                    int64_t L, int num_heads, int num_kv_heads, int64_t D,
                                    float scale, int dtype, int out_dtype, void *out,
                                    nvm_stream_t stream) {
  using namespace nvm;
  if (dtype != NVM_DTYPE_BF16 && dtype != NVM_DTYPE_F16)
    return set_error(NVM_ERR_INVALID, "causal_attention: dtype must be f16 or bf16");
  if (out_dtype != NVM_KV_F32 && out_dtype != NVM_KV_BF16 && out_dtype != NVM_KV_F16)
    return set_error(NVM_ERR_INVALID, "causal_attention: bad out dtype %d", out_dtype);
  if (B < 0 || L < 0 || num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads)
    return set_error(NVM_ERR_INVALID, "causal_attention: bad shape");
  const int R = num_heads / num_kv_heads;
  if ((D != 64 && D != 128) || R > 16 || (16 % R) != 0)
    return set_error(NVM_ERR_UNSUPPORTED,
                     "causal_attention: head dim 64 or 128 and 1, 2, 4, 8 or 16 query heads "
                     "per kv head (got D=%lld, %d)", (long long)D, R);
  if (!(scale > 0.f) || !(scale <= 1.0e15f))
    return set_error(NVM_ERR_UNSUPPORTED,
                     "causal_attention: scale must be positive and finite (got %g)", (double)scale);
  if (B * L == 0) return NVM_OK;
  if (!q || !k || !v || !out) return set_error(NVM_ERR_INVALID, "causal_attention: null pointer");
  if (B * L * num_heads * D >= (1ll << 31) || B * num_kv_heads > (1 << 20))
    return set_error(NVM_ERR_UNSUPPORTED, "causal_attention: tensors beyond 2^31 elements");
  CausalArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.out = out;
  a.out_dt = out_dtype;
  a.B = (int)B;
  a.L = (int)L;
  a.Hq = num_heads;
  a.Hkv = num_kv_heads;
  a.scale2 = scale * kLog2eC;
  hipStream_t st = (hipStream_t)stream;
  hipError_t e;
  if (dtype == NVM_DTYPE_BF16)
    e = D == 128 ? launch_causal_r<DT_BF16, 128>(a, R, st) : launch_causal_r<DT_BF16, 64>(a, R, st);
  else
    e = D == 128 ? launch_causal_r<DT_F16, 128>(a, R, st) : launch_causal_r<DT_F16, 64>(a, R, st);
  if (e != hipSuccess) return set_error(NVM_ERR_HIP, "causal_attention: %s", hipGetErrorString(e));
  return NVM_OK;
}
