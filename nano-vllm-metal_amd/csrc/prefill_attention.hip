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
// A block owns (request b, kv head h, 16 columns per wavefront): a column is
// one (query position, query head) of the heads that share kv head h, so the
// grouped-query heads read each key and value row once, from LDS.  Columns
// are 16 / R positions x the R = Hq / Hkv heads; the block's eight
// wavefronts take consecutive positions.  Per 64-key tile:
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

#include "common.h"
#include "internal.h"
#include "nvm_attention.h"

namespace nvm {

namespace {

constexpr float kLog2eC = 1.4426950408889634f;
constexpr int kCW = 8;      // wavefronts (column tiles) per block
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

// x = p0 + p1 + p2 in the act dtype, for four pairs of values.
template <int DT>
__device__ __forceinline__ void split3c(const float (&x)[8], u32x4 &p0, u32x4 &p1, u32x4 &p2) {
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

template <int DT, int DH, int R>
__global__ __launch_bounds__(64 * kCW) void causal_prefill_kernel(CausalArgs a) {
  using A = Act<DT>;
  constexpr int NC = DH / 32;       // 32-dim steps of a score MFMA
  constexpr int NT = DH / 16;       // 16-dim tiles of the output
  constexpr int PPC = 16 / R;       // query positions per column tile
  constexpr int QB = kCW * PPC;     // query positions per block
  constexpr int KP = DH + 8;        // LDS pitch of a key row (16-bit elements)
  constexpr int VP = kKT / 2 + 4;   // LDS pitch of a transposed value row (dwords)
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
  // this lane's column: position and query head
  const int pos = q0 + wv * PPC + c16 / R;
  const int head = kvh * R + c16 % R;
  const bool col_ok = pos < a.L;
  const int64_t tok0 = (int64_t)b * a.L;  // the request's first token row

  // B operand of the score MFMAs: query (pos, head), dims 32kk + 8G .. +7
  u32x4 qop[NC];
  {
    const float *qp = a.q + ((tok0 + (col_ok ? pos : 0)) * a.Hq + head) * DH;
#pragma unroll
    for (int kk = 0; kk < NC; ++kk) {
      const int d0 = 32 * kk + 8 * G;
      const f32x4 x0 = col_ok ? *(const f32x4 *)(qp + d0) : f32x4{0.f, 0.f, 0.f, 0.f};
      const f32x4 x1 = col_ok ? *(const f32x4 *)(qp + d0 + 4) : f32x4{0.f, 0.f, 0.f, 0.f};
      qop[kk] = u32x4{A::pack2(x0[0], x0[1]), A::pack2(x0[2], x0[3]), A::pack2(x1[0], x1[1]),
                      A::pack2(x1[2], x1[3])};
    }
  }

  // keys of the block: every position below q0 + QB (and below L)
  const int kend = min(q0 + QB, a.L);
  const int ntile = (kend + kKT - 1) / kKT;

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
        s_vt[buf][8 * dg + d][kp2] = A::pack2(lo, hi);
      }
    }
  };

  float m_run = -INFINITY, l_run = 0.f;  // column c16; l_run is this lane's share
  f32x4 oacc[NT];                        // O^T: column c16, dims 16t + 4G + i
#pragma unroll
  for (int t = 0; t < NT; ++t) oacc[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  stage_load(0);
  stage_store(0);
  __syncthreads();
  for (int kt = 0; kt < ntile; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < ntile) stage_load(kt + 1);  // uniform

    // S^T: keys 16u + c16 as the A operand (dims 32kk + 8G .. +7)
    f32x4 acc[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      acc[u] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < NC; ++kk)
        acc[u] = A::mfma16(*(const u32x4 *)&s_k[buf][16 * u + c16][32 * kk + 8 * G], qop[kk],
                           acc[u]);
    }
    // causal mask (key j <= position, j < L), base-2 scores, online softmax
    float sc[4][4];
    float tmax = -INFINITY;
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int j = kt * kKT + 16 * u + 4 * G + i;
        const bool valid = col_ok && j <= pos;
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

    // O^T += V^T . P^T per 32-key chunk
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
      const float x[8] = {pv[2 * kc][0], pv[2 * kc][1], pv[2 * kc][2], pv[2 * kc][3],
                          pv[2 * kc + 1][0], pv[2 * kc + 1][1], pv[2 * kc + 1][2],
                          pv[2 * kc + 1][3]};
      u32x4 pb[3];
      split3c<DT>(x, pb[0], pb[1], pb[2]);
      // key pairs (4G, 4G+1), (4G+2, 4G+3) and the same + 16 of the chunk
      const int kp0 = 16 * kc + 2 * G, kp1 = 16 * kc + 8 + 2 * G;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const uint32_t *row = s_vt[buf][16 * t + c16];
        const u32x2 lo = *(const u32x2 *)&row[kp0];
        const u32x2 hi = *(const u32x2 *)&row[kp1];
        const u32x4 va{lo.x, lo.y, hi.x, hi.y};
#pragma unroll
        for (int part = 0; part < 3; ++part) oacc[t] = A::mfma16(va, pb[part], oacc[t]);
      }
    }
    // the next tile's rows into the other buffer (every wavefront passed the
    // previous tile's barrier: no one reads it any more)
    if (kt + 1 < ntile) stage_store(buf ^ 1);
    __syncthreads();
  }

  // the column's sum (four lane shares), then O = O^T / l
  l_run += __shfl_xor(l_run, 16);
  l_run += __shfl_xor(l_run, 32);
  if (col_ok) {
    const int64_t o0 = ((tok0 + pos) * a.Hq + head) * DH;
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        store_out_c(a.out, a.out_dt, o0 + 16 * t + 4 * G + i,
                    l_run > 0.f ? oacc[t][i] / l_run : 0.f);
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
    case 1: return go(causal_prefill_kernel<DT, DH, 1>, kCW * 16);
    case 2: return go(causal_prefill_kernel<DT, DH, 2>, kCW * 8);
    case 4: return go(causal_prefill_kernel<DT, DH, 4>, kCW * 4);
    case 8: return go(causal_prefill_kernel<DT, DH, 8>, kCW * 2);
    case 16: return go(causal_prefill_kernel<DT, DH, 16>, kCW);
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
