// Multi-query paged attention on the matrix cores: L > 1 new query rows of a
// request over its paged keys and values (declared as a launch in
// internal.h; nvm_paged_attention takes it for f16/bf16 pages, head dims 64
// and 128 and 1, 2, 4, 8 or 16 query heads per kv head).
//
// This is the reference's paged prefill (metal/src/paged_attention.metal:7-134,
// `paged_attention_kv`, dispatched at metal/src/paged_attention.cpp:446-516)
// for chunked prefill and prefill after a prefix: query row i (of L) sees
// context positions j <= i + context_len - L (causal) or all j <
// context_len, softmax(q . k^T * scale) . v with float32 sums.  Positions
// whose page id is negative or beyond the pool are skipped, as in the
// reference's CPU loop.
//
// The structure is the causal prefill kernel's (prefill_attention.hip): a
// block owns (request, kv head, 8 wavefronts x 16 columns), a column being
// one (query row, query head) of the heads that share the kv head, so every
// key and value row is read once per block, from LDS; per 64-key tile the
// keys (act dtype, key-major) and values (transposed, key pairs per dword)
// are staged in LDS, double-buffered, the next tile loaded into registers
// during the current one's products; S^T = K . Q^T and O^T += V^T . P^T run
// on v_mfma_f32_16x16x32 in the page dtype.  What differs:
//   * keys and values come from the pages (16-byte loads of page-dtype rows,
//     no conversion), each tile's positions looked up in the block table;
//   * the query is float32 (the reference op's operand): it is split into
//     three page-dtype parts, so every product stays exact (as in the decode
//     kernel), and the three score MFMAs add them in float32;
//   * a position's validity (in the context, on a valid page) is staged with
//     its key, and the causal bound is i + context_len - L.
#include <math.h>

#include "common.h"
#include "internal.h"
#include "nvm_attention.h"

namespace nvm {

namespace {

constexpr float kLog2eP = 1.4426950408889634f;
constexpr int kPW = 8;   // wavefronts (column tiles) per block
constexpr int kPKT = 64;  // keys per tile

struct PrefillArgs {
  const float *q;
  const uint16_t *kp, *vp;
  const int32_t *bt, *lens;
  void *out;
  int out_dt;
  int B, L, P, page_size, max_pages, Hkv, Hq, causal, n_qb;
  float scale2;
};

__device__ __forceinline__ void store_out_p(void *out, int dt, int64_t i, float v) {
  if (dt == NVM_KV_F32)
    ((float *)out)[i] = v;
  else if (dt == NVM_KV_BF16)
    ((uint16_t *)out)[i] = Act<DT_BF16>::from_f32(v);
  else
    ((uint16_t *)out)[i] = Act<DT_F16>::from_f32(v);
}

// x = p0 + p1 + p2 in the act dtype, for four pairs of values (exact for
// float32 x within the act dtype's range: each part takes the next 8 or 11
// significand bits of the remainder).
template <int DT>
__device__ __forceinline__ void split3p(const float (&x)[8], u32x4 &p0, u32x4 &p1, u32x4 &p2) {
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

template <int DT, int DH, int R>
__global__ __launch_bounds__(64 * kPW) void paged_prefill_kernel(PrefillArgs a) {
  using A = Act<DT>;
  constexpr int NC = DH / 32;      // 32-dim steps of a score MFMA
  constexpr int NT = DH / 16;      // 16-dim tiles of the output
  constexpr int PPC = 16 / R;      // query rows per column tile
  constexpr int QB = kPW * PPC;    // query rows per block
  // LDS pitches (the LDS serves a 16-byte access 32 lanes at a time over
  // 128 banks): key rows of DH + 16 elements (72 or 40 dwords) and value
  // rows of 40 dwords put the 32 lanes of a score or P.V read on distinct
  // banks (pitches of 68 or 36 dwords collide on one bank pair)
  constexpr int KP = DH + 16;      // LDS pitch of a key row (16-bit elements)
  constexpr int VP = kPKT / 2 + 8;  // LDS pitch of a transposed value row (dwords)
  constexpr int DG = DH / 8;       // 8-dim groups of a row
  constexpr int KN = kPKT * DG, VN = (kPKT / 2) * DG;
  constexpr int KI = (KN + 64 * kPW - 1) / (64 * kPW), VI = (VN + 64 * kPW - 1) / (64 * kPW);
  __shared__ __attribute__((aligned(16))) uint16_t s_k[2][kPKT][KP];
  __shared__ __attribute__((aligned(16))) uint32_t s_vt[2][DH][VP];
  __shared__ uint8_t s_ok[2][kPKT];

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int c16 = lane & 15, G = lane >> 4;
  // blocks of later query rows (more keys) first
  const int bh = blockIdx.x % (a.B * a.Hkv);
  const int qb = a.n_qb - 1 - blockIdx.x / (a.B * a.Hkv);
  const int b = bh / a.Hkv, kvh = bh - b * a.Hkv;
  const int q0 = qb * QB;
  const int pos = q0 + wv * PPC + c16 / R;  // this lane's column: query row
  const int head = kvh * R + c16 % R;       // and query head
  const bool col_ok = pos < a.L;
  const int len = a.lens[b];
  const int off = len - a.L;                // causal: row i sees j <= i + off
  const int ctx = min(len, a.max_pages * a.page_size);
  // positions any column of the block may see
  int kend = ctx;
  if (a.causal) kend = min(kend, min(q0 + QB, a.L) + off);
  const int ntile = kend > 0 ? (kend + kPKT - 1) / kPKT : 0;
  const int32_t *bt = a.bt + (int64_t)b * a.max_pages;

  // B operand of the score MFMAs: query (row, head), dims 32kk + 8G .. +7,
  // as three page-dtype parts
  u32x4 qop[3][NC];
  {
    const int64_t n = (int64_t)b * a.Hq + head;
    const float *qp = a.q + (n * a.L + (col_ok ? pos : 0)) * DH;
#pragma unroll
    for (int kk = 0; kk < NC; ++kk) {
      const int d0 = 32 * kk + 8 * G;
      const f32x4 x0 = col_ok ? *(const f32x4 *)(qp + d0) : f32x4{0.f, 0.f, 0.f, 0.f};
      const f32x4 x1 = col_ok ? *(const f32x4 *)(qp + d0 + 4) : f32x4{0.f, 0.f, 0.f, 0.f};
      const float x[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
      split3p<DT>(x, qop[0][kk], qop[1][kk], qop[2][kk]);
    }
  }

  // page row of position j (or -1: outside the context or on no valid page)
  auto row_of = [&](int j) -> int64_t {
    if (j >= kend) return -1;
    const int page = bt[j / a.page_size];
    if (page < 0 || page >= a.P) return -1;
    return ((int64_t)page * a.Hkv + kvh) * a.page_size + j % a.page_size;
  };
  // staging loads of tile kt into registers (invalid positions read zeros)
  u32x4 kreg[KI], vreg[VI][2];
  bool kok[KI];
  auto stage_load = [&](int kt) {
#pragma unroll
    for (int i = 0; i < KI; ++i) {
      const int item = tid + 64 * kPW * i;
      const int key = item / DG, dg = item - key * DG;
      const int64_t r = item < KN ? row_of(kt * kPKT + key) : -1;
      kok[i] = r >= 0;
      kreg[i] = r >= 0 ? ldg16(a.kp + r * DH + 8 * dg) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int i = 0; i < VI; ++i) {
      const int item = tid + 64 * kPW * i;
      const int kp2 = item / DG, dg = item - kp2 * DG;
#pragma unroll
      for (int rr = 0; rr < 2; ++rr) {
        const int64_t r = item < VN ? row_of(kt * kPKT + 2 * kp2 + rr) : -1;
        vreg[i][rr] = r >= 0 ? ldg16(a.vp + r * DH + 8 * dg) : u32x4{0u, 0u, 0u, 0u};
      }
    }
  };
  auto stage_store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < KI; ++i) {
      const int item = tid + 64 * kPW * i;
      if (item >= KN) continue;
      const int key = item / DG, dg = item - key * DG;
      *(u32x4 *)&s_k[buf][key][8 * dg] = kreg[i];
      if (dg == 0) s_ok[buf][key] = kok[i] ? 1 : 0;
    }
#pragma unroll
    for (int i = 0; i < VI; ++i) {
      const int item = tid + 64 * kPW * i;
      if (item >= VN) continue;
      const int kp2 = item / DG, dg = item - kp2 * DG;
#pragma unroll
      for (int d = 0; d < 8; ++d) {
        const uint32_t lo = (vreg[i][0][d >> 1] >> (16 * (d & 1))) & 0xFFFFu;
        const uint32_t hi = (vreg[i][1][d >> 1] >> (16 * (d & 1))) & 0xFFFFu;
        s_vt[buf][8 * dg + d][vt_col(8 * dg + d, kp2)] = lo | (hi << 16);
      }
    }
  };

  float m_run = -INFINITY, l_run = 0.f;  // column c16; l_run is this lane's share
  f32x4 oacc[NT];                        // O^T: column c16, dims 16t + 4G + i
#pragma unroll
  for (int t = 0; t < NT; ++t) oacc[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (ntile > 0) {
    stage_load(0);
    stage_store(0);
  }
  __syncthreads();
  for (int kt = 0; kt < ntile; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < ntile) stage_load(kt + 1);  // uniform

    // S^T: keys 16u + c16 as the A operand (dims 32kk + 8G .. +7), the
    // query's three parts summed in float32
    f32x4 acc[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      acc[u] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < NC; ++kk) {
        const u32x4 kop = *(const u32x4 *)&s_k[buf][16 * u + c16][32 * kk + 8 * G];
#pragma unroll
        for (int part = 0; part < 3; ++part) acc[u] = A::mfma16(kop, qop[part][kk], acc[u]);
      }
    }
    float sc[4][4];
    float tmax = -INFINITY;
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int kl = 16 * u + 4 * G + i;
        const int j = kt * kPKT + kl;
        const bool valid = col_ok && s_ok[buf][kl] && (!a.causal || j <= pos + off);
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

    // O^T += V^T . P^T per 32-key chunk, P in three act-dtype parts
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
      const float x[8] = {pv[2 * kc][0], pv[2 * kc][1], pv[2 * kc][2], pv[2 * kc][3],
                          pv[2 * kc + 1][0], pv[2 * kc + 1][1], pv[2 * kc + 1][2],
                          pv[2 * kc + 1][3]};
      u32x4 pb[3];
      split3p<DT>(x, pb[0], pb[1], pb[2]);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const uint32_t *row = s_vt[buf][16 * t + c16];
        const int sw = vt_swz(t & 7);
        u32x4 va = *(const u32x4 *)&row[(16 * kc + 4 * G) ^ (sw & ~3)];
        if (sw & 2) va = u32x4{va[2], va[3], va[0], va[1]};  // (t unrolled: no branch)
#pragma unroll
        for (int part = 0; part < 3; ++part) oacc[t] = A::mfma16(va, pb[part], oacc[t]);
      }
    }
    if (kt + 1 < ntile) stage_store(buf ^ 1);
    __syncthreads();
  }

  l_run += __shfl_xor(l_run, 16);
  l_run += __shfl_xor(l_run, 32);
  if (col_ok) {
    const int64_t n = (int64_t)b * a.Hq + head;
    const int64_t o0 = (n * a.L + pos) * DH;
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        store_out_p(a.out, a.out_dt, o0 + 16 * t + 4 * G + i,
                    l_run > 0.f ? oacc[t][i] / l_run : 0.f);
  }
}

template <int DT, int DH>
hipError_t launch_r(PrefillArgs a, int R, hipStream_t st) {
  auto go = [&](auto kern, int QB) {
    a.n_qb = (a.L + QB - 1) / QB;
    const int64_t grid = (int64_t)a.n_qb * a.B * a.Hkv;
    if (grid == 0) return hipSuccess;
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(64 * kPW), 0, st, a);
    return hipGetLastError();
  };
  switch (R) {
    case 1: return go(paged_prefill_kernel<DT, DH, 1>, kPW * 16);
    case 2: return go(paged_prefill_kernel<DT, DH, 2>, kPW * 8);
    case 4: return go(paged_prefill_kernel<DT, DH, 4>, kPW * 4);
    case 8: return go(paged_prefill_kernel<DT, DH, 8>, kPW * 2);
    case 16: return go(paged_prefill_kernel<DT, DH, 16>, kPW);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

bool paged_prefill_supports(int64_t L, int64_t D, int kv_dtype, int Hkv, int Hq) {
  const int R = Hq / Hkv;
  return L > 1 && (kv_dtype == NVM_KV_F16 || kv_dtype == NVM_KV_BF16) && (D == 64 || D == 128) &&
         R >= 1 && R <= 16 && 16 % R == 0;
}

hipError_t launch_paged_prefill(const float *q, int64_t B, int64_t L, int64_t D, const void *kp,
                                const void *vp, int64_t P, int64_t page_size, int kv_dtype,
                                const int32_t *bt, int64_t max_pages, const int32_t *lens,
                                float scale, int causal, int Hkv, int Hq, int out_dtype,
                                void *out, hipStream_t st) {
  if (!paged_prefill_supports(L, D, kv_dtype, Hkv, Hq)) return hipErrorInvalidValue;
  PrefillArgs a{};
  a.q = q;
  a.kp = (const uint16_t *)kp;
  a.vp = (const uint16_t *)vp;
  a.bt = bt;
  a.lens = lens;
  a.out = out;
  a.out_dt = out_dtype;
  a.B = (int)B;
  a.L = (int)L;
  a.P = (int)P;
  a.page_size = (int)page_size;
  a.max_pages = (int)max_pages;
  a.Hkv = Hkv;
  a.Hq = Hq;
  a.causal = causal ? 1 : 0;
  a.scale2 = scale * kLog2eP;
  const int R = Hq / Hkv;
  if (kv_dtype == NVM_KV_BF16)
    return D == 128 ? launch_r<DT_BF16, 128>(a, R, st) : launch_r<DT_BF16, 64>(a, R, st);
  return D == 128 ? launch_r<DT_F16, 128>(a, R, st) : launch_r<DT_F16, 64>(a, R, st);
}

}  // namespace nvm
