// Fused element-wise steps of the Qwen3 layer (declared in include/nvm_model.h).
//
// residual_rms_norm_kernel: one 256-thread block per row; each thread keeps
//   its pairs of the row in registers between the sum of squares and the
//   scaling, so the row is read once and written once or twice.
// qk_norm_rope_store_kernel: one wavefront per (token, head) of the fused
//   q/k/v projection output; lane l holds elements 2l and 2l+1 of the head.
//   q and k heads: RMSNorm over the head (wavefront sum), RoPE with the
//   partner half one lane swap away (elements i and i + D/2 sit D/4 lanes
//   apart), rounded like the reference at each step.  k and v heads go to
//   their page slot; q to the float32 attention input.
#include <math.h>

#include "common.h"
#include "internal.h"
#include "nvm_model.h"

namespace nvm {

namespace {

constexpr int kNormThreads = 256;
constexpr int kMaxNormPairs = 16;  // H <= 2 * 256 * 16 = 8192

template <int DT>
__device__ __forceinline__ uint32_t round_pair(float a, float b) {
  return Act<DT>::pack2(a, b);
}

template <int DT>
__global__ __launch_bounds__(kNormThreads) void residual_rms_norm_kernel(
    const uint32_t *__restrict__ h, const uint32_t *__restrict__ r,
    const uint32_t *__restrict__ w, int H2, float eps, uint32_t *__restrict__ h_out,
    uint32_t *__restrict__ x_out) {
  using A = Act<DT>;
  __shared__ float s_part[kNormThreads / 64];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const uint32_t *hr = h + row * H2;
  float v[kMaxNormPairs][2];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < kMaxNormPairs; ++k) {
    const int i = tid + k * kNormThreads;
    if (i < H2) {
      float a = A::lo(hr[i]), b = A::hi(hr[i]);
      if (r) {
        const uint32_t rv = r[row * H2 + i];
        const uint32_t sum = round_pair<DT>(a + A::lo(rv), b + A::hi(rv));
        h_out[row * H2 + i] = sum;
        a = A::lo(sum);
        b = A::hi(sum);
      }
      v[k][0] = a;
      v[k][1] = b;
      ss = fmaf(a, a, fmaf(b, b, ss));
    }
  }
#pragma unroll
  for (int x = 32; x > 0; x >>= 1) ss += __shfl_xor(ss, x);
  if ((tid & 63) == 0) s_part[tid >> 6] = ss;
  __syncthreads();
  const float tot = (s_part[0] + s_part[1]) + (s_part[2] + s_part[3]);
  const float inv = rsqrtf(tot / (float)(2 * H2) + eps);
#pragma unroll
  for (int k = 0; k < kMaxNormPairs; ++k) {
    const int i = tid + k * kNormThreads;
    if (i < H2) {
      const uint32_t wv = w[i];
      x_out[row * H2 + i] =
          round_pair<DT>(v[k][0] * inv * A::lo(wv), v[k][1] * inv * A::hi(wv));
    }
  }
}

// MoE combine + residual add + RMSNorm, one block per token: the token's k
// expert outputs summed in slot order exactly as the combine kernel does
// (y = rnd(sum_j rnd(down_j * score_j))), then h_out = rnd(h + y) and
// x_out = rnd(rms_norm(h_out) * w).  Eight pairs' loads are in flight at once
// (KK: the top-k as a compile-time count, every pair's loads at once, the
// float32 halves included; the arithmetic and its order are the same).
constexpr int kCombChunks = 4;  // 8-value chunks per thread: H <= 256 * 4 * 8

// SPLIT: the down outputs come as the float32 sums of the two halves of the
// down reduction (down_vals).
template <int DT, bool SPLIT, int KK>
__global__ __launch_bounds__(kNormThreads) void moe_combine_residual_norm_kernel(
    const void *__restrict__ down, const uint16_t *__restrict__ scores, int k_arg, int H8,
    const uint16_t *__restrict__ h, const uint16_t *__restrict__ w, float eps,
    uint16_t *__restrict__ h_out, uint16_t *__restrict__ x_out) {
  using A = Act<DT>;
  __shared__ float s_part[kNormThreads / 64];
  const int k = KK ? KK : k_arg;
  const int64_t t = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t H = (int64_t)H8 * 8;
  float hv[kCombChunks][8];
  float ss = 0.f;
#pragma unroll
  for (int q = 0; q < kCombChunks; ++q) {
    const int c = tid + kNormThreads * q;
    if (c >= H8) continue;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    // pairs whose loads are in flight together (KK: all of them)
    constexpr int NB = KK ? KK : SPLIT ? 4 : 8;
    for (int j0 = 0; j0 < k; j0 += NB) {
      float dv[NB][8];
      uint32_t sv[NB];
#pragma unroll
      for (int jj = 0; jj < NB; ++jj) sv[jj] = j0 + jj < k ? scores[t * k + j0 + jj] : 0u;
      down_vals<DT, SPLIT, NB>(down, (int64_t)gridDim.x * k, t, k, j0, H, c, dv);
#pragma unroll
      for (int jj = 0; jj < NB; ++jj) {
        if (j0 + jj >= k) break;
        const float sc = A::to_f32(sv[jj]);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] += round_act<DT>(dv[jj][i] * sc);
      }
    }
    const u32x4 hh = ldg16(h + t * H + 8 * c);
    u32x4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t y = A::pack2(acc[2 * i], acc[2 * i + 1]);
      o[i] = A::pack2(A::lo(hh[i]) + A::lo(y), A::hi(hh[i]) + A::hi(y));
      hv[q][2 * i] = A::lo(o[i]);
      hv[q][2 * i + 1] = A::hi(o[i]);
      ss = fmaf(hv[q][2 * i], hv[q][2 * i], fmaf(hv[q][2 * i + 1], hv[q][2 * i + 1], ss));
    }
    *(u32x4 *)(h_out + t * H + 8 * c) = o;
  }
#pragma unroll
  for (int x = 32; x > 0; x >>= 1) ss += __shfl_xor(ss, x);
  if ((tid & 63) == 0) s_part[tid >> 6] = ss;
  __syncthreads();
  const float tot = (s_part[0] + s_part[1]) + (s_part[2] + s_part[3]);
  const float inv = rsqrtf(tot / (float)H + eps);
#pragma unroll
  for (int q = 0; q < kCombChunks; ++q) {
    const int c = tid + kNormThreads * q;
    if (c >= H8) continue;
    const u32x4 wv = ldg16(w + 8 * c);
    u32x4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      o[i] = A::pack2(hv[q][2 * i] * inv * A::lo(wv[i]), hv[q][2 * i + 1] * inv * A::hi(wv[i]));
    *(u32x4 *)(x_out + t * H + 8 * c) = o;
  }
}

struct QkvArgs {
  const uint32_t *qkv;
  const uint32_t *qw, *kw;
  const int32_t *pos, *pages, *slots;
  const float *cos, *sin;
  uint32_t *kp, *vp;
  float *q_out, *k_out, *v_out;
  int64_t T;
  int Hq, Hkv, D, max_pos, P, page_size;
  float eps;
};

template <int DT>
__global__ __launch_bounds__(256) void qk_norm_rope_store_kernel(QkvArgs a) {
  using A = Act<DT>;
  const int NH = a.Hq + 2 * a.Hkv;
  const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= a.T * NH) return;
  const int lane = threadIdx.x & 63;
  const int64_t t = item / NH;
  const int head = (int)(item - t * NH);
  const int D2 = a.D / 2, half = a.D / 2, Q = a.D / 4;  // pairs per head, half dims, lane offset
  const bool on = lane < D2;
  const uint32_t xv = on ? a.qkv[(t * NH + head) * D2 + lane] : 0u;
  float x0 = A::lo(xv), x1 = A::hi(xv);
  const bool is_q = head < a.Hq, is_v = head >= a.Hq + a.Hkv;
  const int kvh = is_q ? 0 : (is_v ? head - a.Hq - a.Hkv : head - a.Hq);

  if (!is_v) {
    // RMSNorm over the head, rounded (the reference's q_norm / k_norm output)
    float ss = fmaf(x0, x0, x1 * x1);
#pragma unroll
    for (int x = 32; x > 0; x >>= 1) ss += __shfl_xor(ss, x);
    const float inv = rsqrtf(ss / (float)a.D + a.eps);
    const uint32_t wv = on ? (is_q ? a.qw : a.kw)[lane] : 0u;
    const uint32_t y = Act<DT>::pack2(x0 * inv * A::lo(wv), x1 * inv * A::hi(wv));
    x0 = A::lo(y);
    x1 = A::hi(y);
    // RoPE: element e < D/2 pairs with e + D/2, held Q lanes further on
    const bool lo_half = lane < Q;
    const int partner = lo_half ? lane + Q : lane - Q;
    const float p0 = __shfl(x0, partner), p1 = __shfl(x1, partner);
    const int e = 2 * (lo_half ? lane : lane - Q);  // frequency index of element 2*lane
    int p = a.pos[t];
    p = min(max(p, 0), a.max_pos - 1);
    const float c0 = on ? a.cos[(int64_t)p * half + e] : 0.f;
    const float c1 = on ? a.cos[(int64_t)p * half + e + 1] : 0.f;
    const float s0 = on ? a.sin[(int64_t)p * half + e] : 0.f;
    const float s1 = on ? a.sin[(int64_t)p * half + e + 1] : 0.f;
    float r0, r1;
    {
      // products rounded before the sum, as the reference's separate ops do
#pragma clang fp contract(off)
      if (lo_half) {
        r0 = x0 * c0 - p0 * s0;
        r1 = x1 * c1 - p1 * s1;
      } else {
        r0 = p0 * s0 + x0 * c0;
        r1 = p1 * s1 + x1 * c1;
      }
    }
    const uint32_t ro = Act<DT>::pack2(r0, r1);
    x0 = A::lo(ro);
    x1 = A::hi(ro);
    if (is_q) {
      if (on) {
        float *qo = a.q_out + (t * a.Hq + head) * a.D + 2 * lane;
        qo[0] = x0;
        qo[1] = x1;
      }
      return;
    }
  }
  // k (normed, rotated, rounded) or v (as projected): page slot and float copy
  if (!on) return;
  const int pg = a.pages[t];
  const int slot = a.slots[t];
  if (pg >= 0 && pg < a.P && slot >= 0 && slot < a.page_size) {
    const int64_t off = (((int64_t)pg * a.Hkv + kvh) * a.page_size + slot) * D2 + lane;
    (is_v ? a.vp : a.kp)[off] = Act<DT>::pack2(x0, x1);
  }
  float *fo = is_v ? a.v_out : a.k_out;
  if (fo) {
    float *o = fo + (t * a.Hkv + kvh) * a.D + 2 * lane;
    o[0] = x0;
    o[1] = x1;
  }
}

}  // namespace

hipError_t launch_combine_residual_norm(int dtype, const void *down, const void *scores,
                                        int64_t T, int k, int64_t H, const void *h,
                                        const void *w, float eps, void *h_out, void *x_out,
                                        hipStream_t st, bool split) {
  if (T == 0) return hipSuccess;
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3((unsigned)T), dim3(kNormThreads), 0, st, down,
                       (const uint16_t *)scores, k, (int)(H / 8), (const uint16_t *)h,
                       (const uint16_t *)w, eps, (uint16_t *)h_out, (uint16_t *)x_out);
  };
  if (k == 8) {
    if (dtype == DT_BF16)
      split ? go(moe_combine_residual_norm_kernel<DT_BF16, true, 8>)
            : go(moe_combine_residual_norm_kernel<DT_BF16, false, 8>);
    else
      split ? go(moe_combine_residual_norm_kernel<DT_F16, true, 8>)
            : go(moe_combine_residual_norm_kernel<DT_F16, false, 8>);
  } else if (dtype == DT_BF16) {
    split ? go(moe_combine_residual_norm_kernel<DT_BF16, true, 0>)
          : go(moe_combine_residual_norm_kernel<DT_BF16, false, 0>);
  } else {
    split ? go(moe_combine_residual_norm_kernel<DT_F16, true, 0>)
          : go(moe_combine_residual_norm_kernel<DT_F16, false, 0>);
  }
  return hipGetLastError();
}

// Embedding rows of a 4-bit affine-quantised table: out[t, c] =
// rnd(q * s + b) for the row of token t, one packed word (eight values) per
// thread.  q * s is exact in float32 (at most 4 + 11 significant bits); the
// sum is rounded to float32 and then to the activation dtype (Act's
// conversions keep the float32 value), as a float32 dequantisation followed
// by a cast.  Ids outside [0, V) give zero rows.
template <int DT>
__global__ __launch_bounds__(256) void embedding_kernel(const int32_t *__restrict__ tokens,
                                                        const uint32_t *__restrict__ wq,
                                                        const uint16_t *__restrict__ sc,
                                                        const uint16_t *__restrict__ bi, int V,
                                                        int D8, int G, int gs8,
                                                        uint16_t *__restrict__ out, int64_t T) {
  using A = Act<DT>;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // packed word
  if (i >= T * D8) return;
  const int64_t t = i / D8;
  const int w = (int)(i - t * D8);
  const int id = tokens[t];
  u32x4 o = {0u, 0u, 0u, 0u};
  if (id >= 0 && id < V) {
    const uint32_t q = wq[(int64_t)id * D8 + w];
    const int g = w / gs8;
    const float s = A::to_f32(sc[(int64_t)id * G + g]);
    const float b = A::to_f32(bi[(int64_t)id * G + g]);
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = __builtin_fmaf((float)((q >> (4 * j)) & 15u), s, b);
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = A::pack2(v[2 * j], v[2 * j + 1]);
  }
  *(u32x4 *)(out + i * 8) = o;
}

hipError_t launch_embedding(int dtype, const int32_t *tokens, int64_t T, const uint32_t *wq,
                            const void *sc, const void *bi, int64_t V, int64_t D, int gs,
                            void *out, hipStream_t st) {
  if (T == 0) return hipSuccess;
  const int64_t words = T * (D / 8);
  const unsigned grid = (unsigned)((words + 255) / 256);
  if (dtype == DT_BF16)
    hipLaunchKernelGGL(embedding_kernel<DT_BF16>, dim3(grid), dim3(256), 0, st, tokens, wq,
                       (const uint16_t *)sc, (const uint16_t *)bi, (int)V, (int)(D / 8),
                       (int)(D / gs), gs / 8, (uint16_t *)out, T);
  else
    hipLaunchKernelGGL(embedding_kernel<DT_F16>, dim3(grid), dim3(256), 0, st, tokens, wq,
                       (const uint16_t *)sc, (const uint16_t *)bi, (int)V, (int)(D / 8),
                       (int)(D / gs), gs / 8, (uint16_t *)out, T);
  return hipGetLastError();
}

bool combine_residual_norm_supports(int64_t H) { return H % 8 == 0 && H <= 8 * kNormThreads * kCombChunks; }

}  // namespace nvm

extern "C" {

int nvm_residual_rms_norm(const void *h, const void *r, const void *w, int64_t T, int64_t H,
                          float eps, int dtype, void *h_out, void *x_out, nvm_stream_t stream) {
  using namespace nvm;
  if (dtype != NVM_DTYPE_F16 && dtype != NVM_DTYPE_BF16)
    return set_error(NVM_ERR_INVALID, "residual_rms_norm: dtype must be f16 or bf16");
  if (T < 0 || H <= 0 || H % 2)
    return set_error(NVM_ERR_INVALID, "residual_rms_norm: bad shape T=%lld H=%lld", (long long)T,
                     (long long)H);
  if (H > 2 * kNormThreads * kMaxNormPairs)
    return set_error(NVM_ERR_UNSUPPORTED, "residual_rms_norm: H at most %d",
                     2 * kNormThreads * kMaxNormPairs);
  if (T == 0) return NVM_OK;
  if (!h || !w || !x_out || (r && !h_out))
    return set_error(NVM_ERR_INVALID, "residual_rms_norm: null pointer");
  const int H2 = (int)(H / 2);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == NVM_DTYPE_BF16)
    hipLaunchKernelGGL(residual_rms_norm_kernel<DT_BF16>, dim3((unsigned)T), dim3(kNormThreads), 0,
                       st, (const uint32_t *)h, (const uint32_t *)r, (const uint32_t *)w, H2, eps,
                       (uint32_t *)h_out, (uint32_t *)x_out);
  else
    hipLaunchKernelGGL(residual_rms_norm_kernel<DT_F16>, dim3((unsigned)T), dim3(kNormThreads), 0,
                       st, (const uint32_t *)h, (const uint32_t *)r, (const uint32_t *)w, H2, eps,
                       (uint32_t *)h_out, (uint32_t *)x_out);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(NVM_ERR_HIP, "residual_rms_norm: %s", hipGetErrorString(e));
  return NVM_OK;
}

int nvm_qk_norm_rope_store(const void *qkv, int64_t T, int Hq, int Hkv, int64_t D,
                           const void *q_norm_w, const void *k_norm_w, float eps,
                           const int32_t *positions, const float *cos, const float *sin,
                           int64_t max_pos, const int32_t *page_ids, const int32_t *slots,
                           void *key_pages, void *value_pages, int64_t P, int64_t page_size,
                           int dtype, float *q_out, float *k_out, float *v_out,
                           nvm_stream_t stream) {
  using namespace nvm;
  if (dtype != NVM_DTYPE_F16 && dtype != NVM_DTYPE_BF16)
    return set_error(NVM_ERR_INVALID, "qk_norm_rope_store: dtype must be f16 or bf16");
  if (T < 0 || Hq <= 0 || Hkv <= 0 || D <= 0 || max_pos <= 0 || P < 0 || page_size <= 0)
    return set_error(NVM_ERR_INVALID, "qk_norm_rope_store: bad shape");
  if (D % 4 || D > 128)
    return set_error(NVM_ERR_UNSUPPORTED, "qk_norm_rope_store: head dim %lld must be a multiple "
                     "of 4, at most 128", (long long)D);
  if (T == 0) return NVM_OK;
  if (!qkv || !q_norm_w || !k_norm_w || !positions || !cos || !sin || !page_ids || !slots ||
      !q_out || (P > 0 && (!key_pages || !value_pages)))
    return set_error(NVM_ERR_INVALID, "qk_norm_rope_store: null pointer");
  QkvArgs a{};
  a.qkv = (const uint32_t *)qkv;
  a.qw = (const uint32_t *)q_norm_w;
  a.kw = (const uint32_t *)k_norm_w;
  a.pos = positions;
  a.pages = page_ids;
  a.slots = slots;
  a.cos = cos;
  a.sin = sin;
  a.kp = (uint32_t *)key_pages;
  a.vp = (uint32_t *)value_pages;
  a.q_out = q_out;
  a.k_out = k_out;
  a.v_out = v_out;
  a.T = T;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.D = (int)D;
  a.max_pos = (int)max_pos;
  a.P = (int)P;
  a.page_size = (int)page_size;
  a.eps = eps;
  const int64_t items = T * (Hq + 2 * Hkv);
  const unsigned grid = (unsigned)((items + 3) / 4);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == NVM_DTYPE_BF16)
    hipLaunchKernelGGL(qk_norm_rope_store_kernel<DT_BF16>, dim3(grid), dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL(qk_norm_rope_store_kernel<DT_F16>, dim3(grid), dim3(256), 0, st, a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(NVM_ERR_HIP, "qk_norm_rope_store: %s", hipGetErrorString(e));
  return NVM_OK;
}

int nvm_embedding(const int32_t *tokens, int64_t T, const uint32_t *wq, const void *scales,
                  const void *biases, int64_t V, int64_t D, int group_size, int bits, int dtype,
                  void *out, nvm_stream_t stream) {
  using namespace nvm;
  if (dtype != NVM_DTYPE_F16 && dtype != NVM_DTYPE_BF16)
    return set_error(NVM_ERR_INVALID, "embedding: dtype must be f16 or bf16");
  if (bits != 4) return set_error(NVM_ERR_UNSUPPORTED, "embedding: only 4-bit weights");
  if (group_size != 32 && group_size != 64 && group_size != 128)
    return set_error(NVM_ERR_UNSUPPORTED, "embedding: group_size %d not in {32, 64, 128}",
                     group_size);
  if (T < 0 || V <= 0 || D <= 0 || D % group_size)
    return set_error(NVM_ERR_INVALID, "embedding: bad shape T=%lld V=%lld D=%lld", (long long)T,
                     (long long)V, (long long)D);
  if (V > INT32_MAX || T * (D / 8) > (int64_t)UINT32_MAX * 256)
    return set_error(NVM_ERR_UNSUPPORTED, "embedding: table or batch too large");
  if (T == 0) return NVM_OK;
  if (!tokens || !wq || !scales || !biases || !out)
    return set_error(NVM_ERR_INVALID, "embedding: null pointer");
  if (((uintptr_t)out & 15) != 0)
    return set_error(NVM_ERR_INVALID, "embedding: out must be 16-byte aligned");
  const hipError_t e = launch_embedding(dtype == NVM_DTYPE_BF16 ? DT_BF16 : DT_F16, tokens, T, wq,
                                        scales, biases, V, D, group_size, out,
                                        (hipStream_t)stream);
  if (e != hipSuccess) return set_error(NVM_ERR_HIP, "embedding: %s", hipGetErrorString(e));
  return NVM_OK;
}

}  // extern "C"
