// Router: logits = x . dequant(Wr)^T, precise softmax, top-k, renormalisation.
//
// Restates layers/moe.py:37-49 (route_topk) and the router GEMV it calls
// (layers/linear.py:92-126 -> metal/src/quantized_matmul.cpp:117-145).
//
// Every value the reference materialises in the activation dtype (logits,
// probabilities, scores) is produced here as the correctly rounded value of
// the exact mathematical result: the dot products and the softmax run in
// float64 and are rounded once, directly from float64.  A float64 sum of at
// most a few thousand products of a bf16/fp16 activation and an fp32-exact
// weight is within ~2^-40 relative of the exact sum, so the rounded logits,
// and with them the top-k ids, do not depend on summation order.
#include "common.h"
#include "internal.h"

namespace nvm {

namespace {

constexpr int kRouteChunk = 256;  // H elements staged per LDS pass

// part[z][t][e] (or the final act logits when `fin`) for tokens of this block
// (one per lane), experts [e0, e0+EG) and hidden range of split z.
template <int DT, int EG>
__global__ void route_partial_kernel(const uint16_t *__restrict__ x, int T, int H,
                                     const uint32_t *__restrict__ wr,
                                     const uint16_t *__restrict__ sr,
                                     const uint16_t *__restrict__ br, int E, int gs, int HR,
                                     double *__restrict__ part, uint16_t *__restrict__ fin) {
  extern __shared__ double wlds[];  // [EG][kRouteChunk]
  const int tid = threadIdx.x;
  const int t = blockIdx.x * blockDim.x + tid;
  const int e0 = blockIdx.y * EG;
  const int z = blockIdx.z;
  const int h_begin = z * HR;
  const int words_per_row = H / 8;
  const int groups_per_row = H / gs;

  double acc[EG];
#pragma unroll
  for (int e = 0; e < EG; ++e) acc[e] = 0.0;

  const uint16_t *xrow = x + (int64_t)(t < T ? t : 0) * H;

  for (int c0 = 0; c0 < HR; c0 += kRouteChunk) {
    const int len = min(kRouteChunk, HR - c0);
    const int wpr = len / 8;  // words per expert in this chunk
    __syncthreads();
    for (int idx = tid; idx < EG * wpr; idx += blockDim.x) {
      const int e = idx / wpr, wj = idx - e * wpr;
      const int ge = e0 + e;
      double *dst = wlds + e * kRouteChunk + wj * 8;
      if (ge < E) {
        const int col = h_begin + c0 + wj * 8;
        const uint32_t q = wr[(int64_t)ge * words_per_row + col / 8];
        const int g = col / gs;
        const double s = (double)Act<DT>::to_f32(sr[(int64_t)ge * groups_per_row + g]);
        const double b = (double)Act<DT>::to_f32(br[(int64_t)ge * groups_per_row + g]);
#pragma unroll
        for (int j = 0; j < 8; ++j) dst[j] = fma((double)((q >> (4 * j)) & 0xFu), s, b);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) dst[j] = 0.0;
      }
    }
    __syncthreads();
    if (t < T) {
      const uint16_t *xp = xrow + h_begin + c0;
      for (int h = 0; h < len; h += 8) {
        const u32x4 xv = ldg16(xp + h);
        double xd[8];
        xd[0] = Act<DT>::lo(xv.x);
        xd[1] = Act<DT>::hi(xv.x);
        xd[2] = Act<DT>::lo(xv.y);
        xd[3] = Act<DT>::hi(xv.y);
        xd[4] = Act<DT>::lo(xv.z);
        xd[5] = Act<DT>::hi(xv.z);
        xd[6] = Act<DT>::lo(xv.w);
        xd[7] = Act<DT>::hi(xv.w);
#pragma unroll
        for (int e = 0; e < EG; ++e) {
          const double *w = wlds + e * kRouteChunk + h;
#pragma unroll
          for (int j = 0; j < 8; ++j) acc[e] = fma(xd[j], w[j], acc[e]);
        }
      }
    }
  }
  if (t >= T) return;
#pragma unroll
  for (int e = 0; e < EG; ++e) {
    const int ge = e0 + e;
    if (ge >= E) break;
    if (fin)
      fin[(int64_t)t * E + ge] = act_from_f64<DT>(acc[e]);
    else
      part[((int64_t)z * T + t) * E + ge] = acc[e];
  }
}

__device__ __forceinline__ double wave_max(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmax(v, __shfl_xor(v, o));
  return v;
}
__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, o));
  return v;
}

constexpr int kMaxExpertSlots = 8;  // experts per lane: E <= 512

// One wavefront per token: sum the split partials, round the logits, softmax
// in float64, select top-k by (prob desc, index asc), renormalise.
template <int DT>
__global__ __launch_bounds__(256) void route_finalize_kernel(
    const double *__restrict__ part, int splits, int T, int E, int k, int norm,
    uint16_t *__restrict__ probs, int32_t *__restrict__ ids, uint16_t *__restrict__ scores) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (t >= T) return;
  constexpr int P = Act<DT>::kPrec, EMIN = Act<DT>::kEmin;

  double lg[kMaxExpertSlots];
  double mloc = -INFINITY;
#pragma unroll
  for (int j = 0; j < kMaxExpertSlots; ++j) {
    const int e = lane + 64 * j;
    lg[j] = -INFINITY;
    if (e < E) {
      double s = 0.0;
      for (int z = 0; z < splits; ++z) s += part[((int64_t)z * T + t) * E + e];
      lg[j] = round_f64_to(s, P, EMIN);
      mloc = fmax(mloc, lg[j]);
    }
  }
  const double m = wave_max(mloc);
  double p[kMaxExpertSlots];
  double sloc = 0.0;
#pragma unroll
  for (int j = 0; j < kMaxExpertSlots; ++j) {
    const int e = lane + 64 * j;
    p[j] = (e < E) ? exp(lg[j] - m) : 0.0;
    sloc += p[j];
  }
  const double sum = wave_sum(sloc);
  uint32_t key[kMaxExpertSlots];
#pragma unroll
  for (int j = 0; j < kMaxExpertSlots; ++j) {
    const int e = lane + 64 * j;
    key[j] = 0;
    if (e < E) {
      const uint16_t pb = act_from_f64<DT>(p[j] / sum);
      if (probs) probs[(int64_t)t * E + e] = pb;
      // probabilities are >= +0, so their bit patterns order like their values;
      // the low half prefers the lower expert index on ties
      key[j] = ((uint32_t)pb << 16) | (uint32_t)(0xFFFF - e);
    }
  }
  int my_id = 0;
  double my_p = 0.0, psum = 0.0;
  for (int i = 0; i < k; ++i) {
    uint32_t best = 0;
#pragma unroll
    for (int j = 0; j < kMaxExpertSlots; ++j) best = max(best, key[j]);
    best = wave_max_u32(best);
    const int e = 0xFFFF - (int)(best & 0xFFFFu);
    const double pv = (double)Act<DT>::to_f32(best >> 16);
    psum += pv;  // at most k act values: exact in float64
    if (lane == i) {
      my_id = e;
      my_p = pv;
    }
    if ((e & 63) == lane) {
#pragma unroll
      for (int j = 0; j < kMaxExpertSlots; ++j)
        if (j == (e >> 6)) key[j] = 0;
    }
  }
  if (lane < k) {
    double sc = my_p;
    if (norm) {
      const double denom = round_f64_to(psum, P, EMIN);
      sc = my_p / denom;
    }
    ids[(int64_t)t * k + lane] = my_id;
    scores[(int64_t)t * k + lane] = act_from_f64<DT>(sc);
  }
}

template <int DT, int EG>
hipError_t launch_partial_t(const void *x, int64_t T, int64_t H, const uint32_t *wr,
                            const void *sr, const void *br, int64_t E, int gs, int splits,
                            double *partial, void *fin, hipStream_t st) {
  const int waves = (int)std::min<int64_t>(4, (T + 63) / 64);
  const int threads = 64 * waves;
  dim3 grid((unsigned)((T + threads - 1) / threads), (unsigned)((E + EG - 1) / EG),
            (unsigned)splits);
  const size_t lds = sizeof(double) * EG * kRouteChunk;
  hipLaunchKernelGGL((route_partial_kernel<DT, EG>), grid, dim3(threads), lds, st,
                     (const uint16_t *)x, (int)T, (int)H, wr, (const uint16_t *)sr,
                     (const uint16_t *)br, (int)E, gs, (int)(H / splits), partial,
                     (uint16_t *)fin);
  return hipGetLastError();
}

}  // namespace

int route_experts_per_block(int64_t T) { return T >= 512 ? 16 : 4; }

int route_splits(int64_t T, int64_t H) {
  // enough blocks to fill the chip: long H ranges for big token counts,
  // short ones (more splits) for decode-sized batches
  const int64_t target = T >= 512 ? 512 : 128;
  for (int s = 16; s > 1; s >>= 1)
    if (H % s == 0 && (H / s) % 8 == 0 && H / s >= target) return s;
  return 1;
}

hipError_t launch_route_partial(int dtype, const void *x, int64_t T, int64_t H,
                                const uint32_t *wr, const void *sr, const void *br, int64_t E,
                                int gs, int splits, double *partial, void *fin, hipStream_t st) {
  const bool big = route_experts_per_block(T) == 16;
  if (dtype == DT_BF16)
    return big ? launch_partial_t<DT_BF16, 16>(x, T, H, wr, sr, br, E, gs, splits, partial, fin, st)
               : launch_partial_t<DT_BF16, 4>(x, T, H, wr, sr, br, E, gs, splits, partial, fin, st);
  return big ? launch_partial_t<DT_F16, 16>(x, T, H, wr, sr, br, E, gs, splits, partial, fin, st)
             : launch_partial_t<DT_F16, 4>(x, T, H, wr, sr, br, E, gs, splits, partial, fin, st);
}

hipError_t launch_route_finalize(int dtype, const double *partial, int splits, int64_t T,
                                 int64_t E, int k, int norm, void *probs, int32_t *ids,
                                 void *scores, hipStream_t st) {
  dim3 grid((unsigned)((T + 3) / 4));
  if (dtype == DT_BF16)
    hipLaunchKernelGGL((route_finalize_kernel<DT_BF16>), grid, dim3(256), 0, st, partial, splits,
                       (int)T, (int)E, k, norm, (uint16_t *)probs, ids, (uint16_t *)scores);
  else
    hipLaunchKernelGGL((route_finalize_kernel<DT_F16>), grid, dim3(256), 0, st, partial, splits,
                       (int)T, (int)E, k, norm, (uint16_t *)probs, ids, (uint16_t *)scores);
  return hipGetLastError();
}

}  // namespace nvm
