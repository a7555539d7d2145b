// Combine: y[t] = sum_j score[t,j] * expert_output[t,j], back in token order.
//
// Restates `mx.sum(expert_output * expand_dims(expert_scores, -1), axis=-2)`
// (layers/moe.py:85-86).  The product is an activation-dtype tensor in the
// reference, so each term is rounded to act before the float32 sum, which is
// rounded once.  The per-pair expert outputs were already written in flat pair
// order (t*k + j) by the down product, so each thread reads k contiguous
// 16-byte chunks and no atomics are needed: the sum order is fixed.
#include "common.h"
#include "internal.h"

namespace nvm {

namespace {

// SPLIT: the down outputs come as the float32 sums of the two halves of the
// down reduction (down_vals).
template <int DT, bool SPLIT>
__global__ __launch_bounds__(256) void combine_kernel(const void *__restrict__ down,
                                                      const uint16_t *__restrict__ scores,
                                                      int64_t T, int k, int64_t H,
                                                      uint16_t *__restrict__ y) {
  using A = Act<DT>;
  hoist_args(down, scores, T, k, H, y);
  const int64_t chunks = H / 8;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= T * chunks) return;
  const int64_t t = idx / chunks, c = idx - t * chunks;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  // NB pairs per batch, all their loads in flight together
  constexpr int NB = SPLIT ? 4 : 8;
  for (int j0 = 0; j0 < k; j0 += NB) {
    float dv[NB][8];
    uint32_t sv[NB];
#pragma unroll
    for (int jj = 0; jj < NB; ++jj) sv[jj] = j0 + jj < k ? scores[t * k + j0 + jj] : 0u;
    down_vals<DT, SPLIT, NB>(down, T * k, t, k, j0, H, c, dv);
#pragma unroll
    for (int jj = 0; jj < NB; ++jj) {
      if (j0 + jj >= k) break;
      const float s = A::to_f32(sv[jj]);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] += round_act<DT>(dv[jj][i] * s);
    }
  }
  u32x4 o;
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = A::pack2(acc[2 * i], acc[2 * i + 1]);
  *(u32x4 *)(y + t * H + 8 * c) = o;
}

template <bool SPLIT>
hipError_t launch_combine_t(int dtype, const void *down, const void *scores, int64_t T, int k,
                            int64_t H, void *y, hipStream_t st) {
  // one wavefront per block: a decode batch (32 tokens x 2048) spreads over
  // 128 CUs instead of 32 (the kernel is one round trip of latency per thread)
  const int64_t work = T * (H / 8);
  dim3 grid((unsigned)((work + 63) / 64));
  if (dtype == DT_BF16)
    hipLaunchKernelGGL((combine_kernel<DT_BF16, SPLIT>), grid, dim3(64), 0, st, down,
                       (const uint16_t *)scores, T, k, H, (uint16_t *)y);
  else
    hipLaunchKernelGGL((combine_kernel<DT_F16, SPLIT>), grid, dim3(64), 0, st, down,
                       (const uint16_t *)scores, T, k, H, (uint16_t *)y);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_combine(int dtype, const void *down, const void *scores, int64_t T, int k,
                          int64_t H, void *y, hipStream_t st) {
  return launch_combine_t<false>(dtype, down, scores, T, k, H, y, st);
}

hipError_t launch_combine_split(int dtype, const float *part, const void *scores, int64_t T, int k,
                                int64_t H, void *y, hipStream_t st) {
  return launch_combine_t<true>(dtype, part, scores, T, k, H, y, st);
}

}  // namespace nvm
