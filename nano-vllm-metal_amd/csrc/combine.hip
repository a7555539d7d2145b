// Combine: y[t] = sum_j score[t,j] * expert_output[t,j], back in token order.
//
// Restates `mx.sum(expert_output * expand_dims(expert_scores, -1), axis=-2)`
// (layers/moe.py:85-86).  The product is an activation-dtype tensor in the
// reference, so each term is rounded to act before the float32 sum, which is
// rounded once.  The per-pair expert outputs were already written in flat pair
// order (t*k + j) by the down product, so each thread reads k contiguous
// 16-byte chunks and no atomics are needed: the sum order is fixed.
#include <cstdlib>

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

// Small batches: CPT (2 or 4) columns a thread and every pair's loads in
// flight at once, the top-k a compile-time count (KK), so that a decode
// batch spreads over two or four times the wavefronts of combine_kernel with
// that much fewer bytes each (a wavefront's bytes in flight bound its time).
// The arithmetic per column is combine_kernel's.
template <int DT, bool SPLIT, int CPT, int KK>
__global__ __launch_bounds__(64) void combine_narrow_kernel(const void *__restrict__ down,
                                                            const uint16_t *__restrict__ scores,
                                                            int64_t T, int64_t H,
                                                            uint16_t *__restrict__ y) {
  using A = Act<DT>;
  static_assert(CPT == 2 || CPT == 4, "two or four columns a thread");
  hoist_args(down, scores, T, H, y);
  const int64_t groups = H / CPT;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= T * groups) return;
  const int64_t t = idx / groups, c = idx - t * groups;
  const int64_t TK = T * KK;
  // per pair: CPT float32 of each half (SPLIT) or CPT act values
  typedef uint32_t w_t __attribute__((ext_vector_type(SPLIT ? CPT : CPT / 2)));
  w_t lo[KK], hi[KK];
  uint32_t sv[KK];
#pragma unroll
  for (int j = 0; j < KK; ++j) {
    const int64_t p = t * KK + j;
    sv[j] = scores[p];
    if constexpr (SPLIT) {
      const float *part = (const float *)down;
      lo[j] = *(const w_t *)(part + p * H + CPT * c);
      hi[j] = *(const w_t *)(part + (TK + p) * H + CPT * c);
    } else {
      lo[j] = *(const w_t *)((const uint16_t *)down + p * H + CPT * c);
    }
  }
  float acc[CPT];
#pragma unroll
  for (int i = 0; i < CPT; ++i) acc[i] = 0.f;
#pragma unroll
  for (int j = 0; j < KK; ++j) {
    const float s = A::to_f32(sv[j]);
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      float dv;
      if constexpr (SPLIT)
        dv = round_act<DT>(__uint_as_float(lo[j][i]) + __uint_as_float(hi[j][i]));
      else
        dv = (i & 1) ? A::hi(lo[j][i >> 1]) : A::lo(lo[j][i >> 1]);
      acc[i] += round_act<DT>(dv * s);
    }
  }
  typedef uint32_t o_t __attribute__((ext_vector_type(CPT / 2)));
  o_t o;
#pragma unroll
  for (int i = 0; i < CPT / 2; ++i) o[i] = A::pack2(acc[2 * i], acc[2 * i + 1]);
  *(o_t *)(y + t * H + CPT * c) = o;
}

// Columns a thread for the narrow kernel (0: combine_kernel's eight): the
// widest that still gives the launch 256 wavefronts.  NVM_COMBINE_CPT=2/4/8
// overrides it.
int narrow_cpt(int64_t T, int64_t H, int k) {
  if (k != 8 || H % 4 != 0) return 0;
  const char *v = getenv("NVM_COMBINE_CPT");
  if (v && (v[0] == '2' || v[0] == '4')) return v[0] - '0';
  if (v && v[0] == '8') return 0;
  if (T * H / 8 >= 256 * 64) return 0;
  return T * H / 4 >= 256 * 64 ? 4 : 2;
}

template <int DT, bool SPLIT>
hipError_t launch_narrow(int cpt, const void *down, const void *scores, int64_t T, int64_t H,
                         void *y, hipStream_t st) {
  const int64_t work = T * (H / cpt);
  const dim3 grid((unsigned)((work + 63) / 64));
  if (cpt == 4)
    hipLaunchKernelGGL((combine_narrow_kernel<DT, SPLIT, 4, 8>), grid, dim3(64), 0, st, down,
                       (const uint16_t *)scores, T, H, (uint16_t *)y);
  else
    hipLaunchKernelGGL((combine_narrow_kernel<DT, SPLIT, 2, 8>), grid, dim3(64), 0, st, down,
                       (const uint16_t *)scores, T, H, (uint16_t *)y);
  return hipGetLastError();
}

template <bool SPLIT>
hipError_t launch_combine_t(int dtype, const void *down, const void *scores, int64_t T, int k,
                            int64_t H, void *y, hipStream_t st) {
  if (const int cpt = narrow_cpt(T, H, k)) {
    return dtype == DT_BF16 ? launch_narrow<DT_BF16, SPLIT>(cpt, down, scores, T, H, y, st)
                            : launch_narrow<DT_F16, SPLIT>(cpt, down, scores, T, H, y, st);
  }
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
