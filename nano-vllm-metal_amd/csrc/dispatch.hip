// Dispatch: stable counting sort of routed (token, expert) pairs by expert
// (the `argsort` pair of layers/moe.py:16-17), built from sort.h.
//
// Up to kSortChunk pairs sort in one block.  Larger inputs take two launches
// over blocks of kSortChunk pairs: per-block histograms, then each block
// derives its output bases from all histograms (exclusive prefix over
// experts of the totals, plus the counts of the blocks before it) and
// scatters its pairs.  No atomics and no host synchronisation.
#include <algorithm>

#include "internal.h"
#include "sort.h"

namespace nvm {

namespace {

constexpr int kSortThreads = 1024;

int bits_for(int64_t E) {
  int nbits = 0;
  while ((1ll << nbits) < E) ++nbits;
  return nbits;
}

__global__ __launch_bounds__(kSortThreads) void dispatch_kernel(const int32_t *__restrict__ ids,
                                                                int n, int E, int nbits,
                                                                int32_t *__restrict__ offsets,
                                                                int32_t *__restrict__ sorted) {
  extern __shared__ int lds[];
  block_sort([&](int p) { return ids[p]; }, n, E, nbits, lds, offsets, sorted);
}

// Histogram of block b's pairs [b * chunk, ...) into counts[b][E].
__global__ __launch_bounds__(kSortThreads) void dispatch_count_kernel(
    const int32_t *__restrict__ ids, int n, int E, int nbits, int chunk,
    int32_t *__restrict__ counts) {
  extern __shared__ int lds[];
  const int W = blockDim.x >> 6;
  const int tid = threadIdx.x, wv = tid >> 6;
  const int b0 = blockIdx.x * chunk, nb = min(chunk, n - b0);
  int *cnt = lds;  // [W][E]
  for (int i = tid; i < W * E; i += blockDim.x) cnt[i] = 0;
  __syncthreads();
  int start, end;
  sort_range(nb, W, wv, start, end);
  sort_count([&](int p) { return ids[b0 + p]; }, start, end, E, nbits, cnt + wv * E);
  __syncthreads();
  for (int e = tid; e < E; e += blockDim.x) {
    int s = 0;
    for (int w = 0; w < W; ++w) s += cnt[w * E + e];
    counts[(int64_t)blockIdx.x * E + e] = s;
  }
}

// Output bases of block b from all block histograms, then the stable scatter
// of its pairs.  Block 0 also writes the expert offsets.
__global__ __launch_bounds__(kSortThreads) void dispatch_scatter_kernel(
    const int32_t *__restrict__ ids, int n, int E, int nbits, int chunk, int nblocks,
    const int32_t *__restrict__ counts, int32_t *__restrict__ offsets,
    int32_t *__restrict__ sorted) {
  extern __shared__ int lds[];
  const int W = blockDim.x >> 6;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int b0 = blockIdx.x * chunk, nb = min(chunk, n - b0);
  int *cnt = lds;           // [W][E]
  int *tot = lds + W * E;   // [E]: totals, then expert offsets
  int *pre = tot + E;       // [E]: pairs of expert e in blocks before this one
  for (int i = tid; i < W * E; i += blockDim.x) cnt[i] = 0;
  for (int e = tid; e < E; e += blockDim.x) {
    int t = 0, p = 0;
    for (int b = 0; b < nblocks; ++b) {
      const int c = counts[(int64_t)b * E + e];
      t += c;
      p += b < (int)blockIdx.x ? c : 0;
    }
    tot[e] = t;
    pre[e] = p;
  }
  __syncthreads();
  int start, end;
  sort_range(nb, W, wv, start, end);
  auto get = [&](int p) { return ids[b0 + p]; };
  sort_count(get, start, end, E, nbits, cnt + wv * E);
  if (wv == 0) {
    int carry = 0;
    for (int c0 = 0; c0 < E; c0 += 64) {
      const int e = c0 + lane;
      const int v = e < E ? tot[e] : 0;
      const int inc = wave_incl_scan(v, lane);
      if (e < E) {
        tot[e] = carry + inc - v;
        if (blockIdx.x == 0) offsets[e] = carry + inc - v;
      }
      carry += __shfl(inc, 63);
    }
    if (lane == 0 && blockIdx.x == 0) offsets[E] = carry;
  }
  __syncthreads();
  // run[w][e] = offset[e] + earlier blocks + earlier wavefronts of this block
  for (int e = tid; e < E; e += blockDim.x) {
    int run = tot[e] + pre[e];
    for (int w = 0; w < W; ++w) {
      const int c = cnt[w * E + e];
      cnt[w * E + e] = run;
      run += c;
    }
  }
  __syncthreads();
  // pair indices of the whole input are written
  sort_scatter(get, start, end, E, nbits, cnt + wv * E, sorted, b0);
}

// launch_dispatch_hist: block b sorts the pairs of count runs [b CB, (b+1) CB)
// (runs of cb_pairs pairs).  Its output bases come from the run histograms:
// the expert totals (offsets) and the pairs of each expert in earlier runs.
// Thread (quad, part) sums experts 4 quad..4 quad+3 over runs part, part + P,
// ... with 16-byte loads, eight in flight at a time (E a multiple of 4), and
// the P parts meet in LDS.
constexpr int kHistLoads = 8;
__global__ __launch_bounds__(kSortThreads) void dispatch_hist_kernel(
    const int32_t *__restrict__ ids, int n, int E, int nbits, const int32_t *__restrict__ counts,
    int n_cb, int cb_pairs, int CB, int32_t *__restrict__ offsets, int32_t *__restrict__ sorted) {
  extern __shared__ int lds[];
  const int W = blockDim.x >> 6;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int Q = E / 4;                // expert quads
  const int P = (int)blockDim.x / Q;  // parts (blockDim >= Q)
  const int cb0 = blockIdx.x * CB;
  const int b0 = cb0 * cb_pairs, nb = min(CB * cb_pairs, n - b0);
  int *cnt = lds;           // [W][E]
  int *tot = lds + W * E;   // [E]: totals, then expert offsets
  int *pre = tot + E;       // [E]: pairs of expert e in runs before this block's
  int *ps = pre + E;        // [P][E] partial totals
  int *pp = ps + P * E;     // [P][E] partial prefixes
  for (int i = tid; i < W * E; i += blockDim.x) cnt[i] = 0;
  if (tid < P * Q) {
    const int qd = tid % Q, p = tid / Q;
    const rsrc_t cr = make_rsrc(counts, (uint32_t)((int64_t)n_cb * E * 4));
    u32x4 t = {0u, 0u, 0u, 0u}, q = {0u, 0u, 0u, 0u};
    for (int r0 = p; r0 < n_cb; r0 += kHistLoads * P) {
      u32x4 v[kHistLoads];
#pragma unroll
      for (int u = 0; u < kHistLoads; ++u) {
        const int r = r0 + u * P;
        v[u] = bload16(cr, r < n_cb ? (r * E + 4 * qd) * 4 : kMaskedOffset, 0);
      }
#pragma unroll
      for (int u = 0; u < kHistLoads; ++u) {
        t += v[u];
        if (r0 + u * P < cb0) q += v[u];
      }
    }
    *(u32x4 *)(ps + p * E + 4 * qd) = t;
    *(u32x4 *)(pp + p * E + 4 * qd) = q;
  }
  __syncthreads();
  for (int e = tid; e < E; e += blockDim.x) {
    int t = 0, q = 0;
    for (int p = 0; p < P; ++p) {
      t += ps[p * E + e];
      q += pp[p * E + e];
    }
    tot[e] = t;
    pre[e] = q;
  }
  __syncthreads();
  int start, end;
  sort_range(nb, W, wv, start, end);
  auto get = [&](int p) { return ids[b0 + p]; };
  sort_count(get, start, end, E, nbits, cnt + wv * E);
  if (wv == 0) {
    int carry = 0;
    for (int c0 = 0; c0 < E; c0 += 64) {
      const int e = c0 + lane;
      const int v = e < E ? tot[e] : 0;
      const int inc = wave_incl_scan(v, lane);
      if (e < E) {
        tot[e] = carry + inc - v;
        if (blockIdx.x == 0) offsets[e] = carry + inc - v;
      }
      carry += __shfl(inc, 63);
    }
    if (lane == 0 && blockIdx.x == 0) offsets[E] = carry;
  }
  __syncthreads();
  // run[w][e] = offset[e] + earlier runs + earlier wavefronts of this block
  for (int e = tid; e < E; e += blockDim.x) {
    int run = tot[e] + pre[e];
    for (int w = 0; w < W; ++w) {
      const int c = cnt[w * E + e];
      cnt[w * E + e] = run;
      run += c;
    }
  }
  __syncthreads();
  sort_scatter(get, start, end, E, nbits, cnt + wv * E, sorted, b0);
}

}  // namespace

hipError_t launch_dispatch_hist(const int32_t *ids, int64_t n, int64_t E, const int32_t *counts,
                                int64_t n_cb, int cb_pairs, int32_t *offsets, int32_t *sorted,
                                hipStream_t st) {
  if (n <= 0 || cb_pairs <= 0 || E <= 0 || E > kMaxExperts || n_cb * cb_pairs < n)
    return hipErrorInvalidValue;
  const int nbits = bits_for(E);
  const int W = kSortThreads / 64;
  if (E % 4 != 0 || E / 4 > kSortThreads) return hipErrorInvalidValue;
  const int P = kSortThreads / ((int)E / 4);
  // about 1024 pairs a block, whole runs
  const int CB = std::max(1, 1024 / cb_pairs);
  if ((int64_t)CB * cb_pairs > kSortChunk) return hipErrorInvalidValue;
  const int nblocks = (int)((n_cb + CB - 1) / CB);
  const size_t lds = sizeof(int) * (size_t)(W * E + 2 * E + 2 * P * E);
  if (lds > 65536) return hipErrorInvalidValue;
  hipLaunchKernelGGL(dispatch_hist_kernel, dim3(nblocks), dim3(kSortThreads), lds, st, ids, (int)n,
                     (int)E, nbits, counts, (int)n_cb, cb_pairs, CB, offsets, sorted);
  return hipGetLastError();
}

int64_t dispatch_workspace_bytes(int64_t n, int64_t E) {
  if (n <= kSortChunk) return 0;
  return (int64_t)sizeof(int32_t) * ((n + kSortChunk - 1) / kSortChunk) * E;
}

hipError_t launch_dispatch(const int32_t *ids, int64_t n, int64_t E, int32_t *offsets,
                           int32_t *sorted, void *workspace, hipStream_t st) {
  const int nbits = bits_for(E);
  const int W = kSortThreads / 64;
  if (n <= kSortChunk) {
    const size_t lds = sizeof(int) * (size_t)(W * E + E);
    hipLaunchKernelGGL(dispatch_kernel, dim3(1), dim3(kSortThreads), lds, st, ids, (int)n, (int)E,
                       nbits, offsets, sorted);
    return hipGetLastError();
  }
  if (!workspace) return hipErrorInvalidValue;
  const int nblocks = (int)((n + kSortChunk - 1) / kSortChunk);
  int32_t *counts = (int32_t *)workspace;
  hipLaunchKernelGGL(dispatch_count_kernel, dim3(nblocks), dim3(kSortThreads),
                     sizeof(int) * (size_t)W * E, st, ids, (int)n, (int)E, nbits, kSortChunk,
                     counts);
  hipLaunchKernelGGL(dispatch_scatter_kernel, dim3(nblocks), dim3(kSortThreads),
                     sizeof(int) * (size_t)(W * E + 2 * E), st, ids, (int)n, (int)E, nbits,
                     kSortChunk, nblocks, counts, offsets, sorted);
  return hipGetLastError();
}

}  // namespace nvm
