// Dispatch: stable counting sort of routed (token, expert) pairs by expert.
//
// Replaces the `argsort(flat_expert_ids)` of layers/moe.py:16-17: for each
// expert in ascending order, the pair indices that chose it, ascending.  The
// ordering path uses no atomics: within a wavefront, lanes holding the same
// expert find each other with ballots over the bits of the expert id, their
// rank is a popcount of the lower-lane mask, and one leader lane per expert
// advances the wavefront's private counter.  Wavefronts own contiguous pair
// ranges, and their bases come from a prefix over (expert, wavefront), so the
// result is deterministic and identical to a stable sort.
#include "common.h"
#include "internal.h"

namespace nvm {

namespace {

constexpr int kDispatchThreads = 1024;

__device__ __forceinline__ uint64_t peers_of(int e, bool valid, int nbits) {
  uint64_t peers = __ballot(valid);
  for (int b = 0; b < nbits; ++b) {
    const bool bit = (e >> b) & 1;
    const uint64_t m = __ballot(bit);
    peers &= bit ? m : ~m;
  }
  return peers;
}

__device__ __forceinline__ int wave_incl_scan(int v, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int u = __shfl_up(v, o);
    if (lane >= o) v += u;
  }
  return v;
}

// One block of 1024 threads.  Pairs with ids outside [0, E) are dropped.
__global__ __launch_bounds__(kDispatchThreads) void dispatch_kernel(
    const int32_t *__restrict__ ids, int n, int E, int nbits, int32_t *__restrict__ offsets,
    int32_t *__restrict__ sorted) {
  extern __shared__ int lds[];
  const int W = blockDim.x >> 6;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  int *cnt = lds;            // [W][E]: per-wavefront counts, then bases
  int *base = lds + W * E;   // [E]: expert base offsets
  for (int i = tid; i < W * E; i += blockDim.x) cnt[i] = 0;
  __syncthreads();

  const int chunk = (((n + W - 1) / W) + 63) & ~63;
  const int start = min(n, wv * chunk), end = min(n, start + chunk);
  const uint64_t lower = (1ull << lane) - 1ull;

  // pass 1: per-wavefront histogram
  for (int p0 = start; p0 < end; p0 += 64) {
    const int p = p0 + lane;
    int e = p < end ? ids[p] : -1;
    const bool valid = e >= 0 && e < E;
    if (!valid) e = 0;
    const uint64_t peers = peers_of(e, valid, nbits);
    if (valid && (peers & lower) == 0) cnt[wv * E + e] += __popcll(peers);
  }
  __syncthreads();

  // per-expert totals; per-wavefront counts become exclusive prefixes
  for (int e = tid; e < E; e += blockDim.x) {
    int run = 0;
    for (int w = 0; w < W; ++w) {
      const int c = cnt[w * E + e];
      cnt[w * E + e] = run;
      run += c;
    }
    base[e] = run;
  }
  __syncthreads();

  // exclusive scan of the totals by wavefront 0
  if (wv == 0) {
    int carry = 0;
    for (int c0 = 0; c0 < E; c0 += 64) {
      const int e = c0 + lane;
      const int v = e < E ? base[e] : 0;
      const int inc = wave_incl_scan(v, lane);
      if (e < E) {
        base[e] = carry + inc - v;
        offsets[e] = carry + inc - v;
      }
      carry += __shfl(inc, 63);
    }
    if (lane == 0) offsets[E] = carry;
  }
  __syncthreads();

  // pass 2: order-preserving scatter
  for (int p0 = start; p0 < end; p0 += 64) {
    const int p = p0 + lane;
    int e = p < end ? ids[p] : -1;
    const bool valid = e >= 0 && e < E;
    if (!valid) e = 0;
    const uint64_t peers = peers_of(e, valid, nbits);
    if (valid) {
      const int run = cnt[wv * E + e];
      sorted[base[e] + run + __popcll(peers & lower)] = p;
    }
    // every lane has read its run before the leader advances it
    __builtin_amdgcn_wave_barrier();
    if (valid && (peers & lower) == 0) cnt[wv * E + e] += __popcll(peers);
    __builtin_amdgcn_wave_barrier();
  }
}

}  // namespace

hipError_t launch_dispatch(const int32_t *ids, int64_t n, int64_t E, int32_t *offsets,
                           int32_t *sorted, hipStream_t st) {
  int nbits = 0;
  while ((1ll << nbits) < E) ++nbits;
  const int W = kDispatchThreads / 64;
  const size_t lds = sizeof(int) * (size_t)(W * E + E);
  hipLaunchKernelGGL(dispatch_kernel, dim3(1), dim3(kDispatchThreads), lds, st, ids, (int)n,
                     (int)E, nbits, offsets, sorted);
  return hipGetLastError();
}

}  // namespace nvm
