// Stable counting sort of routed pairs by expert, as device building blocks.
//
// Restates the `argsort(flat_expert_ids)` of layers/moe.py:16-17: for each
// expert in ascending order, the pair indices that chose it, ascending.  The
// ordering path uses no atomics: within a wavefront, lanes holding the same
// expert find each other with ballots over the bits of the expert id, their
// rank is a popcount of the lower-lane mask, and one leader lane per expert
// advances the wavefront's private counter.  Wavefronts own contiguous pair
// ranges, and their bases come from a prefix over (expert, wavefront), so the
// result is deterministic and identical to a stable sort.  Pairs whose id
// lies outside [0, E) are left out.
#pragma once

#include "common.h"

namespace nvm {

// Lanes of the wavefront holding the same expert id as this lane.
__device__ __forceinline__ uint64_t sort_peers(int e, bool valid, int nbits) {
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

// Pair range [start, end) of wavefront w when W wavefronts split n pairs in
// 64-pair steps.
__device__ __forceinline__ void sort_range(int n, int W, int w, int &start, int &end) {
  const int chunk = (((n + W - 1) / W) + 63) & ~63;
  start = min(n, w * chunk);
  end = min(n, start + chunk);
}

// Pass 1: this wavefront's histogram of its pair range into cnt[E] (LDS,
// zeroed by the caller).  `get(p)` returns the id of pair p.
template <class Get>
__device__ __forceinline__ void sort_count(Get get, int start, int end, int E, int nbits, int *cnt) {
  const int lane = threadIdx.x & 63;
  const uint64_t lower = (1ull << lane) - 1ull;
  for (int p0 = start; p0 < end; p0 += 64) {
    const int p = p0 + lane;
    int e = p < end ? get(p) : -1;
    const bool valid = e >= 0 && e < E;
    if (!valid) e = 0;
    const uint64_t peers = sort_peers(e, valid, nbits);
    if (valid && (peers & lower) == 0) cnt[e] += __popcll(peers);
  }
}

// Pass 2: order-preserving scatter of this wavefront's pair range; run[e]
// (LDS) holds the wavefront's first output slot for expert e and advances.
// Pair p is written as pbase + p.
template <class Get>
__device__ __forceinline__ void sort_scatter(Get get, int start, int end, int E, int nbits, int *run,
                                             int32_t *sorted, int pbase = 0) {
  const int lane = threadIdx.x & 63;
  const uint64_t lower = (1ull << lane) - 1ull;
  for (int p0 = start; p0 < end; p0 += 64) {
    const int p = p0 + lane;
    int e = p < end ? get(p) : -1;
    const bool valid = e >= 0 && e < E;
    if (!valid) e = 0;
    const uint64_t peers = sort_peers(e, valid, nbits);
    if (valid) sorted[run[e] + __popcll(peers & lower)] = pbase + p;
    // every lane has read its run before the leader advances it
    __builtin_amdgcn_wave_barrier();
    if (valid && (peers & lower) == 0) run[e] += __popcll(peers);
    __builtin_amdgcn_wave_barrier();
  }
}

// The whole sort in one block.  lds: (W + 1) * E ints.  The block's threads
// must all call it.  offsets[E+1] is the exclusive prefix of the histogram.
template <class Get>
__device__ void block_sort(Get get, int n, int E, int nbits, int *lds, int32_t *offsets,
                           int32_t *sorted) {
  const int W = blockDim.x >> 6;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  int *cnt = lds;           // [W][E]: per-wavefront counts, then bases
  int *base = lds + W * E;  // [E]
  for (int i = tid; i < W * E; i += blockDim.x) cnt[i] = 0;
  __syncthreads();
  int start, end;
  sort_range(n, W, wv, start, end);
  sort_count(get, start, end, E, nbits, cnt + wv * E);
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
  for (int e = tid; e < W * E; e += blockDim.x) cnt[e] += base[e % E];
  __syncthreads();
  sort_scatter(get, start, end, E, nbits, cnt + wv * E, sorted);
}

}  // namespace nvm
