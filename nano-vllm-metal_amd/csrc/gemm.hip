// Prefill-regime grouped W4A16 expert products (many routed rows per expert).
//
// Replaces `mx.gather_qmm` inside grouped_expert_linear (layers/moe.py:21-32)
// for prefill-sized batches, with SwiGLU (layers/moe.py:84) fused into the
// gate/up epilogue.  Work is a list of (expert, 128-row m-tile) pairs built on
// the device from the expert offsets (prefix sum of ceil(count_e / 128)), so no
// host synchronisation is needed and empty experts cost nothing.
//
// Per 64-wide k-step a 256-thread block gathers 128 activation rows into LDS,
// dequantises 2 x 128 weight rows (w = q*s + b in float32, rounded to the
// activation dtype, as MLX's own GPU quantised matmul does) into LDS, and four
// wavefronts (2 x 2) each run 2 x 2 x 2 v_mfma_f32_32x32x16 per 16-wide k
// slice.  Rows are padded to 144 bytes so the 16-byte fragment reads of 32
// consecutive rows hit distinct LDS banks.
#include "common.h"
#include "internal.h"

namespace nvm {

namespace {

constexpr int BM = kGemmBM, BN = kGemmBN, BK = 64, PITCH = BK + 8;

template <int DT, bool DUAL>
__global__ __launch_bounds__(256) void gemm_kernel(const GroupedArgs a) {
  using A = Act<DT>;
  __shared__ __attribute__((aligned(16))) uint16_t As[BM * PITCH];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2 * BN * PITCH];
  __shared__ int s_arow[BM];
  __shared__ int s_tiles[kMaxExperts + 1];

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int mt = blockIdx.y;
  // m-tile list: exclusive prefix over experts of ceil(count / BM), built by
  // wavefront 0 from the expert offsets (E <= kMaxExperts)
  if (wv == 0) {
    int carry = 0;
    for (int c0 = 0; c0 < a.E; c0 += 64) {
      const int e = c0 + lane;
      const int tv = e < a.E ? (a.offsets[e + 1] - a.offsets[e] + BM - 1) / BM : 0;
      int inc = tv;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int u = __shfl_up(inc, o);
        if (lane >= o) inc += u;
      }
      if (e < a.E) s_tiles[e] = carry + inc - tv;
      carry += __shfl(inc, 63);
    }
    if (lane == 0) s_tiles[a.E] = carry;
  }
  __syncthreads();
  if (mt >= s_tiles[a.E]) return;
  // largest expert whose first tile is <= mt (skips experts with no tiles)
  int lo = 0, hi = a.E - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (s_tiles[mid] <= mt)
      lo = mid;
    else
      hi = mid - 1;
  }
  const int e = lo;
  const int m0 = a.offsets[e] + (mt - s_tiles[e]) * BM;
  const int mcnt = min(BM, a.offsets[e + 1] - m0);
  const int n0 = blockIdx.x * (DUAL ? BN : 2 * BN);
  const int n1 = DUAL ? n0 : n0 + BN;  // first row of the second weight tile
  const uint32_t *W1 = DUAL ? a.w1 : a.w0;
  const uint16_t *S1 = DUAL ? a.s1 : a.s0;
  const uint16_t *B1 = DUAL ? a.b1 : a.b0;
  const int KW = a.K >> 3, GPR = a.K / a.gs;

  for (int i = tid; i < BM; i += 256)
    s_arow[i] = i < mcnt ? (a.a_map ? a.a_map[m0 + i] / a.a_div : m0 + i) : -1;

  const int wm = wv & 1, wn = wv >> 1;
  const int l32 = lane & 31, kh = lane >> 5;
  f32x16 acc[2][2][2];
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[m][i][j][r] = 0.f;

  for (int k0 = 0; k0 < a.K; k0 += BK) {
    __syncthreads();
    // activations: 128 rows x 8 chunks of 16 bytes
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int idx = tid + 256 * c;
      const int row = idx >> 3, ch = idx & 7;
      const int ar = s_arow[row];
      u32x4 v = {0, 0, 0, 0};
      if (ar >= 0) v = ldg16(a.act + (int64_t)ar * a.act_ld + k0 + 8 * ch);
      *(u32x4 *)(As + row * PITCH + 8 * ch) = v;
    }
    // weights: 2 tiles x 128 rows x 2 halves of 32 codes
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int idx = tid + 256 * c;
      const int mat = idx >> 8, row = (idx >> 1) & 127, half = idx & 1;
      const int grow = (mat ? n1 : n0) + row;
      u32x4 o[4];
      if (grow < a.R) {
        const int64_t r = (int64_t)e * a.R + grow;
        const uint32_t *Wm = mat ? W1 : a.w0;
        const uint16_t *Sm = mat ? S1 : a.s0;
        const uint16_t *Bm = mat ? B1 : a.b0;
        const u32x4 q = ldg16(Wm + r * KW + (k0 >> 3) + 4 * half);
        const float s = A::to_f32(Sm[r * GPR + k0 / a.gs]);
        const float b = A::to_f32(Bm[r * GPR + k0 / a.gs]);
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const uint32_t qw = q[w];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float v0 = fmaf((float)((qw >> (8 * j)) & 0xFu), s, b);
            const float v1 = fmaf((float)((qw >> (8 * j + 4)) & 0xFu), s, b);
            o[w][j] = A::pack2(v0, v1);
          }
        }
      } else {
#pragma unroll
        for (int w = 0; w < 4; ++w) o[w] = u32x4{0, 0, 0, 0};
      }
      u32x4 *dst = (u32x4 *)(Bs + mat * BN * PITCH + row * PITCH + 32 * half);
#pragma unroll
      for (int w = 0; w < 4; ++w) dst[w] = o[w];
    }
    __syncthreads();

#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      u32x4 af[2], bf[2][2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        af[i] = *(const u32x4 *)(As + (64 * wm + 32 * i + l32) * PITCH + 16 * ks + 8 * kh);
#pragma unroll
      for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          bf[m][j] = *(const u32x4 *)(Bs + m * BN * PITCH + (64 * wn + 32 * j + l32) * PITCH +
                                      16 * ks + 8 * kh);
#pragma unroll
      for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j) acc[m][i][j] = A::mfma32(af[i], bf[m][j], acc[m][i][j]);
    }
  }

  // C fragment of v_mfma_f32_32x32x16: lane l, register 4*i+j holds
  // row 8*i + 4*(l/32) + j, column l%32
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int nn = 64 * wn + 32 * j + l32;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = 64 * wm + 32 * i + 8 * (r >> 2) + 4 * kh + (r & 3);
        if (m >= mcnt) continue;
        const int slot = m0 + m;
        const int64_t orow = a.o_map ? a.o_map[slot] : slot;
        uint16_t *op = a.out + orow * a.out_ld;
        if (DUAL) {
          if (n0 + nn < a.R) {
            const float gv = round_act<DT>(acc[0][i][j][r]);
            const float uv = round_act<DT>(acc[1][i][j][r]);
            op[n0 + nn] = A::from_f32(gv / (1.0f + __expf(-gv)) * uv);
          }
        } else {
          if (n0 + nn < a.R) op[n0 + nn] = A::from_f32(acc[0][i][j][r]);
          if (n1 + nn < a.R) op[n1 + nn] = A::from_f32(acc[1][i][j][r]);
        }
      }
    }
}

template <int DT>
hipError_t launch_t(bool dual, const GroupedArgs &a, int64_t max_m_tiles, hipStream_t st) {
  const int cols = dual ? BN : 2 * BN;
  dim3 grid((unsigned)((a.R + cols - 1) / cols), (unsigned)max_m_tiles);
  if (dual)
    hipLaunchKernelGGL((gemm_kernel<DT, true>), grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((gemm_kernel<DT, false>), grid, dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm(int dtype, bool dual, const GroupedArgs &a, int64_t max_m_tiles,
                       hipStream_t st) {
  return dtype == DT_BF16 ? launch_t<DT_BF16>(dual, a, max_m_tiles, st)
                          : launch_t<DT_F16>(dual, a, max_m_tiles, st);
}

}  // namespace nvm
