// Decode-regime grouped W4A16 expert products (few routed rows per expert).
//
// Replaces `mx.gather_qmm` inside grouped_expert_linear (layers/moe.py:21-32)
// for decode-sized batches, fused with SwiGLU (layers/moe.py:84,
// layers/activation.py:21-24) for the gate/up pair.
//
// Weight bytes dominate, so each expert's rows are streamed from HBM once and
// applied to every row routed to that expert (up to 16 per pass).  The inner
// product runs on the matrix cores without rounding the weights: a 4-bit code
// q becomes the exact 16-bit float M+q (M = 128 for bf16, 1024 for fp16) by
// OR-ing it into a constant, v_mfma_f32_16x16x32 accumulates x.(M+q) over one
// 64-wide quantisation group, and the group is folded in float32 as
//   sum_i x_i w_i = s * sum_i x_i (M + q_i) + (b - M s) * sum_i x_i,
// which is the reference's w = q*s + b (metal/src/quantized_matmul.cpp:135).
//
// MFMA roles (16x16x32): A = activations [16 rows x 32 k], B = weights
// [32 k x 16 output features], C[row][feature].  Lane l supplies A row l%16
// and B column l%16 for k-slots 8*(l/16)..+7, and holds C rows 4*(l/16)..+3
// of column l%16.  Within a 64-element group, lane group G = l/16 takes packed
// words 2G (first MFMA) and 2G+1 (second MFMA): 8 bytes per lane per row,
// 32 contiguous bytes per row across the four lane groups.
#include "common.h"
#include "internal.h"

namespace nvm {

namespace {

template <int DT, bool DUAL, int NT>
__global__ __launch_bounds__(256) void gemv_kernel(const GroupedArgs a) {
  using A = Act<DT>;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int e = blockIdx.y;
  const int r0 = (blockIdx.x * (blockDim.x >> 6) + wv) * (16 * NT);
  if (r0 >= a.R) return;
  const int nb = a.offsets[e], ne = a.offsets[e + 1];
  if (nb >= ne) return;

  const int col = lane & 15, G = lane >> 4;
  const int KW = a.K >> 3, KG = a.K >> 6, GPR = a.K / a.gs;
  const int gsh = a.gs == 128 ? 1 : 0;  // 64-groups per scale group: 1 or 2

  const uint32_t *wp0[NT], *wp1[NT];
  const uint16_t *sp0[NT], *bp0[NT], *sp1[NT], *bp1[NT];
  bool tv[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    tv[t] = r0 + 16 * t < a.R;
    const int64_t row = (int64_t)e * a.R + (tv[t] ? r0 + 16 * t + col : 0);
    wp0[t] = a.w0 + row * KW + 2 * G;
    sp0[t] = a.s0 + row * GPR;
    bp0[t] = a.b0 + row * GPR;
    if (DUAL) {
      wp1[t] = a.w1 + row * KW + 2 * G;
      sp1[t] = a.s1 + row * GPR;
      bp1[t] = a.b1 + row * GPR;
    }
  }

  for (int nc = nb; nc < ne; nc += 16) {
    const int cnt = min(16, ne - nc);
    const bool has = col < cnt;
    const int arow = has ? (a.a_map ? a.a_map[nc + col] / a.a_div : nc + col) : 0;
    const uint16_t *ap = a.act + (int64_t)arow * a.act_ld + 16 * G;

    f32x4 o0[NT], o1[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      o0[t] = f32x4{0.f, 0.f, 0.f, 0.f};
      o1[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    // register double buffer: loads for group g+1 are issued before the
    // matrix work of group g
    u32x4 xa = {0, 0, 0, 0}, xb = {0, 0, 0, 0};
    u32x2 q0[NT], q1[NT];
    uint16_t s0v[NT], b0v[NT], s1v[NT], b1v[NT];
    auto load = [&](int g, u32x4 &la, u32x4 &lb, u32x2 *lq0, u32x2 *lq1, uint16_t *ls0,
                    uint16_t *lb0, uint16_t *ls1, uint16_t *lb1) {
      if (has) {
        la = ldg16(ap + 64 * g);
        lb = ldg16(ap + 64 * g + 8);
      }
      const int sg = g >> gsh;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        if (!tv[t]) continue;
        lq0[t] = ldg8(wp0[t] + 8 * g);
        ls0[t] = sp0[t][sg];
        lb0[t] = bp0[t][sg];
        if (DUAL) {
          lq1[t] = ldg8(wp1[t] + 8 * g);
          ls1[t] = sp1[t][sg];
          lb1[t] = bp1[t][sg];
        }
      }
    };
    load(0, xa, xb, q0, q1, s0v, b0v, s1v, b1v);

    for (int g = 0; g < KG; ++g) {
      const u32x4 ca = xa, cb = xb;
      u32x2 cq0[NT], cq1[NT];
      uint16_t cs0[NT], cb0[NT], cs1[NT], cb1[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        cq0[t] = q0[t];
        cs0[t] = s0v[t];
        cb0[t] = b0v[t];
        if (DUAL) {
          cq1[t] = q1[t];
          cs1[t] = s1v[t];
          cb1[t] = b1v[t];
        }
      }
      if (g + 1 < KG) load(g + 1, xa, xb, q0, q1, s0v, b0v, s1v, b1v);

      const u32x4 A0 = pair_order(ca), A1 = pair_order(cb);
      // sum of this lane's 16 activations, then of the row's 64 (4 lane groups)
      float sx = 0.f;
      sx = A::dot2(ca.x, A::kOne2, sx);
      sx = A::dot2(ca.y, A::kOne2, sx);
      sx = A::dot2(ca.z, A::kOne2, sx);
      sx = A::dot2(ca.w, A::kOne2, sx);
      sx = A::dot2(cb.x, A::kOne2, sx);
      sx = A::dot2(cb.y, A::kOne2, sx);
      sx = A::dot2(cb.z, A::kOne2, sx);
      sx = A::dot2(cb.w, A::kOne2, sx);
      sx += __shfl_xor(sx, 16);
      sx += __shfl_xor(sx, 32);
      float sxv[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) sxv[v] = __shfl(sx, 4 * G + v);

#pragma unroll
      for (int t = 0; t < NT; ++t) {
        if (!tv[t]) continue;
        {
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
          acc = A::mfma16(A0, nibble_pairs<DT>(cq0[t].x), acc);
          acc = A::mfma16(A1, nibble_pairs<DT>(cq0[t].y), acc);
          const float s = A::to_f32(cs0[t]), b = A::to_f32(cb0[t]);
          const float bp = fmaf(-A::kMagic, s, b);
#pragma unroll
          for (int v = 0; v < 4; ++v) o0[t][v] = fmaf(s, acc[v], fmaf(bp, sxv[v], o0[t][v]));
        }
        if (DUAL) {
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
          acc = A::mfma16(A0, nibble_pairs<DT>(cq1[t].x), acc);
          acc = A::mfma16(A1, nibble_pairs<DT>(cq1[t].y), acc);
          const float s = A::to_f32(cs1[t]), b = A::to_f32(cb1[t]);
          const float bp = fmaf(-A::kMagic, s, b);
#pragma unroll
          for (int v = 0; v < 4; ++v) o1[t][v] = fmaf(s, acc[v], fmaf(bp, sxv[v], o1[t][v]));
        }
      }
    }

#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (!tv[t]) continue;
      const int rowc = r0 + 16 * t + col;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int tok = 4 * G + v;
        if (tok >= cnt) continue;
        const int n = nc + tok;
        const int64_t orow = a.o_map ? a.o_map[n] : n;
        uint16_t r;
        if (DUAL) {
          // reference rounding points: gate and up outputs are act tensors,
          // silu(gate) * up is rounded once more
          const float gv = round_act<DT>(o0[t][v]);
          const float uv = round_act<DT>(o1[t][v]);
          r = A::from_f32(gv / (1.0f + __expf(-gv)) * uv);
        } else {
          r = A::from_f32(o0[t][v]);
        }
        a.out[orow * a.out_ld + rowc] = r;
      }
    }
  }
}

template <int DT>
hipError_t launch_t(bool dual, const GroupedArgs &a, hipStream_t st) {
  constexpr int NT = 2, WAVES = 4;
  const int rows_per_block = 16 * NT * WAVES;
  dim3 grid((unsigned)((a.R + rows_per_block - 1) / rows_per_block), (unsigned)a.E);
  if (dual)
    hipLaunchKernelGGL((gemv_kernel<DT, true, NT>), grid, dim3(64 * WAVES), 0, st, a);
  else
    hipLaunchKernelGGL((gemv_kernel<DT, false, NT>), grid, dim3(64 * WAVES), 0, st, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gemv(int dtype, bool dual, const GroupedArgs &a, hipStream_t st) {
  return dtype == DT_BF16 ? launch_t<DT_BF16>(dual, a, st) : launch_t<DT_F16>(dual, a, st);
}

}  // namespace nvm
