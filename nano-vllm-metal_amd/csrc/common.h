// Device-side helpers shared by the MoE kernels (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nvm {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

enum { DT_F16 = 0, DT_BF16 = 1 };

// Activation-dtype traits.  Activations, scales and biases travel as raw
// 16-bit patterns; arithmetic is float32 (products) or float64 (router).
template <int DT>
struct Act;

template <>
struct Act<DT_BF16> {
  // Two copies of bf16(128.0) in one dword.  OR-ing a 4-bit code into the low
  // mantissa bits gives the exact value 128 + q (the bf16 ulp at 128 is 1).
  static constexpr uint32_t kMagic2 = 0x43004300u;
  static constexpr float kMagic = 128.0f;
  static constexpr int kCodeShift = 0;  // mantissa bit of the code's lsb
  static constexpr uint32_t kOne2 = 0x3F803F80u;  // (1.0, 1.0)
  static constexpr int kPrec = 8;                 // significant bits
  static constexpr int kEmin = -126;              // exponent of the smallest normal

  __device__ static __forceinline__ float to_f32(uint32_t h) { return __uint_as_float(h << 16); }
  __device__ static __forceinline__ float lo(uint32_t d) { return __uint_as_float(d << 16); }
  __device__ static __forceinline__ float hi(uint32_t d) { return __uint_as_float(d & 0xFFFF0000u); }
  __device__ static __forceinline__ uint16_t from_f32(float f) {
    return __builtin_bit_cast(uint16_t, (__bf16)f);  // round to nearest even
  }
  __device__ static __forceinline__ uint32_t pack2(float a, float b) {
    bf16x2 v = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, v);
  }
  __device__ static __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a),
                                           __builtin_bit_cast(bf16x2, b), c, false);
  }
  __device__ static __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  __device__ static __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};

template <>
struct Act<DT_F16> {
  // Two copies of fp16(64.0) with the code in mantissa bits 4..7: the weight
  // of bit 4 at 64 is 1, so the value is 64 + q exactly.  (Bits 0..3 would
  // need M = 1024, and the M*s*sum(x) term that cancels afterwards would cost
  // sixteen times more float32 precision.)
  static constexpr uint32_t kMagic2 = 0x54005400u;
  static constexpr float kMagic = 64.0f;
  static constexpr int kCodeShift = 4;
  static constexpr uint32_t kOne2 = 0x3C003C00u;
  static constexpr int kPrec = 11;
  static constexpr int kEmin = -14;

  __device__ static __forceinline__ float to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
  }
  __device__ static __forceinline__ float lo(uint32_t d) { return to_f32(d & 0xFFFFu); }
  __device__ static __forceinline__ float hi(uint32_t d) { return to_f32(d >> 16); }
  // The float32 operand is kept as such (empty asm): left free, the compiler
  // fuses a preceding fma or multiply and this conversion into one
  // v_fma_mixlo_f16, which rounds the exact result straight to fp16 and
  // parts from the float32 value rounded to fp16 where that is an fp16 tie.
  __device__ static __forceinline__ uint16_t from_f32(float f) {
    asm volatile("" : "+v"(f));
    return __builtin_bit_cast(uint16_t, (_Float16)f);
  }
  __device__ static __forceinline__ uint32_t pack2(float a, float b) {
    asm volatile("" : "+v"(a), "+v"(b));
    f16x2 v = {(_Float16)a, (_Float16)b};
    return __builtin_bit_cast(uint32_t, v);
  }
  __device__ static __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c,
                                  false);
  }
  __device__ static __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  __device__ static __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};

// Round a float32 value to the activation dtype and back (one rounding).
template <int DT>
__device__ __forceinline__ float round_act(float f) {
  return Act<DT>::to_f32(Act<DT>::from_f32(f));
}

// silu of layers/activation.py:21-24 on an act value g, with the result of
// each of its ops rounded to the activation dtype, as the reference's act
// tensors are: e = exp(-|g|), d = 1 + e, s = 1 / d, sg = where(g < 0, 1 - s,
// s), g * sg.  1 + e, 1 - s and g * sg are exact in float32 before their
// rounding.  The reciprocal is v_rcp_f32 (1 ulp): 1 / d of an act value d in
// [1, 2] lies at least 2^-23 (fp16) or 2^-17 (bf16) from an act rounding tie
// unless it is exact, so its rounded value is the correctly rounded one.
template <int DT>
__device__ __forceinline__ float silu_act(float g) {
  const float e = round_act<DT>(__expf(-fabsf(g)));
  const float d = round_act<DT>(1.0f + e);
  const float s = round_act<DT>(__builtin_amdgcn_rcpf(d));
  const float sg = g < 0.0f ? round_act<DT>(1.0f - s) : s;
  return round_act<DT>(g * sg);
}

// Two values rounded to the activation dtype and back with one packed
// conversion (each rounds as round_act rounds it).
template <int DT>
__device__ __forceinline__ void round_act2(float &a, float &b) {
  const uint32_t p = Act<DT>::pack2(a, b);
  a = Act<DT>::lo(p);
  b = Act<DT>::hi(p);
}

// SwiGLU of two gate/up pairs of act values: the act pair
// (rnd(silu_act(g0) * u0), rnd(silu_act(g1) * u1)), packed as Act::pack2
// packs it.  Each rounding of silu_act, done for two values at once.
template <int DT>
__device__ __forceinline__ uint32_t swiglu_act2(float g0, float g1, float u0, float u1) {
  float e0 = __expf(-fabsf(g0)), e1 = __expf(-fabsf(g1));
  round_act2<DT>(e0, e1);
  float d0 = 1.0f + e0, d1 = 1.0f + e1;
  round_act2<DT>(d0, d1);
  float s0 = __builtin_amdgcn_rcpf(d0), s1 = __builtin_amdgcn_rcpf(d1);
  round_act2<DT>(s0, s1);
  float t0 = 1.0f - s0, t1 = 1.0f - s1;
  round_act2<DT>(t0, t1);
  float r0 = g0 * (g0 < 0.0f ? t0 : s0), r1 = g1 * (g1 < 0.0f ? t1 : s1);
  round_act2<DT>(r0, r1);
  return Act<DT>::pack2(r0 * u0, r1 * u1);
}

// Round a float64 value to a floating format with `prec` significant bits and
// smallest normal exponent `emin`, ties to even, directly from float64.  The
// scaling by a power of two and rint() are both exact, so this is the single
// correctly rounded result (no double rounding through float32).
__device__ __forceinline__ double round_f64_to(double v, int prec, int emin) {
  if (v == 0.0) return v;
  int e = ilogb(v);
  if (e < emin) e = emin;
  const int sh = (prec - 1) - e;
  return ldexp(rint(ldexp(v, sh)), -sh);
}

template <int DT>
__device__ __forceinline__ uint16_t act_from_f64(double v) {
  // the rounded value is representable in the act dtype, so the float
  // conversions below are exact
  return Act<DT>::from_f32((float)round_f64_to(v, Act<DT>::kPrec, Act<DT>::kEmin));
}

// v_perm_b32: bytes of {hi, lo} picked by the selector (0-3 from lo, 4-7 from hi).
__device__ __forceinline__ uint32_t perm_b32(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

// Reorder 8 consecutive 16-bit values x0..x7 (held as 4 dwords) into the pair
// order (x0,x4)(x1,x5)(x2,x6)(x3,x7) that nibble_pairs() produces for codes.
__device__ __forceinline__ u32x4 pair_order(u32x4 d) {
  u32x4 o;
  o.x = perm_b32(d.z, d.x, 0x05040100u);
  o.y = perm_b32(d.z, d.x, 0x07060302u);
  o.z = perm_b32(d.w, d.y, 0x05040100u);
  o.w = perm_b32(d.w, d.y, 0x07060302u);
  return o;
}

// Expand one packed word (codes q0..q7 at bits 4j) into four dwords of
// 16-bit floats (M+q0, M+q4)(M+q1, M+q5)(M+q2, M+q6)(M+q3, M+q7), exactly,
// where M is the dtype's magic constant and SH its code shift (bf16: M = 128,
// codes in mantissa bits 0..3; fp16: M = 64, bits 4..7).  With `mask` =
// 0x000F000F << SH in an SGPR and `magic` (two copies of M) in a VGPR, each
// dword is one v_and_or_b32 after at most one shift (three of the four):
// gfx9 VOP3 encodings take no literal and read at most one SGPR, so with both
// constants as literals the compiler would emit an AND and an OR.
template <int S>
__device__ __forceinline__ uint32_t shift_by(uint32_t w) {
  if constexpr (S >= 0)
    return w << S;
  else
    return w >> -S;
}
template <int SH>
__device__ __forceinline__ u32x4 nibble_pairs_v(uint32_t w, uint32_t mask, uint32_t magic) {
  u32x4 o;
  o.x = (shift_by<SH>(w) & mask) | magic;
  o.y = (shift_by<SH - 4>(w) & mask) | magic;
  o.z = (shift_by<SH - 8>(w) & mask) | magic;
  o.w = (shift_by<SH - 12>(w) & mask) | magic;
  return o;
}
// The constants above as register values the compiler cannot fold back into
// literals (each is one move; only ordinary VALU/SALU code consumes them).
__device__ __forceinline__ uint32_t sgpr_const(uint32_t v) {
  uint32_t r;
  asm volatile("s_mov_b32 %0, %1" : "=s"(r) : "i"(v));
  return r;
}
__device__ __forceinline__ uint32_t vgpr_const(uint32_t v) {
  uint32_t r;
  asm volatile("v_mov_b32 %0, %1" : "=v"(r) : "i"(v));
  return r;
}

// Kernel arguments are read from the kernarg segment by scalar loads that the
// compiler places at their first use, often inside branches and each behind its
// own wait.  Naming them all in one empty asm statement at kernel entry issues
// the loads together: one memory round trip instead of one per use.
template <class T>
__device__ __forceinline__ void hoist_arg(const T &v) {
  asm volatile("" ::"s"(v));
}
template <class... T>
__device__ __forceinline__ void hoist_args(const T &...v) {
  (hoist_arg(v), ...);
}

__device__ __forceinline__ u32x4 ldg16(const void *p) { return *(const u32x4 *)p; }

// The down outputs of pairs t k + j0 .. t k + j0 + NB - 1 (those below k) at
// columns 8c .. 8c + 7, as float32 values of the act dtype: from the act
// tensor down [pairs][H], or (SPLIT) from the float32 sums of the two halves
// of the down reduction, part [2][TK][H], as rnd(lo + hi) (the down
// product's own output rounding).  Pairs past k read as zero.
template <int DT, bool SPLIT, int NB>
__device__ __forceinline__ void down_vals(const void *down, int64_t TK, int64_t t, int k, int j0,
                                          int64_t H, int64_t c, float (&dv)[NB][8]) {
  using A = Act<DT>;
  if constexpr (SPLIT) {
    const float *part = (const float *)down;
    u32x4 lo[NB][2], hi[NB][2];
#pragma unroll
    for (int jj = 0; jj < NB; ++jj) {
      const u32x4 z = {0u, 0u, 0u, 0u};
      lo[jj][0] = lo[jj][1] = hi[jj][0] = hi[jj][1] = z;
      if (j0 + jj < k) {  // uniform
        const int64_t p = t * k + j0 + jj;
        lo[jj][0] = ldg16(part + p * H + 8 * c);
        lo[jj][1] = ldg16(part + p * H + 8 * c + 4);
        hi[jj][0] = ldg16(part + (TK + p) * H + 8 * c);
        hi[jj][1] = ldg16(part + (TK + p) * H + 8 * c + 4);
      }
    }
#pragma unroll
    for (int jj = 0; jj < NB; ++jj)
#pragma unroll
      for (int i = 0; i < 8; ++i)
        dv[jj][i] = round_act<DT>(__uint_as_float(lo[jj][i >> 2][i & 3]) +
                                  __uint_as_float(hi[jj][i >> 2][i & 3]));
  } else {
    const uint16_t *dn = (const uint16_t *)down;
    u32x4 v[NB];
#pragma unroll
    for (int jj = 0; jj < NB; ++jj) {
      v[jj] = u32x4{0u, 0u, 0u, 0u};
      if (j0 + jj < k) v[jj] = ldg16(dn + ((t * k + j0 + jj) * H + 8 * c));  // uniform
    }
#pragma unroll
    for (int jj = 0; jj < NB; ++jj)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        dv[jj][2 * i] = A::lo(v[jj][i]);
        dv[jj][2 * i + 1] = A::hi(v[jj][i]);
      }
  }
}
__device__ __forceinline__ u32x2 ldg8(const void *p) { return *(const u32x2 *)p; }

// Raw buffer loads: a uniform descriptor (base, size in bytes) plus a 32-bit
// per-lane byte offset and a uniform offset.  Reads at or beyond `bytes`
// return zero, which the kernels use to mask lanes without branches.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr uint32_t kBufferFlags = 0x00020000u;  // raw 32-bit data format (gfx9 family)
constexpr int kMaskedOffset = 0x7FFFFFF0;      // beyond every descriptor the kernels build

__device__ __forceinline__ rsrc_t make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes,
                                           (int)kBufferFlags);
}
__device__ __forceinline__ u32x4 bload16(rsrc_t r, int voff, int soff) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}
__device__ __forceinline__ u32x2 bload8(rsrc_t r, int voff, int soff) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0));
}
__device__ __forceinline__ uint32_t bload4(rsrc_t r, int voff, int soff) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
}
__device__ __forceinline__ uint32_t bload2(rsrc_t r, int voff, int soff) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, 0);
}

// fp16 copies of bf16 activations (the prefill GEMMs' operands) keep bf16's
// range through a power-of-two shift per row and 64-value group: a group
// whose largest |x| is 2^15 or more is stored as x * 2^-s, s = e - 14 for
// that largest value's exponent e (so every stored value is below 2^15 and
// exact: bf16 has fewer significand bits than fp16), every other group as it
// is (s = 0).  The GEMMs undo the shift on their float32 sums.
//
// Largest |x| of eight bf16 values (four dwords), as a bf16 bit pattern.
__device__ __forceinline__ uint32_t bf16_absmax_bits(u32x4 v) {
  typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));
  auto a = [](uint32_t d) { return __builtin_bit_cast(u16x2, d & 0x7FFF7FFFu); };
  const u16x2 m = __builtin_elementwise_max(__builtin_elementwise_max(a(v.x), a(v.y)),
                                            __builtin_elementwise_max(a(v.z), a(v.w)));
  return max((uint32_t)m.x, (uint32_t)m.y);
}
// The shift of a group from its largest |x| (bf16 bits): exponent field - 141.
__device__ __forceinline__ int f16_shift_of(uint32_t absmax_bits) {
  return max(0, (int)(absmax_bits >> 7) - 141);
}
// 2^d as a float32, for |d| <= 126.
__device__ __forceinline__ float pow2f(int d) { return __uint_as_float((uint32_t)(127 + d) << 23); }
// Eight bf16 values -> fp16 of x * 2^-sh (exact for the group's values within
// 2^-29 of its largest; smaller ones round toward zero), in the pair order
// (x0,x4)(x1,x5)(x2,x6)(x3,x7).  v_cvt_pkrtz_f16_f32 rounds toward zero.
__device__ __forceinline__ u32x4 bf16_to_f16_pairs(u32x4 v, int sh) {
  const float f = pow2f(-sh);
  auto el = [&](int i) {
    return __uint_as_float((i & 1) ? (v[i >> 1] & 0xFFFF0000u) : (v[i >> 1] << 16)) * f;
  };
  u32x4 o;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    o[j] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(el(j), el(j + 4)));
  return o;
}
// Maximum over each aligned group of 8 lanes (quad swaps, then the half-row
// mirror), every lane of the group active.
__device__ __forceinline__ uint32_t max8_lanes(uint32_t v);

// Wavefront reductions: DPP butterflies inside each 16-lane row (quad_perm
// [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror), then the four
// row results combined from scalar readlanes.  The combination order is fixed,
// so the result is the same in every lane and on every run.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint64_t lo = dpp_u32<CTRL>((uint32_t)u), hi = dpp_u32<CTRL>((uint32_t)(u >> 32));
  return __builtin_bit_cast(double, lo | (hi << 32));
}
__device__ __forceinline__ double readlane_f64(double v, int lane) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint64_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, lane);
  const uint64_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), lane);
  return __builtin_bit_cast(double, lo | (hi << 32));
}

__device__ __forceinline__ uint32_t max8_lanes(uint32_t v) {
  v = max(v, dpp_u32<0xB1>(v));
  v = max(v, dpp_u32<0x4E>(v));
  return max(v, dpp_u32<0x141>(v));
}

template <class Op>
__device__ __forceinline__ double wave_reduce_f64(double v, Op op) {
  v = op(v, dpp_f64<0xB1>(v));
  v = op(v, dpp_f64<0x4E>(v));
  v = op(v, dpp_f64<0x141>(v));
  v = op(v, dpp_f64<0x140>(v));
  return op(op(readlane_f64(v, 0), readlane_f64(v, 16)), op(readlane_f64(v, 32), readlane_f64(v, 48)));
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, dpp_u32<0xB1>(v));
  v = max(v, dpp_u32<0x4E>(v));
  v = max(v, dpp_u32<0x141>(v));
  v = max(v, dpp_u32<0x140>(v));
  const uint32_t a = max((uint32_t)__builtin_amdgcn_readlane((int)v, 0),
                         (uint32_t)__builtin_amdgcn_readlane((int)v, 16));
  const uint32_t b = max((uint32_t)__builtin_amdgcn_readlane((int)v, 32),
                         (uint32_t)__builtin_amdgcn_readlane((int)v, 48));
  return max(a, b);
}

}  // namespace nvm
