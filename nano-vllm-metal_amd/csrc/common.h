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
  // Two copies of fp16(1024.0): the fp16 ulp at 1024 is 1, so 1024 + q is exact.
  static constexpr uint32_t kMagic2 = 0x64006400u;
  static constexpr float kMagic = 1024.0f;
  static constexpr uint32_t kOne2 = 0x3C003C00u;
  static constexpr int kPrec = 11;
  static constexpr int kEmin = -14;

  __device__ static __forceinline__ float to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
  }
  __device__ static __forceinline__ float lo(uint32_t d) { return to_f32(d & 0xFFFFu); }
  __device__ static __forceinline__ float hi(uint32_t d) { return to_f32(d >> 16); }
  __device__ static __forceinline__ uint16_t from_f32(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);
  }
  __device__ static __forceinline__ uint32_t pack2(float a, float b) {
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
// where M is the dtype's magic constant (128 for bf16, 1024 for fp16).
template <int DT>
__device__ __forceinline__ u32x4 nibble_pairs(uint32_t w) {
  constexpr uint32_t m = Act<DT>::kMagic2;
  u32x4 o;
  o.x = (w & 0x000F000Fu) | m;
  o.y = ((w >> 4) & 0x000F000Fu) | m;
  o.z = ((w >> 8) & 0x000F000Fu) | m;
  o.w = ((w >> 12) & 0x000F000Fu) | m;
  return o;
}

__device__ __forceinline__ u32x4 ldg16(const void *p) { return *(const u32x4 *)p; }
__device__ __forceinline__ u32x2 ldg8(const void *p) { return *(const u32x2 *)p; }

}  // namespace nvm
