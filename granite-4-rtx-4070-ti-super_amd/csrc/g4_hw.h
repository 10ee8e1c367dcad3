// g4_hw.h - gfx950 hardware conversions used on the hot paths.
//
//   pack_bf16_hw   v_cvt_pk_bf16_f32: two f32 -> two bf16, round to nearest
//                  even. For every non-NaN input it equals the reference's
//                  integer formula (g4::f32_to_bf16); a NaN input gives a quiet
//                  NaN (the formula can map some NaN payloads elsewhere). The
//                  device self-test (selftest.hip) checks all 2^32 patterns.
//   fp8x2_encode   two correctly rounded e4m3 codes of y / s. The hardware
//                  converter (v_cvt_pk_fp8_f32, OCP e4m3, round to nearest
//                  even) runs on q = y * (1 / s) scaled by (1 - 2^-21) and by
//                  (1 + 2^-21): q is within 2^-22 (relative) of the exact
//                  quotient t, so [q (1 - 2^-21), q (1 + 2^-21)] holds t, and
//                  rounding is monotonic: when both ends give the same code,
//                  that is t's code. Otherwise (t within 2^-21 of a midpoint,
//                  about one element in 10^5), or for |q| >= 448, NaN and inf,
//                  the lane takes the exact software path fp8_encode_fast.
#ifndef G4_HW_H
#define G4_HW_H

#include <hip/hip_runtime.h>

#include <cstdint>

#include "g4_math.h"

namespace g4 {

typedef float hw_f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 hw_bf16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_bf16_hw(float lo, float hi) {
  const hw_f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, hw_bf16x2));
}

__device__ __forceinline__ uint32_t fp8x2_hw(float a, float b) {
  return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false)) & 0xffffu;
}

constexpr float kBracketLo = 1.0f - 0x1p-21f;
constexpr float kBracketHi = 1.0f + 0x1p-21f;

// Codes of y0 / s and y1 / s in bits [7:0] and [15:8]; requires
// fp8_fast_scale(s) and inv = 1 / s.
__device__ __forceinline__ uint32_t fp8x2_encode(float y0, float y1, float s, float inv) {
  const float q0 = y0 * inv, q1 = y1 * inv;
  const uint32_t lo = fp8x2_hw(q0 * kBracketLo, q1 * kBracketLo);
  const uint32_t hi = fp8x2_hw(q0 * kBracketHi, q1 * kBracketHi);
  const bool ok = (lo == hi) & (fabsf(q0) < 448.0f) & (fabsf(q1) < 448.0f);
  if (__builtin_expect(ok, 1)) return lo;
  return fp8_encode_fast(y0, s, inv) | (fp8_encode_fast(y1, s, inv) << 8);
}

// Scale-generic pair encode (see fp8_encode_scaled).
__device__ __forceinline__ uint32_t fp8x2_encode_scaled(float y0, float y1, float s, float inv,
                                                        bool fast) {
  if (fast) return fp8x2_encode(y0, y1, s, inv);
  return fp8_encode_scaled(y0, s, inv, false) | (fp8_encode_scaled(y1, s, inv, false) << 8);
}

}  // namespace g4

#endif  // G4_HW_H
