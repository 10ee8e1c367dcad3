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

// Per-launch constants of the pair / octet encoders: the scale, half of it,
// its reciprocal, and the reciprocal pre-multiplied by the bracket ends. For
// a positive y, RN(y * RN(inv * (1 - 2^-21))) <= y / s <= RN(y * RN(inv * (1 + 2^-21)))
// (each rounding moves the product by at most 2^-24 relative, the bracket
// by 2^-21), so converting the two ends brackets the exact quotient exactly
// as the q * (1 -+ 2^-21) form of fp8x2_encode does.
struct Fp8Enc {
  float s, s_half, inv, inv_lo, inv_hi;
  bool fast;
};

__host__ __device__ __forceinline__ Fp8Enc fp8_enc_of(float s) {
  Fp8Enc e;
  e.s = s;
  e.s_half = 0.5f * s;
  e.fast = fp8_fast_scale(s);
  e.inv = e.fast ? 1.0f / s : 0.0f;
  e.inv_lo = e.inv * kBracketLo;
  e.inv_hi = e.inv * kBracketHi;
  return e;
}

// Four codes where the bracket ends lo and hi (4 codes each, no NaN code)
// may disagree. Where they do, the exact quotient lies between the two
// adjacent codes, whose midpoint m = (|v_lo| + |v_hi|) / 2 is exact in f32
// (two 4-bit significands one step apart), and the sign of the exact residual
// |y| - m s, one fused multiply-add of the exact sum against s / 2 (s >= 2^-100
// keeps every term far from underflow), picks the code: above the midpoint
// the larger magnitude (hi), below it lo, on it the even code (round to
// nearest even, the LSB of the 3-bit mantissa). Where they agree, v_lo = v_hi
// and the result is that code either way.
template <int B>
__device__ __forceinline__ uint32_t fp8_take_hi(uint32_t lo, uint32_t hi, float y, float s_half) {
  const float vl = __builtin_amdgcn_cvt_f32_fp8(static_cast<int>(lo), B);
  const float vh = __builtin_amdgcn_cvt_f32_fp8(static_cast<int>(hi), B);
  const float r = fmaf(-(fabsf(vl) + fabsf(vh)), s_half, fabsf(y));
  const bool up = (r > 0.0f) || (r == 0.0f && ((lo >> (8 * B)) & 1u) != 0u);
  return up ? (0xffu << (8 * B)) : 0u;
}

__device__ __forceinline__ uint32_t fp8x4_resolve(uint32_t lo, uint32_t hi, const float* y,
                                                  float s_half) {
  const uint32_t take_hi = fp8_take_hi<0>(lo, hi, y[0], s_half) | fp8_take_hi<1>(lo, hi, y[1], s_half) |
                           fp8_take_hi<2>(lo, hi, y[2], s_half) | fp8_take_hi<3>(lo, hi, y[3], s_half);
  return (hi & take_hi) | (lo & ~take_hi);
}

// Eight codes (byte e of the result = element e). FAST (fp8_fast_scale(s)):
// four hardware conversions per bracket end, each writing one 16-bit half of
// a code word. Both ends agreeing is the common case; a disagreement (the
// quotient on or within 2^-21 of a midpoint between two codes: frequent for
// scales such as 1 or 2^k / 7, where bf16 inputs land exactly on midpoints)
// is settled by fp8x4_resolve; a NaN code (|y / s| >= 464, NaN or inf input)
// sends the octet to the exact software path. !FAST: the f64 path. Callers
// branch once per launch on the uniform fast flag, so the hot loop carries no
// f64 code.
template <bool FAST>
__device__ __forceinline__ uint2 fp8x8_encode(const float (&y)[8], const Fp8Enc& e) {
  if (!FAST) {
    uint32_t c[2] = {0u, 0u};
#pragma unroll
    for (int i = 0; i < 8; ++i) c[i >> 2] |= fp8_encode_scaled(y[i], e.s, e.inv, false) << (8 * (i & 3));
    return make_uint2(c[0], c[1]);
  }
  uint32_t lo0 = __builtin_amdgcn_cvt_pk_fp8_f32(y[0] * e.inv_lo, y[1] * e.inv_lo, 0, false);
  lo0 = __builtin_amdgcn_cvt_pk_fp8_f32(y[2] * e.inv_lo, y[3] * e.inv_lo, lo0, true);
  uint32_t lo1 = __builtin_amdgcn_cvt_pk_fp8_f32(y[4] * e.inv_lo, y[5] * e.inv_lo, 0, false);
  lo1 = __builtin_amdgcn_cvt_pk_fp8_f32(y[6] * e.inv_lo, y[7] * e.inv_lo, lo1, true);
  uint32_t hi0 = __builtin_amdgcn_cvt_pk_fp8_f32(y[0] * e.inv_hi, y[1] * e.inv_hi, 0, false);
  hi0 = __builtin_amdgcn_cvt_pk_fp8_f32(y[2] * e.inv_hi, y[3] * e.inv_hi, hi0, true);
  uint32_t hi1 = __builtin_amdgcn_cvt_pk_fp8_f32(y[4] * e.inv_hi, y[5] * e.inv_hi, 0, false);
  hi1 = __builtin_amdgcn_cvt_pk_fp8_f32(y[6] * e.inv_hi, y[7] * e.inv_hi, hi1, true);
  // |y * inv_hi| >= |y * inv_lo|, so a NaN code at the lo end implies one at
  // the hi end: checking the hi words covers both.
  const uint32_t nan_bits =
      (((hi0 & 0x7f7f7f7fu) + 0x01010101u) | ((hi1 & 0x7f7f7f7fu) + 0x01010101u)) & 0x80808080u;
  if (__builtin_expect(nan_bits != 0u, 0)) {
    uint32_t c[2] = {0u, 0u};
#pragma unroll
    for (int i = 0; i < 8; ++i) c[i >> 2] |= fp8_encode_fast(y[i], e.s, e.inv) << (8 * (i & 3));
    return make_uint2(c[0], c[1]);
  }
  if (__builtin_expect(((lo0 ^ hi0) | (lo1 ^ hi1)) != 0u, 0)) {
    lo0 = fp8x4_resolve(lo0, hi0, y, e.s_half);
    lo1 = fp8x4_resolve(lo1, hi1, y + 4, e.s_half);
  }
  return make_uint2(lo0, lo1);
}

// The same for a 16-byte vector of bf16 values.
template <bool FAST>
__device__ __forceinline__ uint2 fp8x8_encode_bf16(const uint32_t (&w)[4], const Fp8Enc& e) {
  float y[8];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    y[2 * p] = __builtin_bit_cast(float, w[p] << 16);
    y[2 * p + 1] = __builtin_bit_cast(float, w[p] & 0xffff0000u);
  }
  return fp8x8_encode<FAST>(y, e);
}

// silu(g) * u in f32 (hardware exp and reciprocal): the SwiGLU activation
// of the SwiGLU ops and of the gate|up GEMM epilogue.
__device__ __forceinline__ float silu_mul(float g, float u) {
  const float e = __expf(-g);
  const float sig = __builtin_amdgcn_rcpf(1.0f + e);
  return g * sig * u;
}

}  // namespace g4

#endif  // G4_HW_H
