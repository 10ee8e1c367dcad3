// g4_math.h - scalar conversions shared by the gfx950 kernels and their
// host-side self-test entry points (the same inline code runs on both sides,
// so the CPU tests can sweep it exhaustively against the oracle).
//
//   bf16 <-> f32      round-to-nearest-even by the reference's integer formula
//                     (kernel_math.h:49-55, device_math.cuh:31-35).
//   fp8 e4m3 encode   the reference's weight quantiser applied to a scaled
//                     value: code = RNE_e4m3(double(y) / double(s)) with |v| >= 464
//                     saturating to +-448 and NaN -> 0x7F (fp8_convert.cc:47-122,
//                     gpu_pack.cc:48-51). The fast form below never divides:
//                     it brackets y/s between two grid points using y * (1/s)
//                     and decides the rounding direction from the exact sign of
//                     y - mid * s (one fused multiply-add), so the result is the
//                     correctly rounded code whenever 2^-100 <= s < inf.
//   KV quantisation   s = amax / qmax (IEEE division), code = clamp(round half away
//                     (x / s)) (kernel_math.h:71-173, device_math.cuh:105-210).
#ifndef G4_MATH_H
#define G4_MATH_H

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

namespace g4 {

__host__ __device__ __forceinline__ float bf16_to_f32(uint32_t bits16) {
  return __builtin_bit_cast(float, bits16 << 16);
}

__host__ __device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

// Low / high bf16 of a packed pair, as f32.
__host__ __device__ __forceinline__ float lo_bf16(uint32_t w) {
  return __builtin_bit_cast(float, w << 16);
}
__host__ __device__ __forceinline__ float hi_bf16(uint32_t w) {
  return __builtin_bit_cast(float, w & 0xffff0000u);
}
__host__ __device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  return f32_to_bf16(lo) | (f32_to_bf16(hi) << 16);
}

// ---------------------------------------------------------------------------
// FP8 e4m3.
// ---------------------------------------------------------------------------

// Correctly rounded e4m3 code of a double (the slow path for scales outside
// the fast range, and the host-side check of the fast path). Grid: k * 2^-9
// below 2^-6 (k = 8 is the first normal), k * 2^(e-3) for k = 8..16 in
// [2^e, 2^(e+1)). Power-of-two scalings are exact; rint() rounds ties to even.
__host__ __device__ inline uint32_t fp8_encode_f64(double t) {
  if (t != t) return 0x7Fu;
  const uint64_t tb = __builtin_bit_cast(uint64_t, t);
  const uint32_t sign = static_cast<uint32_t>(tb >> 56) & 0x80u;
  const double a = __builtin_bit_cast(double, tb & 0x7fffffffffffffffull);
  if (a >= 464.0) return sign | 0x7Eu;
  if (a < 0x1p-6) return sign | static_cast<uint32_t>(rint(a * 512.0));
  int e = static_cast<int>((tb >> 52) & 0x7ff) - 1023;  // a in [2^e, 2^(e+1))
  const double p = __builtin_bit_cast(double, static_cast<uint64_t>(3 - e + 1023) << 52);
  uint32_t k = static_cast<uint32_t>(rint(a * p));  // 8..16
  if (k == 16u) {
    k = 8u;
    ++e;
  }
  const uint32_t code = (static_cast<uint32_t>(e + 7) << 3) | (k - 8u);
  return sign | (code > 0x7Eu ? 0x7Eu : code);
}

// Fast correctly rounded code of y / s, for 2^-100 <= s < inf, inv = 1 / s.
//
// q = |y| * inv is within a few ulp of t = |y| / s, so the e4m3 interval
// [lo, hi] that holds q also decides t's rounding: t rounds up exactly when
// t > mid = (lo + hi) / 2, i.e. when |y| - mid * s > 0. fmaf evaluates that
// difference with one rounding, which keeps its sign (mid has at most 5
// significant bits and s >= 2^-100, so a non-zero difference is far above the
// f32 underflow threshold). A zero difference is an exact tie: even code wins.
// q >= 448 (or NaN / inf) are handled first: every t >= 432 rounds to 448.
__host__ __device__ __forceinline__ uint32_t fp8_encode_fast(float y, float s, float inv) {
  const uint32_t yb = __builtin_bit_cast(uint32_t, y);
  const uint32_t sign = (yb >> 24) & 0x80u;
  const float a = __builtin_bit_cast(float, yb & 0x7fffffffu);
  const float q = a * inv;
  if (!(q < 448.0f)) return (q != q) ? 0x7Fu : (sign | 0x7Eu);
  uint32_t lo;
  float mid;
  if (q < 0x1p-6f) {
    const float k = floorf(q * 512.0f);  // exact: power-of-two scaling
    lo = static_cast<uint32_t>(k);
    mid = (k + 0.5f) * 0x1p-9f;
  } else {
    const uint32_t qb = __builtin_bit_cast(uint32_t, q);
    lo = (((qb >> 23) - 120u) << 3) | ((qb >> 20) & 7u);
    mid = __builtin_bit_cast(float, (qb & 0xfff00000u) | 0x00080000u);
  }
  const float r = fmaf(-mid, s, a);
  const uint32_t up = (r > 0.0f) | ((r == 0.0f) & (lo & 1u));
  return sign | (lo + up);
}

// Scale-generic entry: s <= 0 gives code 0 (the reference's all-zero tensor
// case, gpu_pack.cc:299-302); tiny or non-finite scales take the f64 path.
__host__ __device__ __forceinline__ uint32_t fp8_encode_scaled(float y, float s, float inv,
                                                               bool fast) {
  if (fast) return fp8_encode_fast(y, s, inv);
  if (!(s > 0.0f)) return 0u;
  return fp8_encode_f64(static_cast<double>(y) / static_cast<double>(s));
}

__host__ __device__ __forceinline__ bool fp8_fast_scale(float s) {
  return s >= 0x1p-100f && s < 3.0e38f;
}

// scale = float(amax / 448) in double, as the reference's fp8_scale_for.
__host__ __device__ __forceinline__ float fp8_scale_for(float amax) {
  return static_cast<float>(static_cast<double>(amax) / 448.0);
}

// ---------------------------------------------------------------------------
// KV quantisation.
// ---------------------------------------------------------------------------

// Signed code clamp(round_half_away(x / s), -qmax, qmax); s == 0 -> 0.
__host__ __device__ __forceinline__ int kv_code(float x, float s, int qmax) {
  if (s == 0.0f) return 0;
  const float r = roundf(x / s);
  const float c = fminf(fmaxf(r, -static_cast<float>(qmax)), static_cast<float>(qmax));
  return static_cast<int>(c);
}

// True when kv_code_inv may take the reciprocal form for scale s: the
// reciprocal and every residual that can decide a code stay normal.
__host__ __device__ __forceinline__ bool kv_recip_ok(float s) {
  return s >= 0x1p-96f && s < 0x1p100f;
}

// kv_code with inv = 1.0f / s (correctly rounded) precomputed: the quotient
// q0 = x * inv is corrected once with its exact residual r = x - q0 * s
// (one fma), and RN(q0 + r * inv) is the correctly rounded x / s (Markstein,
// "Computation of elementary functions on the IBM RISC System/6000", 1990:
// a correctly rounded reciprocal and a faithful quotient suffice). So the
// code equals kv_code's bit for bit, with a few VALU operations instead of
// an IEEE division. Scales outside kv_recip_ok use the division.
__host__ __device__ __forceinline__ int kv_code_inv(float x, float s, float inv, int qmax) {
  if (!kv_recip_ok(s)) return kv_code(x, s, qmax);
  const float q0 = x * inv;
  // |q0| >= 256 saturates every code (qmax <= 127) and may be inf, whose
  // residual would be NaN: keep q0 there.
  const float q = fabsf(q0) < 256.0f ? fmaf(fmaf(-q0, s, x), inv, q0) : q0;
  const float c = fminf(fmaxf(roundf(q), -static_cast<float>(qmax)), static_cast<float>(qmax));
  return static_cast<int>(c);
}

}  // namespace g4

#endif  // G4_MATH_H
