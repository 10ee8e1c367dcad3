// g4_wave.h - wave64 cross-lane reductions for gfx950.
//
// Reductions inside a 16-lane DPP row use four data-parallel-primitive moves
// (quad_perm xor 1, quad_perm xor 2, row_half_mirror, row_mirror); after them
// every lane of the row holds the row's result, with the same operand order in
// every lane, so floating-point sums are identical across the row. Combining
// the four rows of a wave reads lanes 0, 16, 32 and 48 (v_readlane), which
// leaves a wave-uniform value.
#ifndef G4_WAVE_H
#define G4_WAVE_H

#include <hip/hip_runtime.h>

#include <cstdint>

namespace g4 {

// DPP control words (GFX9 encoding).
constexpr int kDppQuadXor1 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;   // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // row_half_mirror: lane i <- 7 - i within 8
constexpr int kDppMirror = 0x140;      // row_mirror: lane i <- 15 - i within 16
constexpr int kDppRor8 = 0x128;        // row_ror:8: lane i <- (i + 8) mod 16 within 16

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, 0xF, 0xF, false));
}

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(float, dpp_u32<CTRL>(__builtin_bit_cast(uint32_t, v)));
}

template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
  const uint64_t b = __builtin_bit_cast(uint64_t, v);
  const uint64_t lo = dpp_u32<CTRL>(static_cast<uint32_t>(b));
  const uint64_t hi = dpp_u32<CTRL>(static_cast<uint32_t>(b >> 32));
  return __builtin_bit_cast(double, lo | (hi << 32));
}

// Max over aligned groups of LANES (4, 8 or 16) lanes; every lane of the group
// receives the result.
template <int LANES>
__device__ __forceinline__ float group_max(float v) {
  v = fmaxf(v, dpp_f32<kDppQuadXor1>(v));
  v = fmaxf(v, dpp_f32<kDppQuadXor2>(v));
  if (LANES >= 8) v = fmaxf(v, dpp_f32<kDppHalfMirror>(v));
  if (LANES >= 16) v = fmaxf(v, dpp_f32<kDppMirror>(v));
  return v;
}

__device__ __forceinline__ double row16_sum(double v) {
  v = v + dpp_f64<kDppQuadXor1>(v);
  v = v + dpp_f64<kDppQuadXor2>(v);
  v = v + dpp_f64<kDppHalfMirror>(v);
  v = v + dpp_f64<kDppMirror>(v);
  return v;
}

__device__ __forceinline__ double readlane_f64(double v, int lane) {
  const uint64_t b = __builtin_bit_cast(uint64_t, v);
  const uint64_t lo = static_cast<uint32_t>(
      __builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(b)), lane));
  const uint64_t hi = static_cast<uint32_t>(
      __builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(b >> 32)), lane));
  return __builtin_bit_cast(double, lo | (hi << 32));
}

__device__ __forceinline__ float readlane_f32(float v, int lane) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Wave-uniform sum / max over all 64 lanes (every lane must be active).
__device__ __forceinline__ double wave_sum(double v) {
  v = row16_sum(v);
  return (readlane_f64(v, 0) + readlane_f64(v, 16)) + (readlane_f64(v, 32) + readlane_f64(v, 48));
}

__device__ __forceinline__ float wave_max(float v) {
  v = group_max<16>(v);
  return fmaxf(fmaxf(readlane_f32(v, 0), readlane_f32(v, 16)),
               fmaxf(readlane_f32(v, 32), readlane_f32(v, 48)));
}

// Issue priority from progress: a wave that has done `done` of its `total`
// work items takes priority 3 (none done) down to 0 (the last quarter). The
// SIMD's arbiter picks the highest priority first and the oldest wave among
// equals, so without this the first-dispatched of the workgroups sharing a
// CU runs ahead and the last finishes late, leaving the CU's tail with too
// few waves to keep its loads in flight. done / total: the first active
// lane's values are used.
__device__ __forceinline__ void wave_priority_by_progress(int done, int total) {
  done = __builtin_amdgcn_readfirstlane(done);
  total = __builtin_amdgcn_readfirstlane(total);
  const int q = total > 0 ? (4 * done) / total : 4;
  if (q <= 0) __builtin_amdgcn_s_setprio(3);
  else if (q == 1) __builtin_amdgcn_s_setprio(2);
  else if (q == 2) __builtin_amdgcn_s_setprio(1);
  else __builtin_amdgcn_s_setprio(0);
}

}  // namespace g4

#endif  // G4_WAVE_H
