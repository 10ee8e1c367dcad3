// selftest.hip - on-device exhaustive checks of the hardware conversion paths
// against the library's exact software arithmetic (which the CPU tests sweep
// against the oracle). Mirrors the reference's own device probe entry points
// (granite4_fp8_decode_all, kernels_phase2.cu:844-859): a test harness calls
// them and reads back mismatch counts.
#include "g4_common.h"
#include "g4_hw.h"
#include "g4_math.h"
#include "granite4_layerops.h"

namespace g4 {
namespace {

// result[0] = mismatches, result[1] = first mismatching input bits.
__device__ void record(unsigned long long* result, uint32_t bits) {
  if (atomicAdd(&result[0], 1ull) == 0ull) result[1] = bits;
}

// Every f32 bit pattern except NaNs: v_cvt_pk_bf16_f32 vs the integer formula.
__global__ __launch_bounds__(kBlock) void bf16_selftest_kernel(unsigned long long* result) {
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kBlock;
  for (uint64_t u = static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x; u < (1ull << 32);
       u += stride) {
    const uint32_t bits = static_cast<uint32_t>(u);
    const float f = __builtin_bit_cast(float, bits);
    if (f != f) continue;
    const uint32_t hw = pack_bf16_hw(f, -f);
    const uint32_t sw = f32_to_bf16(f) | (f32_to_bf16(-f) << 16);
    if (hw != sw) record(result, bits);
  }
}

// Every non-negative f32 y with y / s <= 470, and its negation: the hardware
// pair encoder and the octet encoder (y and -y of four consecutive patterns
// per octet) vs the exact software encoder.
__global__ __launch_bounds__(kBlock) void fp8_selftest_kernel(float s, uint32_t limit,
                                                              unsigned long long* result) {
  const float inv = 1.0f / s;
  const Fp8Enc enc = fp8_enc_of(s);
  const uint32_t stride = gridDim.x * kBlock;
  for (uint32_t base = 4u * (blockIdx.x * kBlock + threadIdx.x); base < limit; base += 4u * stride) {
    float y[8];
    uint32_t sw[2] = {0u, 0u};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t bits = base + k < limit ? base + k : limit - 1u;
      y[2 * k] = __builtin_bit_cast(float, bits);
      y[2 * k + 1] = -y[2 * k];
      const uint32_t c = fp8_encode_fast(y[2 * k], s, inv);
      const uint32_t pair = c | ((c | 0x80u) << 8);
      sw[k >> 1] |= pair << (16 * (k & 1));
      if (fp8x2_encode(y[2 * k], y[2 * k + 1], s, inv) != pair) record(result, bits);
    }
    const uint2 hw = fp8x8_encode<true>(y, enc);
    if (hw.x != sw[0] || hw.y != sw[1]) record(result, base);
  }
}

}  // namespace
}  // namespace g4

using namespace g4;

extern "C" {

int granite4_selftest_bf16(unsigned long long* d_result) {
  if (d_result == nullptr) return -1;
  hipLaunchKernelGGL(bf16_selftest_kernel, kPersistBlocks * 4, kBlock, 0, stream(), d_result);
  return launch_status("granite4_selftest_bf16");
}

int granite4_selftest_fp8(float scale, unsigned long long* d_result) {
  if (d_result == nullptr || !fp8_fast_scale(scale)) return -1;
  const double top = 470.0 * static_cast<double>(scale);
  if (!(top < 3.0e38)) return -1;
  const uint32_t limit = __builtin_bit_cast(uint32_t, static_cast<float>(top)) + 1u;
  hipLaunchKernelGGL(fp8_selftest_kernel, kPersistBlocks * 4, kBlock, 0, stream(), scale, limit,
                     d_result);
  return launch_status("granite4_selftest_fp8");
}

}  // extern "C"
