// g4_common.h - launch plumbing shared by the kernel translation units.
#ifndef G4_COMMON_H
#define G4_COMMON_H

#include <hip/hip_runtime.h>

#include <climits>
#include <cstdint>
#include <cstdio>

namespace g4 {

constexpr int kBlock = 256;            // threads per workgroup (4 waves)
constexpr int kMaxVerifyRows = 16;     // model_config.h:56
constexpr int kMaxHeadDim = 256;       // model_config.h:52
constexpr int kCUs = 256;              // MI355X compute units
constexpr int kPersistBlocks = kCUs * 8;  // grid cap for grid-stride kernels

// The calling thread's launch stream (default: the per-thread stream, the
// reference's --default-stream per-thread build).
hipStream_t stream();

// Reports a failed launch (or a sticky device error) like the reference's
// G4_CUDA_CHECK: message on stderr, -1 to the caller.
int launch_status(const char* what);

inline bool fits_int(long long v) { return v >= 0 && v <= INT_MAX; }

// 16-byte vector of 8 bf16 values.
struct alignas(16) V8 {
  uint32_t w[4];
};

__device__ __forceinline__ V8 ld8(const uint16_t* p) {
  const uint4 v = *reinterpret_cast<const uint4*>(p);
  return V8{{v.x, v.y, v.z, v.w}};
}
__device__ __forceinline__ void st8(uint16_t* p, const V8& v) {
  *reinterpret_cast<uint4*>(p) = make_uint4(v.w[0], v.w[1], v.w[2], v.w[3]);
}
__device__ __forceinline__ float v8_get(const V8& v, int e) {
  return (e & 1) ? __builtin_bit_cast(float, v.w[e >> 1] & 0xffff0000u)
                 : __builtin_bit_cast(float, v.w[e >> 1] << 16);
}

}  // namespace g4

#endif  // G4_COMMON_H
