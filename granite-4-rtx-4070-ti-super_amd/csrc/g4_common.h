// g4_common.h - launch plumbing shared by the kernel translation units.
#ifndef G4_COMMON_H
#define G4_COMMON_H

#include <hip/hip_runtime.h>

#include <climits>
#include <cstdint>
#include <cstdio>
#include <type_traits>

namespace g4 {

constexpr int kBlock = 256;            // threads per workgroup (4 waves)
constexpr int kMaxVerifyRows = 16;     // model_config.h:56
constexpr int kMaxHeadDim = 256;       // model_config.h:52
constexpr int kCUs = 256;              // MI355X compute units
constexpr int kPersistBlocks = kCUs * 8;  // grid cap for grid-stride kernels
// FP8 workspace layout (bytes):
//   [0, 4096)          f32 partial maxima of the two-launch form's amax pass
//                      (its grid is capped at kMaxPartials)
//   [4096, 12288)      u64 tagged slots of the single-launch form's grid
//                      maximum (one per workgroup, at most kMaxPartials)
//   [12288, 12544)     u32 generation word of those slots at +0, u32 sticky
//                      synchronisation-error word at +64 (set to 1 when a
//                      bounded wait of the single-launch form gave up; read
//                      and cleared by granite4_fp8_sync_status), u64 tagged
//                      grid maximum at +128 (+ padding)
//   [12544, ...)       f32 per row: the norm's 1 / rms from pass 1 to pass 2
// The slots, the generation word and the grid maximum must start zero-filled.
constexpr int kMaxPartials = 1024;
constexpr size_t kWorkSlotsOff = 4096;
constexpr size_t kWorkGenOff = kWorkSlotsOff + 8 * kMaxPartials;
constexpr size_t kWorkRowOff = kWorkGenOff + 256;
__host__ __device__ inline float* work_partials(void* w) { return static_cast<float*>(w); }
__host__ __device__ inline unsigned long long* work_slots(void* w) {
  return reinterpret_cast<unsigned long long*>(static_cast<char*>(w) + kWorkSlotsOff);
}
__host__ __device__ inline unsigned* work_gen(void* w) {
  return reinterpret_cast<unsigned*>(static_cast<char*>(w) + kWorkGenOff);
}
__host__ __device__ inline unsigned* work_err(void* w) {
  return reinterpret_cast<unsigned*>(static_cast<char*>(w) + kWorkGenOff + 64);
}
__host__ __device__ inline unsigned long long* work_result(void* w) {
  return reinterpret_cast<unsigned long long*>(static_cast<char*>(w) + kWorkGenOff + 128);
}
// Measurement builds (-DG4_TRACE_FP8, never the shipped library): the
// single-launch FP8 kernels store s_memrealtime (100 MHz) at fixed points,
// 8 slots per workgroup, into the workspace's per-row area
// (bench.py --only fp8_trace reads them back).
#ifdef G4_TRACE_FP8
// gs: the launch's GridSync (its generation word sits at kWorkGenOff).
#define G4_TRACE_MARK(gs, i)                                                               \
  if (threadIdx.x == 0)                                                                    \
  reinterpret_cast<unsigned long long*>(reinterpret_cast<char*>((gs).gen) - kWorkGenOff +  \
                                        kWorkRowOff)[blockIdx.x * 8 + (i)] =               \
      __builtin_amdgcn_s_memrealtime()
#else
#define G4_TRACE_MARK(gs, i)
#endif

__host__ __device__ inline float* work_row_r(void* w) {
  return reinterpret_cast<float*>(static_cast<char*>(w) + kWorkRowOff);
}

// The calling thread's launch stream (default: the per-thread stream, the
// reference's --default-stream per-thread build).
hipStream_t stream();

// Reports a failed launch (or a sticky device error) like the reference's
// G4_CUDA_CHECK: message on stderr, -1 to the caller.
int launch_status(const char* what);

// How many workgroups of `threads` threads of `kernel` the current device
// holds at once (occupancy per CU x CUs); 0 if the query fails. The
// single-launch FP8 forms launch at most this many, so that every workgroup
// is resident for the grid synchronisation. Cached per (device, kernel).
int resident_blocks(const void* kernel, int threads);

// Process-wide FP8 launch mode (granite4_set_fp8_launch_mode): 0 = single
// launch where the tensor fits, 1 = always two launches, 2 = single launch
// through hipLaunchCooperativeKernel.
int fp8_launch_mode();

// Launches a kernel that synchronises its grid (the single-launch FP8
// forms): a plain launch, or in FP8 launch mode 2 a cooperative launch, for
// which the runtime checks that every workgroup can be resident at once.
template <class K, class... A>
void launch_grid_sync(K kern, unsigned grid, unsigned block, hipStream_t st, A... args) {
  if (fp8_launch_mode() == 2) {
    void* p[] = {static_cast<void*>(&args)...};
    (void)hipLaunchCooperativeKernel(reinterpret_cast<const void*>(kern), dim3(grid), dim3(block),
                                     p, 0, st);
    return;
  }
  hipLaunchKernelGGL(kern, grid, block, 0, st, args...);
}

// The current device's static FP8 scratch (granite4_add_rmsnorm_fp8_noalloc):
// its device address, set up on first use; nullptr on failure.
void* static_scratch(const char* what);

// Process-wide poll limit of the single-launch forms' bounded waits
// (granite4_debug_set_sync_spin_limit; default kSyncSpinLimit). 0 makes every
// wait give up at once: a host-forced failure for testing the error path.
int fp8_sync_spin_limit();

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
// Non-temporal (streaming) forms for operands read or written once: measured
// on MI355X they lift a pure read stream from ~6.0 to ~6.9 TB/s and a copy
// from ~5.6 to ~6.1 TB/s (the probe in probe.hip).
typedef unsigned g4_u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ V8 ld8_nt(const uint16_t* p) {
  const g4_u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const g4_u32x4*>(p));
  return V8{{v.x, v.y, v.z, v.w}};
}
__device__ __forceinline__ void st8_nt(uint16_t* p, const V8& v) {
  const g4_u32x4 w = {v.w[0], v.w[1], v.w[2], v.w[3]};
  __builtin_nontemporal_store(w, reinterpret_cast<g4_u32x4*>(p));
}
template <bool NT>
__device__ __forceinline__ V8 ld8_t(const uint16_t* p) {
  return NT ? ld8_nt(p) : ld8(p);
}
typedef unsigned g4_u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void st_u32x2_nt(void* p, uint32_t a, uint32_t b) {
  const g4_u32x2 w = {a, b};
  __builtin_nontemporal_store(w, reinterpret_cast<g4_u32x2*>(p));
}
__device__ __forceinline__ float4 ld_f4_nt(const float* p) {
  typedef float f4 __attribute__((ext_vector_type(4)));
  const f4 v = __builtin_nontemporal_load(reinterpret_cast<const f4*>(p));
  return make_float4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float v8_get(const V8& v, int e) {
  return (e & 1) ? __builtin_bit_cast(float, v.w[e >> 1] & 0xffff0000u)
                 : __builtin_bit_cast(float, v.w[e >> 1] << 16);
}

// Maximum of n per-workgroup partials (pass 2 of the FP8 ops), returned to
// every thread of the workgroup. Plain loads: the partials were written by
// the previous launch on the same stream.
__device__ __forceinline__ float reduce_partials(const float* part, int n) {
  __shared__ float s_red[4];
  float m = 0.0f;
  for (int i = threadIdx.x; i < n; i += 256) m = fmaxf(m, part[i]);
  m = fmaxf(m, __shfl_xor(m, 1));
  m = fmaxf(m, __shfl_xor(m, 2));
  m = fmaxf(m, __shfl_xor(m, 4));
  m = fmaxf(m, __shfl_xor(m, 8));
  m = fmaxf(m, __shfl_xor(m, 16));
  m = fmaxf(m, __shfl_xor(m, 32));
  if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = m;
  __syncthreads();
  m = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
  __syncthreads();
  return m;
}

// Workgroup maximum written to part[blockIdx.x] (pass 1 of the FP8 ops).
__device__ __forceinline__ void write_partial(float* part, float m) {
  __shared__ float s_red[4];
  m = fmaxf(m, __shfl_xor(m, 1));
  m = fmaxf(m, __shfl_xor(m, 2));
  m = fmaxf(m, __shfl_xor(m, 4));
  m = fmaxf(m, __shfl_xor(m, 8));
  m = fmaxf(m, __shfl_xor(m, 16));
  m = fmaxf(m, __shfl_xor(m, 32));
  if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) part[blockIdx.x] = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
}

// q = n / d for n < 2^31 via a double reciprocal and one correction step.
__device__ __forceinline__ int div_fast(int n, int d, double inv_d) {
  int q = static_cast<int>(static_cast<double>(n) * inv_d);
  const int r = n - q * d;
  q += (r >= d) - (r < 0);
  return q;
}

// Grid-stride sweep over items [0, total), U items per lane per step (a
// grid stride apart), all of a step's loads issued before any is used.
// sweep_begin issues the first step's loads, so a kernel can start them
// before other work with a long latency (the FP8 encode passes reduce the
// amax partials meanwhile); sweep_run processes that step and the rest.
// load(i) returns item i's raw registers; body(i, raw) computes and stores.
// Loads are unconditional: indices past the end are clamped to total - 1 (a
// re-read of one cached vector) and body runs only for indices < total.
// Requires total >= 1.
template <int U, class Raw>
struct Sweep {
  int v0, total, step;
  Raw x[U];
};

template <int U, class Load>
__device__ __forceinline__ auto sweep_begin(int total, Load load) {
  Sweep<U, decltype(load(0))> s;
  s.v0 = blockIdx.x * kBlock + threadIdx.x;
  s.total = total;
  s.step = gridDim.x * kBlock;
#pragma unroll
  for (int k = 0; k < U; ++k) s.x[k] = load(min(s.v0 + k * s.step, total - 1));
  return s;
}

template <int U, class Raw, class Load, class Body>
__device__ __forceinline__ void sweep_run(Sweep<U, Raw>& s, Load load, Body body) {
  while (s.v0 < s.total) {
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int v = s.v0 + k * s.step;
      if (v >= s.total) break;
      body(v, s.x[k]);
    }
    s.v0 += U * s.step;
    if (s.v0 >= s.total) break;
#pragma unroll
    for (int k = 0; k < U; ++k) s.x[k] = load(min(s.v0 + k * s.step, s.total - 1));
  }
}

// FP8 encode of a stored bf16 [rows][I] tensor (I % 8 == 0) under the scale
// from n_partials per-workgroup maxima, as the SwiGLU op's second pass
// (swiglu.hip). False on a launch error.
bool launch_encode_bf16(const uint16_t* act, int rows, int I, const float* partials, int n_partials,
                        uint8_t* codes, float* scale_out);

}  // namespace g4

#endif  // G4_COMMON_H
