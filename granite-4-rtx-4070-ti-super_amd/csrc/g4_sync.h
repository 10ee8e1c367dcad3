// g4_sync.h - one grid-wide maximum inside a launch, for the single-launch
// FP8 forms (the per-tensor scale needs the maximum over every workgroup's
// values before any code is written).
//
// Protocol: each workgroup publishes its maximum in its own 64-bit slot as
// (tag << 32 | f32 bits) with one relaxed, device-scope store, then polls
// every slot (one lane per slot, device-scope relaxed loads) until each holds
// the current tag. The tag is the workspace's generation word + 1, read at
// the start of the launch; workgroup 0 stores the new generation once it has
// seen every slot, which no workgroup can precede: each read the word before
// publishing. Tags are compared for equality, so the slots only need to
// start different from the first tag (a zero-filled workspace).
//
// Costs, measured on MI355X: ~2.6 us per synchronisation with 256
// workgroups. A release store instead of the relaxed one (the value and the
// tag share one word, so no ordering is needed) cost ~12.8 us: at device
// scope it writes back the whole L2. Same-address atomic counters cost
// ~8 us.
//
// Requirements: every workgroup of the grid resident at once (the host checks
// the occupancy before choosing this form), and one such launch at a time per
// workspace. The wait is bounded: a slot that never arrives (which those
// requirements exclude) ends the wait after kSyncSpinLimit polls, and the
// returned maximum is NaN, so the op reports a NaN scale rather than hang.
#ifndef G4_SYNC_H
#define G4_SYNC_H

#include <hip/hip_runtime.h>

#include <cstdint>

namespace g4 {

constexpr int kSyncSpinLimit = 1 << 20;

struct GridSync {
  unsigned long long* slots;  // [gridDim.x] tagged maxima
  unsigned* gen;              // generation word
};

// Issued at kernel start (thread 0; the value is used after the compute
// phase, so the load's latency is hidden).
__device__ __forceinline__ unsigned grid_sync_tag(const GridSync& gs) {
  return threadIdx.x == 0 ? __hip_atomic_load(gs.gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u
                          : 0u;
}

// Maximum of m over every thread of the grid (non-negative values; NaN
// inputs are ignored as fmaxf does). tag0: grid_sync_tag's value (read in
// thread 0 only). Every thread of the workgroup must call it.
__device__ __forceinline__ float grid_max(float m, const GridSync& gs, unsigned tag0) {
  __shared__ float s_red[16];
  __shared__ unsigned s_tag;
  __shared__ unsigned s_bad;
  const int wave = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
  if ((threadIdx.x & 63) == 0) s_red[wave] = m;
  if (threadIdx.x == 0) {
    s_tag = tag0;
    s_bad = 0u;
  }
  __syncthreads();
  const unsigned tag = s_tag;
  if (threadIdx.x == 0) {
    float bm = s_red[0];
    for (int i = 1; i < nw; ++i) bm = fmaxf(bm, s_red[i]);
    __hip_atomic_store(&gs.slots[blockIdx.x],
                       (static_cast<unsigned long long>(tag) << 32) | __float_as_uint(bm),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  float mm = 0.0f;
  bool late = false;
  for (int j = threadIdx.x; j < static_cast<int>(gridDim.x); j += blockDim.x) {
    unsigned long long v;
    int spin = 0;
    do {
      v = __hip_atomic_load(&gs.slots[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } while (static_cast<unsigned>(v >> 32) != tag && ++spin < kSyncSpinLimit);
    if (static_cast<unsigned>(v >> 32) != tag) late = true;
    mm = fmaxf(mm, __uint_as_float(static_cast<unsigned>(v)));
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mm = fmaxf(mm, __shfl_xor(mm, o));
  __syncthreads();  // s_red is reused below
  if ((threadIdx.x & 63) == 0) s_red[wave] = mm;
  if (late) s_bad = 1u;
  __syncthreads();
  float r = s_red[0];
  for (int i = 1; i < nw; ++i) r = fmaxf(r, s_red[i]);
  if (s_bad != 0u) r = __builtin_nanf("");
  if (blockIdx.x == 0 && threadIdx.x == 0)
    __hip_atomic_store(gs.gen, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return r;
}

}  // namespace g4

#endif  // G4_SYNC_H
