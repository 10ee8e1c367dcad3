// g4_sync.h - one grid-wide maximum inside a launch, for the single-launch
// FP8 forms (the per-tensor scale needs the maximum over every workgroup's
// values before any code is written).
//
// Protocol: workgroups 1.. publish their maximum in their own 64-bit slot as
// (tag << 32 | f32 bits) with one relaxed, device-scope store. Workgroup 0
// polls every slot (device-scope relaxed loads, all of a thread's slots in
// flight together) until each holds the current tag, then stores the tagged
// grid maximum in one result word and the new generation; the other
// workgroups poll that one word from one thread. Grids of at most
// kSyncAllToAll workgroups skip the second hop: every workgroup publishes
// and polls every slot itself (one lane per slot). The tag is the workspace's
// generation word + 1, read at the start of the launch; workgroup 0 stores
// the new generation only once it has seen every slot, and each workgroup
// read the word before publishing. Tags are compared for equality, so the
// slots and the result word only need to start different from the first tag
// (a zero-filled workspace).
//
// Costs, measured on MI355X: ~2 us from the last workgroup's arrival to the
// maximum reaching every workgroup (two store -> poll hops). Polling every
// slot from every workgroup (grid^2 loads per round) took ~3 us: the polls
// crowded out the stores they waited for. A release store instead of the
// relaxed one (the value and the tag share one word, so no ordering is
// needed) cost ~12.8 us: at device scope it writes back the whole L2.
// Same-address atomic counters cost ~8 us.
//
// Requirements: every workgroup of the grid resident at once (the host checks
// the occupancy before choosing this form), kSyncThreads-thread workgroups,
// at most kSyncThreads * kSyncSlotsPerThread of them (GridSync::blocks), and one such launch at a time per
// workspace. The waits are bounded: a slot or result that never arrives
// (which those requirements exclude) ends the wait after gs.spin_limit
// polls (kSyncSpinLimit unless a test lowers it), the returned maximum is
// NaN, so the op reports a NaN scale rather than hang, and the workspace's
// sticky error word is set to 1 for the host to read
// (granite4_fp8_sync_status). A spin limit of 0 gives up before polling:
// workgroup 0 publishes a NaN maximum, so every workgroup of the launch
// deterministically ends with NaN and the error word set. After a give-up
// that is not forced this way, workgroups may disagree (one saw every slot,
// another gave up), so the whole call's codes and scale are invalid whenever
// the error word is set. Both forms advance the generation in every call,
// give-ups included, so the next call on the workspace starts clean without
// a clear.
#ifndef G4_SYNC_H
#define G4_SYNC_H

#include <hip/hip_runtime.h>

#include <cstdint>

namespace g4 {

constexpr int kSyncSpinLimit = 1 << 20;

struct GridSync {
  unsigned long long* slots;   // [blocks] tagged maxima
  unsigned* gen;               // generation word
  unsigned long long* result;  // tagged grid maximum (gathered by workgroup 0)
  int blocks;                  // the launch's grid size (gridDim.x), passed so
                               // the gather does not read the dispatch packet
  unsigned* err;               // sticky error word (1: a wait gave up)
  int spin_limit;              // polls before a wait gives up
};

// Workgroup size of every launch that synchronises (a constant, so no
// dispatch-packet load sits on the synchronisation path).
constexpr int kSyncThreads = 256;

constexpr int kSyncSlotsPerThread = 4;  // kMaxPartials / 256-thread workgroups

// Grids of at most this many workgroups synchronise in one hop (all-to-all
// polling by one wave each); larger ones in two (through workgroup 0).
// Measured at T = 8 (A/B on one box): add+RMSNorm->FP8 on 8 workgroups 5.80
// -> 5.14 us with one hop; SwiGLU->FP8 on 50 workgroups 5.32 -> 5.44 us (its
// 2500 polls per round cost more than the hop saves).
constexpr int kSyncAllToAll = 32;

// Issued at kernel start (thread 0; the value is used after the compute
// phase, so the load's latency is hidden).
// Every thread loads the word (one request per wave): a load in thread 0
// only would be waited for inside its branch, a round trip before wave 0's
// first data load.
__device__ __forceinline__ unsigned grid_sync_tag(const GridSync& gs) {
  return __hip_atomic_load(gs.gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
}

// Maximum of m over every thread of the grid (non-negative values; NaN
// inputs are ignored as fmaxf does). tag0: grid_sync_tag's value; thread
// 0's is the one used (it has arrived before thread 0 publishes, so the
// generation cannot have advanced past it). Every thread of the workgroup
// must call it; kSyncThreads * kSyncSlotsPerThread must cover gs.blocks.
//
// Two levels: workgroups 1.. publish their maximum in their slot; workgroup
// 0 polls every slot (each thread its <= kSyncSlotsPerThread slots, all
// loads in flight together), publishes the tagged grid maximum in the result
// word and the new generation; the others poll that one word from one
// thread. Polling traffic is ~2 grid loads per round instead of grid^2:
// measured, all-to-all polling kept ~3 us between the last arrival and the
// first workgroup seeing the maximum, the polls crowding out the store they
// wait for.
__device__ __forceinline__ float grid_max(float m, const GridSync& gs, unsigned tag0) {
  __shared__ float s_red[16];
  __shared__ unsigned s_tag;
  __shared__ float s_out;
  const int wave = threadIdx.x >> 6;
  constexpr int nw = kSyncThreads / 64;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
  if ((threadIdx.x & 63) == 0) s_red[wave] = m;
  if (threadIdx.x == 0) s_tag = tag0;
  __syncthreads();
  const unsigned tag = s_tag;
  if (gs.blocks <= kSyncAllToAll) {
    // Small grids: one hop. Every workgroup publishes its maximum, and wave
    // 0 polls every slot (one lane each, kSyncAllToAll loads per round)
    // until all carry the tag. Workgroup 0 advances the generation once it
    // has seen every slot (every workgroup read it before publishing).
    if (threadIdx.x == 0) {
      float bm = s_red[0];
      for (int i = 1; i < nw; ++i) bm = fmaxf(bm, s_red[i]);
      __hip_atomic_store(&gs.slots[blockIdx.x],
                         (static_cast<unsigned long long>(tag) << 32) | __float_as_uint(bm),
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (wave == 0) {
      const int lane = threadIdx.x;
      bool seen = lane >= gs.blocks;
      float v = 0.0f;
      int spin = 0;
      bool late = gs.spin_limit <= 0;
      while (!late) {
        if (!seen) {
          const unsigned long long w =
              __hip_atomic_load(&gs.slots[lane], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          if (static_cast<unsigned>(w >> 32) == tag) {
            seen = true;
            v = __uint_as_float(static_cast<unsigned>(w));
          }
        }
        if (__all(seen)) break;
        if (++spin >= gs.spin_limit) late = true;
      }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
      if (lane == 0) {
        // Workgroup 0 advances the generation also after a give-up, so the
        // next call's tag differs from every slot this call wrote.
        if (late) __hip_atomic_store(gs.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (blockIdx.x == 0)
          __hip_atomic_store(gs.gen, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_out = late ? __builtin_nanf("") : v;
      }
    }
    __syncthreads();
    return s_out;
  }
  if (blockIdx.x != 0) {
    if (threadIdx.x == 0) {
      float bm = s_red[0];
      for (int i = 1; i < nw; ++i) bm = fmaxf(bm, s_red[i]);
      __hip_atomic_store(&gs.slots[blockIdx.x],
                         (static_cast<unsigned long long>(tag) << 32) | __float_as_uint(bm),
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      unsigned long long v;
      int spin = 0;
      for (;;) {
        v = __hip_atomic_load(gs.result, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (static_cast<unsigned>(v >> 32) == tag || ++spin >= gs.spin_limit) break;
        __builtin_amdgcn_s_sleep(1);
      }
      const bool ok = static_cast<unsigned>(v >> 32) == tag;
      if (!ok) __hip_atomic_store(gs.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_out = ok ? __uint_as_float(static_cast<unsigned>(v)) : __builtin_nanf("");
    }
    __syncthreads();
    return s_out;
  }
  // Workgroup 0: gather.
  float mm = s_red[0];
  for (int i = 1; i < nw; ++i) mm = fmaxf(mm, s_red[i]);
  bool need[kSyncSlotsPerThread];
#pragma unroll
  for (int k = 0; k < kSyncSlotsPerThread; ++k) {
    const int j = threadIdx.x + k * kSyncThreads;
    need[k] = j > 0 && j < gs.blocks;
  }
  int spin = 0;
  bool late = gs.spin_limit <= 0;
  while (!late) {
    unsigned long long v[kSyncSlotsPerThread];
#pragma unroll
    for (int k = 0; k < kSyncSlotsPerThread; ++k)
      if (need[k])
        v[k] = __hip_atomic_load(&gs.slots[threadIdx.x + k * kSyncThreads], __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
    bool any = false;
#pragma unroll
    for (int k = 0; k < kSyncSlotsPerThread; ++k) {
      if (!need[k]) continue;
      if (static_cast<unsigned>(v[k] >> 32) == tag) {
        mm = fmaxf(mm, __uint_as_float(static_cast<unsigned>(v[k])));
        need[k] = false;
      } else {
        any = true;
      }
    }
    if (!any) break;
    if (++spin >= gs.spin_limit) late = true;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mm = fmaxf(mm, __shfl_xor(mm, o));
  __syncthreads();  // s_red is reused below
  if ((threadIdx.x & 63) == 0) s_red[wave] = late ? __builtin_nanf("") : mm;
  __syncthreads();
  if (threadIdx.x == 0) {
    float r = s_red[0];
    bool bad = r != r;
    for (int i = 1; i < nw; ++i) {
      bad |= s_red[i] != s_red[i];
      r = fmaxf(r, s_red[i]);
    }
    if (bad) {
      r = __builtin_nanf("");
      __hip_atomic_store(gs.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __hip_atomic_store(gs.result, (static_cast<unsigned long long>(tag) << 32) | __float_as_uint(r),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(gs.gen, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_out = r;
  }
  __syncthreads();
  return s_out;
}

}  // namespace g4

#endif  // G4_SYNC_H
