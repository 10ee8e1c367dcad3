// probe.hip - streaming bandwidth probes (the reference's kernels_bench.cu
// read / copy roofline measurement, kernels_bench.cu:36-53): the achievable
// HBM rate on this device, measured rather than assumed, and the known-size
// kernels that calibrate rocprof's FETCH_SIZE / WRITE_SIZE counters.
#include "g4_common.h"
#include "granite4_layerops.h"

namespace g4 {
namespace {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint4 ld_nt(const uint4* p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void st_nt(uint4* p, const uint4& v) {
  const u32x4 w = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(w, reinterpret_cast<u32x4*>(p));
}

// Each lane moves UNROLL 16-byte vectors per iteration, all loads first; NT
// selects non-temporal (streaming) loads and stores.
template <int UNROLL, bool NT>
__global__ __launch_bounds__(kBlock) void copy_kernel(const uint4* src, uint4* dst, long long n) {
  const long long step = static_cast<long long>(gridDim.x) * kBlock * UNROLL;
  for (long long i = static_cast<long long>(blockIdx.x) * kBlock * UNROLL + threadIdx.x; i < n;
       i += step) {
    uint4 v[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u)
      if (i + u * kBlock < n) v[u] = NT ? ld_nt(src + i + u * kBlock) : src[i + u * kBlock];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u)
      if (i + u * kBlock < n) {
        if (NT) st_nt(dst + i + u * kBlock, v[u]);
        else dst[i + u * kBlock] = v[u];
      }
  }
}

template <int UNROLL, bool NT>
__global__ __launch_bounds__(kBlock) void read_kernel(const uint4* src, long long n,
                                                      unsigned* sink) {
  const long long step = static_cast<long long>(gridDim.x) * kBlock * UNROLL;
  unsigned acc = 0;
  for (long long i = static_cast<long long>(blockIdx.x) * kBlock * UNROLL + threadIdx.x; i < n;
       i += step) {
    uint4 v[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u)
      v[u] = (i + u * kBlock < n) ? (NT ? ld_nt(src + i + u * kBlock) : src[i + u * kBlock])
                                  : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  if (acc == 0x9e3779b9u) sink[0] = acc;  // keeps the loads live; practically never stored
}

}  // namespace
}  // namespace g4

using namespace g4;

extern "C" {

int granite4_bw_probe(const void* src, void* dst, size_t bytes, int mode, int blocks) {
  if (src == nullptr || bytes < 16 || (bytes & 15) != 0 || (mode == 1 && dst == nullptr) ||
      blocks <= 0)
    return -1;
  const long long n = static_cast<long long>(bytes / 16);
  const uint4* s = static_cast<const uint4*>(src);
  const hipStream_t st = stream();
  switch (mode) {
    case 0: hipLaunchKernelGGL((read_kernel<4, false>), blocks, kBlock, 0, st, s, n, static_cast<unsigned*>(dst)); break;
    case 1: hipLaunchKernelGGL((copy_kernel<4, false>), blocks, kBlock, 0, st, s, static_cast<uint4*>(dst), n); break;
    case 2: hipLaunchKernelGGL((read_kernel<4, true>), blocks, kBlock, 0, st, s, n, static_cast<unsigned*>(dst)); break;
    case 3: hipLaunchKernelGGL((copy_kernel<4, true>), blocks, kBlock, 0, st, s, static_cast<uint4*>(dst), n); break;
    case 4: hipLaunchKernelGGL((copy_kernel<1, false>), blocks, kBlock, 0, st, s, static_cast<uint4*>(dst), n); break;
    case 5: hipLaunchKernelGGL((copy_kernel<8, true>), blocks, kBlock, 0, st, s, static_cast<uint4*>(dst), n); break;
    default: return -1;
  }
  return launch_status("granite4_bw_probe");
}

}  // extern "C"
