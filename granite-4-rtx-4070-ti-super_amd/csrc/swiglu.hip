// swiglu.hip - SwiGLU activation for gfx950, bf16 or FP8 e4m3 output.
//
// act = bf16(g * (1 / (1 + exp(-g))) * u), g = gu[r][i], u = gu[r][I + i]
// (prefill_gemm.cu:1194-1203; the decode epilogue kernels_phase2.cu:643-651
// has the same operation order). exp is the hardware base-2 exponential on a
// pre-scaled argument and the reciprocal the hardware v_rcp_f32: both are
// within a few f32 ulp, so act is within one bf16 ulp of the reference's
// evaluation (the bar the parity tests hold it to).
//
// Streaming layout: one lane owns one 16-byte vector (8 values) of the gate
// half and the matching vector of the up half; a grid-stride loop over
// [rows][I / 8] vectors with two vectors in flight per lane. HBM-bound: 4 B
// read + 2 B (bf16) or 1 B (FP8) written per element.
//
// FP8 output uses the same two-launch scheme as the add+RMSNorm kernel
// (norm.hip): pass 1 writes one partial max |act| per workgroup (grid capped
// at kMaxPartials), pass 2 reduces the partials, recomputes act and writes
// the codes.
#include "g4_common.h"
#include "g4_hw.h"
#include "g4_math.h"
#include "g4_wave.h"
#include "granite4_layerops.h"

namespace g4 {
namespace {

enum : int { kOutBf16 = 0, kOutAmax = 1, kOutFp8 = 2 };

struct SwArgs {
  const void* gu;  // bf16 [rows][2I] (or f32 for the reference's prefill_silu_mul)
  int rows, I;
  uint16_t* act;     // bf16 output (kOutBf16) or optional copy (kOutAmax)
  uint8_t* codes;    // kOutFp8
  float* scale_out;  // kOutFp8
  float* partials;   // kOutAmax writes [gridDim.x]; kOutFp8 reads [n_partials]
  int n_partials;
  double inv_nv;     // 1 / (I / 8)
  const uint16_t* act_in;  // kOutFp8: encode this stored bf16 act instead of recomputing
};

__device__ __forceinline__ float silu_mul(float g, float u) {
  const float e = __expf(-g);
  const float sig = __builtin_amdgcn_rcpf(1.0f + e);
  return g * sig * u;
}

// Vector v (8 elements) of the [rows][I / 8] output: act offset 8 v, gate
// offset 8 v + r I (the row stride of gu is 2I), up offset one I further.
template <bool F32IN, bool NT>
__device__ __forceinline__ void load_gu(const SwArgs& a, int v, int nv, float* g, float* u,
                                        long long* out_off) {
  const int r = div_fast(v, nv, a.inv_nv);
  *out_off = 8LL * v;
  const long long gofs = 8LL * v + static_cast<long long>(r) * a.I;
  if (F32IN) {
    const float* p = static_cast<const float*>(a.gu) + gofs;
    const float4 g0 = ld_f4_nt(p);
    const float4 g1 = ld_f4_nt(p + 4);
    const float4 u0 = ld_f4_nt(p + a.I);
    const float4 u1 = ld_f4_nt(p + a.I + 4);
    g[0] = g0.x; g[1] = g0.y; g[2] = g0.z; g[3] = g0.w;
    g[4] = g1.x; g[5] = g1.y; g[6] = g1.z; g[7] = g1.w;
    u[0] = u0.x; u[1] = u0.y; u[2] = u0.z; u[3] = u0.w;
    u[4] = u1.x; u[5] = u1.y; u[6] = u1.z; u[7] = u1.w;
  } else {
    const uint16_t* p = static_cast<const uint16_t*>(a.gu) + gofs;
    const V8 gv = ld8_t<NT>(p);
    const V8 uv = ld8_t<NT>(p + a.I);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      g[e] = v8_get(gv, e);
      u[e] = v8_get(uv, e);
    }
  }
}

template <int MODE, bool F32IN>
__global__ __launch_bounds__(kBlock) void swiglu_kernel(SwArgs a) {
  const int nv = a.I >> 3;
  const int total = a.rows * nv;
  const int step = gridDim.x * kBlock;
  float s = 0.0f, inv = 0.0f;
  bool fast = false;
  if (MODE == kOutFp8) {
    s = fp8_scale_for(reduce_partials(a.partials, a.n_partials));
    fast = fp8_fast_scale(s);
    inv = fast ? 1.0f / s : 0.0f;
    if (blockIdx.x == 0 && threadIdx.x == 0) *a.scale_out = s;
  }
  float m = 0.0f;
  constexpr int U = 4;  // vectors (of gate and of up) in flight per lane
  for (int v0 = blockIdx.x * kBlock + threadIdx.x; v0 < total; v0 += U * step) {
    float g[U][8], u[U][8];
    long long off[U];
#pragma unroll
    for (int k = 0; k < U; ++k)
      if (v0 + k * step < total) load_gu<F32IN, true>(a, v0 + k * step, nv, g[k], u[k], &off[k]);
#pragma unroll
    for (int k = 0; k < U; ++k) {
      if (v0 + k * step >= total) break;
      uint32_t w[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        w[e] = pack_bf16_hw(silu_mul(g[k][2 * e], u[k][2 * e]),
                            silu_mul(g[k][2 * e + 1], u[k][2 * e + 1]));
      if (MODE == kOutBf16 || (MODE == kOutAmax && a.act != nullptr))
        st8_nt(a.act + off[k], V8{{w[0], w[1], w[2], w[3]}});
      if (MODE == kOutAmax) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          m = fmaxf(m, fmaxf(lo_bf16(w[e] & 0x7fff7fffu), hi_bf16(w[e] & 0x7fff7fffu)));
      }
      if (MODE == kOutFp8) {
        uint32_t c[2] = {0u, 0u};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t pair = fp8x2_encode_scaled(lo_bf16(w[e]), hi_bf16(w[e]), s, inv, fast);
          c[e >> 1] |= pair << (16 * (e & 1));
        }
        st_u32x2_nt(a.codes + off[k], c[0], c[1]);
      }
    }
  }
  if (MODE == kOutAmax) write_partial(a.partials, m);
}

// FP8 encode of a stored bf16 [rows][I] tensor under the per-tensor scale
// from the pass-1 partials (8 elements per lane per step, two steps in flight).
__global__ __launch_bounds__(kBlock) void encode_bf16_kernel(SwArgs a) {
  constexpr int U = 4;  // vectors in flight per lane
  const int total = a.rows * (a.I >> 3);
  const int step = gridDim.x * kBlock;
  const float s = fp8_scale_for(reduce_partials(a.partials, a.n_partials));
  const bool fast = fp8_fast_scale(s);
  const float inv = fast ? 1.0f / s : 0.0f;
  if (blockIdx.x == 0 && threadIdx.x == 0) *a.scale_out = s;
  for (int v0 = blockIdx.x * kBlock + threadIdx.x; v0 < total; v0 += U * step) {
    V8 x[U];
#pragma unroll
    for (int k = 0; k < U; ++k)
      if (v0 + k * step < total) x[k] = ld8_nt(a.act_in + 8LL * (v0 + k * step));
#pragma unroll
    for (int k = 0; k < U; ++k) {
      if (v0 + k * step >= total) break;
      uint32_t c[2] = {0u, 0u};
#pragma unroll
      for (int e = 0; e < 4; ++e)
        c[e >> 1] |= fp8x2_encode_scaled(lo_bf16(x[k].w[e]), hi_bf16(x[k].w[e]), s, inv, fast)
                     << (16 * (e & 1));
      st_u32x2_nt(a.codes + 8LL * (v0 + k * step), c[0], c[1]);
    }
  }
}

// Element-wise fallback for I not a multiple of 8 (bf16 / f32 in, bf16 out).
template <bool F32IN>
__global__ __launch_bounds__(kBlock) void swiglu_scalar_kernel(SwArgs a) {
  const long long total = static_cast<long long>(a.rows) * a.I;
  for (long long i = static_cast<long long>(blockIdx.x) * kBlock + threadIdx.x; i < total;
       i += static_cast<long long>(gridDim.x) * kBlock) {
    const long long r = i / a.I, c = i - r * a.I;
    float g, u;
    if (F32IN) {
      const float* p = static_cast<const float*>(a.gu) + r * 2 * a.I + c;
      g = p[0];
      u = p[a.I];
    } else {
      const uint16_t* p = static_cast<const uint16_t*>(a.gu) + r * 2 * a.I + c;
      g = bf16_to_f32(p[0]);
      u = bf16_to_f32(p[a.I]);
    }
    a.act[i] = static_cast<uint16_t>(f32_to_bf16(silu_mul(g, u)));
  }
}

unsigned grid_for(long long vectors, int cap) {
  const long long want = (vectors + 4LL * kBlock - 1) / (4LL * kBlock);
  return static_cast<unsigned>(want < cap ? (want > 0 ? want : 1) : cap);
}

// Vector indices are 32-bit: rows * I / 8 plus one grid stride must fit.
bool sw_args_ok(const void* gu, int rows, int I) {
  return gu != nullptr && rows > 0 && I > 0 &&
         static_cast<long long>(rows) * (I / 8) + 4LL * kPersistBlocks * kBlock < INT_MAX &&
         static_cast<long long>(rows) * I < INT_MAX;
}

SwArgs sw_args(const void* gu, int rows, int I) {
  SwArgs a{};
  a.gu = gu;
  a.rows = rows;
  a.I = I;
  a.inv_nv = I >= 8 ? 1.0 / static_cast<double>(I / 8) : 0.0;
  return a;
}

}  // namespace
}  // namespace g4

using namespace g4;

extern "C" {

int granite4_swiglu(const uint16_t* d_gu, int rows, int I, uint16_t* d_act) {
  if (!sw_args_ok(d_gu, rows, I) || d_act == nullptr) {
    std::fprintf(stderr, "granite4: granite4_swiglu: invalid arguments\n");
    return -1;
  }
  SwArgs a = sw_args(d_gu, rows, I);
  a.act = d_act;
  if (I % 8 == 0)
    hipLaunchKernelGGL((swiglu_kernel<kOutBf16, false>),
                       grid_for(static_cast<long long>(rows) * (I / 8), kPersistBlocks), kBlock, 0,
                       stream(), a);
  else
    hipLaunchKernelGGL((swiglu_scalar_kernel<false>), kPersistBlocks, kBlock, 0, stream(), a);
  return launch_status("granite4_swiglu");
}

int granite4_prefill_silu_mul(const float* gu, int I, int rows, uint16_t* act) {
  if (!sw_args_ok(gu, rows, I) || act == nullptr) {
    std::fprintf(stderr, "granite4: granite4_prefill_silu_mul: invalid arguments\n");
    return -1;
  }
  SwArgs a = sw_args(gu, rows, I);
  a.act = act;
  if (I % 8 == 0)
    hipLaunchKernelGGL((swiglu_kernel<kOutBf16, true>),
                       grid_for(static_cast<long long>(rows) * (I / 8), kPersistBlocks), kBlock, 0,
                       stream(), a);
  else
    hipLaunchKernelGGL((swiglu_scalar_kernel<true>), kPersistBlocks, kBlock, 0, stream(), a);
  return launch_status("granite4_prefill_silu_mul");
}

int granite4_swiglu_fp8(const uint16_t* d_gu, int rows, int I, uint8_t* d_codes,
                        float* d_scale, void* d_work, uint16_t* d_act) {
  if (!sw_args_ok(d_gu, rows, I) || I % 8 != 0 || d_codes == nullptr || d_scale == nullptr ||
      d_work == nullptr) {
    std::fprintf(stderr, "granite4: granite4_swiglu_fp8: invalid arguments (I %% 8 == 0)\n");
    return -1;
  }
  const unsigned grid = grid_for(static_cast<long long>(rows) * (I / 8), kMaxPartials);
  SwArgs p1 = sw_args(d_gu, rows, I);
  p1.act = d_act;
  p1.partials = work_partials(d_work);
  hipLaunchKernelGGL((swiglu_kernel<kOutAmax, false>), grid, kBlock, 0, stream(), p1);
  if (launch_status("granite4_swiglu_fp8 (amax)") != 0) return -1;
  SwArgs p2 = sw_args(d_gu, rows, I);
  p2.codes = d_codes;
  p2.scale_out = d_scale;
  p2.partials = work_partials(d_work);
  p2.n_partials = static_cast<int>(grid);
  if (d_act != nullptr) {
    // Pass 1 stored the bf16 act: pass 2 only encodes it (2 B read instead
    // of re-reading 4 B of gate|up and re-evaluating the SiLU).
    p2.act_in = d_act;
    hipLaunchKernelGGL(encode_bf16_kernel, grid_for(static_cast<long long>(rows) * (I / 8), kPersistBlocks),
                       kBlock, 0, stream(), p2);
  } else {
    hipLaunchKernelGGL((swiglu_kernel<kOutFp8, false>), grid, kBlock, 0, stream(), p2);
  }
  return launch_status("granite4_swiglu_fp8 (encode)");
}

}  // extern "C"
