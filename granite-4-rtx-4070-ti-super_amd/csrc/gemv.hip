// gemv.hip - batch-1 decode GEMVs (bf16 activation x fp8 weight rows) with
// the decode step's non-GEMM ops fused in: the RMSNorm of the residual as a
// prologue, the SwiGLU of gate/up and the residual add as epilogues.
//
// Arithmetic (the reference's decode GEMVs, gemv_row_dequant
// forward_gpu.cu:934-994, silu_gate_up_kernel kernels_phase2.cu:590-651):
// y[n] = scale * sum_k fp8(W[n][k]) * a[k] in f32 (this kernel's own sum
// order), then
//   bf16       out[n] = bf16(y)
//   residual   out[n] = bf16(residual[n] + resid_scale * y)   (in place)
//   swiglu     act[i] = bf16(g * (1 / (1 + exp(-g))) * u), g = sg * sum_gate,
//              u = su * sum_up.
// The norm prologue rebuilds a = bf16(x * r * w), r = 1 / sqrt(sum(x^2) / K +
// eps) with the sum of squares in double, as add+RMSNorm computes it
// (kernels_phase2.cu:51-132): every workgroup normalises the whole row for
// itself (8 KB from L2), which costs less than a separate launch.
//
// Layout: 256-thread workgroups of 16 weight rows (swiglu: 8 gate + the 8
// matching up rows). The workgroup walks its rows in order with G4_GEMV_DEPTH
// rows of loads in flight, its 4 waves reading each row together (wave w the
// quarter [w K/4, (w+1) K/4), 16 bytes per lane per 1024-byte chunk,
// non-temporal), so each workgroup's accesses stay inside a few contiguous
// rows. Measured: one row per wave streamed 1 KB at a time left thousands of
// scattered 1 KB streams open and reached 2.4-3.1 TB/s. A lane's activations
// are the same for every row (its K positions are fixed), so they live in
// registers (f32); there is no LDS staging. Sums: per-lane f32 partials, a
// wave reduction, then the 4 waves' partials in a fixed order.

#include "g4_common.h"
#include "g4_hw.h"
#include "g4_math.h"
#include "g4_wave.h"
#include "granite4_layerops.h"

#include <cmath>
#include <cstdio>

namespace g4 {
namespace {

enum : int { kProNone = 0, kProNorm = 1 };
enum : int { kEpiOut = 0, kEpiResid = 1, kEpiSwiglu = 2 };

#ifndef G4_GEMV_DEPTH
#define G4_GEMV_DEPTH 4
#endif
constexpr int kRows = 16;                 // weight rows per workgroup
constexpr int kDepth = G4_GEMV_DEPTH;     // rows of loads in flight
constexpr int kMaxChunks = 4;             // 1024-byte chunks per wave per row: K <= 16384
constexpr int kMaxK = 4 * kMaxChunks * 1024;

struct GemvArgs {
  const uint16_t* x;      // activation, or the residual row to normalise
  const uint16_t* gamma;  // norm weight (kProNorm)
  float eps;
  const uint8_t* w[3];    // weight segments [n_i][K]
  float s[3];             // their scales
  uint16_t* o[3];         // their outputs (kEpiOut); o[0] = out / act otherwise
  int seg1, seg2, N;      // rows [0, seg1) from w[0], [seg1, seg2) from w[1], the rest w[2]
  int K;
  const uint16_t* residual;  // kEpiResid (may alias o[0])
  float rs;
  int I;                  // kEpiSwiglu: act columns (w[0] gate, w[1] up)
};

__device__ __forceinline__ uint4 ld_u4_nt(const uint8_t* p) {
  const g4_u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const g4_u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float wave_sum_f32(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

__device__ __forceinline__ void fp8x16_to_f32(const uint4& q, float (&f)[16]) {
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w[i]), false);
    const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w[i]), true);
    f[4 * i] = lo[0];
    f[4 * i + 1] = lo[1];
    f[4 * i + 2] = hi[0];
    f[4 * i + 3] = hi[1];
  }
}

// Weight row r (0..15) of the workgroup, or nullptr past the end (n: its
// output index). swiglu: rows 0..7 gate, 8..15 up, of the same 8 act columns.
template <int EPI>
__device__ __forceinline__ const uint8_t* row_ptr(const GemvArgs& a, int r, int& n) {
  if (EPI == kEpiSwiglu) {
    const int c = blockIdx.x * (kRows / 2) + (r % (kRows / 2));
    n = c;
    if (c >= a.I) return nullptr;
    return (r < kRows / 2 ? a.w[0] : a.w[1]) + static_cast<size_t>(c) * a.K;
  }
  const int i = blockIdx.x * kRows + r;
  n = i;
  if (i >= a.N) return nullptr;
  if (i < a.seg1) return a.w[0] + static_cast<size_t>(i) * a.K;
  if (i < a.seg2) return a.w[1] + static_cast<size_t>(i - a.seg1) * a.K;
  return a.w[2] + static_cast<size_t>(i - a.seg2) * a.K;
}

// Workgroup barrier for LDS exchanges only (waits for this wave's LDS
// operations, not for its weight loads in flight).
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <int PRO, int EPI, int kChunks>
__global__ __launch_bounds__(256) void gemv_kernel(GemvArgs a) {
  __shared__ double s_ss[4];
  __shared__ float s_part[4][kRows];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int K = a.K;
  const int kq = K / 4;                 // bytes of each row this wave reads
  const int kw = wave * kq;             // its first byte
  // Lane chunk c covers bytes [kw + 1024 c + 16 lane, +16) of every row.
  bool cin[kChunks];
  int koff[kChunks];
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
    const int o = 1024 * c + 16 * lane;
    cin[c] = o < kq;
    koff[c] = kw + (cin[c] ? o : 0);  // out-of-range chunks reread the first (zeroed later)
  }
  const uint8_t* rows[kRows];
  int ns[kRows];
  bool live[kRows];
#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    rows[r] = row_ptr<EPI>(a, r, ns[r]);
    live[r] = rows[r] != nullptr;
    if (!live[r]) rows[r] = a.w[0];
  }

  // Rows of weights stream in order, kDepth rows in flight; the 4 waves read
  // each row together (4 contiguous quarters), so the workgroup's accesses
  // stay within a few contiguous rows at any time. Every load is
  // unconditional (out-of-range data is zeroed before use).
  uint4 buf[kDepth][kChunks];
  const auto load_row = [&](int r, uint4 (&dst)[kChunks]) {
#pragma unroll
    for (int c = 0; c < kChunks; ++c) dst[c] = ld_u4_nt(rows[r] + koff[c]);
  };
#pragma unroll
  for (int r = 0; r < kDepth; ++r) load_row(r, buf[r]);

  // Prologue: the lane's 16 activations per chunk, in registers (f32).
  float av[kChunks][16];
  uint4 xr[kChunks][2];
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
    xr[c][0] = *reinterpret_cast<const uint4*>(a.x + koff[c]);
    xr[c][1] = *reinterpret_cast<const uint4*>(a.x + koff[c] + 8);
  }
  if (PRO == kProNorm) {
    double ss = 0.0;
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
      if (!cin[c]) continue;
      const uint32_t w[8] = {xr[c][0].x, xr[c][0].y, xr[c][0].z, xr[c][0].w,
                             xr[c][1].x, xr[c][1].y, xr[c][1].z, xr[c][1].w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float lo = lo_bf16(w[e]), hi = hi_bf16(w[e]);
        ss += static_cast<double>(lo * lo);
        ss += static_cast<double>(hi * hi);
      }
    }
    ss = wave_sum(ss);
    if (lane == 0) s_ss[wave] = ss;
    lds_barrier();
    ss = s_ss[0] + s_ss[1] + s_ss[2] + s_ss[3];
    const float rr = 1.0f / sqrtf(static_cast<float>(ss / K) + a.eps);
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
      const uint4 g0 = *reinterpret_cast<const uint4*>(a.gamma + koff[c]);
      const uint4 g1 = *reinterpret_cast<const uint4*>(a.gamma + koff[c] + 8);
      const uint32_t xv[8] = {xr[c][0].x, xr[c][0].y, xr[c][0].z, xr[c][0].w,
                              xr[c][1].x, xr[c][1].y, xr[c][1].z, xr[c][1].w};
      const uint32_t gv[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t y = pack_bf16_hw(lo_bf16(xv[e]) * rr * lo_bf16(gv[e]),
                                        hi_bf16(xv[e]) * rr * hi_bf16(gv[e]));
        av[c][2 * e] = lo_bf16(y);
        av[c][2 * e + 1] = hi_bf16(y);
      }
    }
  } else {
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
      const uint32_t xv[8] = {xr[c][0].x, xr[c][0].y, xr[c][0].z, xr[c][0].w,
                              xr[c][1].x, xr[c][1].y, xr[c][1].z, xr[c][1].w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        av[c][2 * e] = lo_bf16(xv[e]);
        av[c][2 * e + 1] = hi_bf16(xv[e]);
      }
    }
  }

  float acc[kRows];
#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    const int slot = r % kDepth;
    float sum = 0.0f;
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
      uint4 q = buf[slot][c];
      if (!(cin[c] && live[r])) q = make_uint4(0u, 0u, 0u, 0u);
      float wf[16];
      fp8x16_to_f32(q, wf);
#pragma unroll
      for (int e = 0; e < 16; ++e) sum = fmaf(wf[e], av[c][e], sum);
    }
    acc[r] = sum;
    if (r + kDepth < kRows) load_row(r + kDepth, buf[slot]);
  }
#pragma unroll
  for (int r = 0; r < kRows; ++r) acc[r] = wave_sum_f32(acc[r]);
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < kRows; ++r) s_part[wave][r] = acc[r];
  }
  lds_barrier();
  if (threadIdx.x >= kRows) return;
  const int r = threadIdx.x;
  const float tot = (s_part[0][r] + s_part[1][r]) + (s_part[2][r] + s_part[3][r]);

  if (EPI == kEpiSwiglu) {
    if (r >= kRows / 2) return;
    const int c = blockIdx.x * (kRows / 2) + r;
    if (c >= a.I) return;
    const float gsum = tot;
    const float usum = (s_part[0][r + kRows / 2] + s_part[1][r + kRows / 2]) +
                       (s_part[2][r + kRows / 2] + s_part[3][r + kRows / 2]);
    a.o[0][c] = static_cast<uint16_t>(f32_to_bf16(silu_mul(a.s[0] * gsum, a.s[1] * usum)));
    return;
  }
  const int n = blockIdx.x * kRows + r;
  if (n >= a.N) return;
  if (EPI == kEpiResid) {
    const float y = a.s[0] * tot;
    const float res = __uint_as_float(static_cast<uint32_t>(a.residual[n]) << 16);
    a.o[0][n] = static_cast<uint16_t>(f32_to_bf16(res + a.rs * y));
  } else {
    const int seg = n < a.seg1 ? 0 : (n < a.seg2 ? 1 : 2);
    const int base = seg == 0 ? 0 : (seg == 1 ? a.seg1 : a.seg2);
    a.o[seg][n - base] = static_cast<uint16_t>(f32_to_bf16(a.s[seg] * tot));
  }
}

bool gemv_k_ok(int K) { return K >= 64 && K % 64 == 0 && K <= kMaxK; }
bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Chunks per wave per row: K / 4 bytes in 1024-byte chunks.
template <int PRO, int EPI>
int launch_gemv(const GemvArgs& a, unsigned grid, const char* what) {
  const int ch = (a.K / 4 + 1023) / 1024;
  const hipStream_t st = stream();
  if (ch <= 1) hipLaunchKernelGGL((gemv_kernel<PRO, EPI, 1>), grid, 256, 0, st, a);
  else if (ch == 2) hipLaunchKernelGGL((gemv_kernel<PRO, EPI, 2>), grid, 256, 0, st, a);
  else hipLaunchKernelGGL((gemv_kernel<PRO, EPI, 4>), grid, 256, 0, st, a);
  return launch_status(what);
}

int gemv_out(int pro, const uint16_t* x, const uint16_t* gamma, float eps,
             const uint8_t* const (&w)[3], const float (&s)[3], uint16_t* const (&o)[3],
             const int (&n)[3], int K, const char* what) {
  const int N = n[0] + n[1] + n[2];
  if (x == nullptr || !al16(x) || !gemv_k_ok(K) || N <= 0 ||
      (pro == kProNorm && (gamma == nullptr || !al16(gamma) || !std::isfinite(eps))) ||
      static_cast<long long>(N) * K >= (1LL << 40)) {
    std::fprintf(stderr, "granite4: %s: invalid arguments (K %% 64 == 0, K <= %d)\n", what, kMaxK);
    return -1;
  }
  GemvArgs a{};
  a.x = x;
  a.gamma = gamma;
  a.eps = eps;
  for (int i = 0; i < 3; ++i) {
    if (n[i] > 0 && (w[i] == nullptr || o[i] == nullptr || !al16(w[i]) || !std::isfinite(s[i]))) {
      std::fprintf(stderr, "granite4: %s: invalid arguments\n", what);
      return -1;
    }
    a.w[i] = w[i];
    a.s[i] = s[i];
    a.o[i] = o[i];
  }
  a.seg1 = n[0];
  a.seg2 = n[0] + n[1];
  a.N = N;
  a.K = K;
  const unsigned grid = static_cast<unsigned>((N + kRows - 1) / kRows);
  return pro == kProNorm ? launch_gemv<kProNorm, kEpiOut>(a, grid, what)
                         : launch_gemv<kProNone, kEpiOut>(a, grid, what);
}

int gemv_swiglu(int pro, const uint16_t* x, const uint16_t* gamma, float eps, const uint8_t* wg,
                const uint8_t* wu, float sg, float su, int N, int K, uint16_t* out,
                const char* what) {
  if (x == nullptr || wg == nullptr || wu == nullptr || out == nullptr || !al16(x) || !al16(wg) ||
      !al16(wu) || !gemv_k_ok(K) || N <= 0 || !std::isfinite(sg) || !std::isfinite(su) ||
      (pro == kProNorm && (gamma == nullptr || !al16(gamma) || !std::isfinite(eps))) ||
      static_cast<long long>(N) * K >= (1LL << 40)) {
    std::fprintf(stderr, "granite4: %s: invalid arguments (K %% 64 == 0, K <= %d)\n", what, kMaxK);
    return -1;
  }
  GemvArgs a{};
  a.x = x;
  a.gamma = gamma;
  a.eps = eps;
  a.w[0] = wg;
  a.w[1] = wu;
  a.s[0] = sg;
  a.s[1] = su;
  a.o[0] = out;
  a.I = N;
  a.N = N;
  a.K = K;
  const unsigned grid = static_cast<unsigned>((N + kRows / 2 - 1) / (kRows / 2));
  return pro == kProNorm ? launch_gemv<kProNorm, kEpiSwiglu>(a, grid, what)
                         : launch_gemv<kProNone, kEpiSwiglu>(a, grid, what);
}

}  // namespace
}  // namespace g4

using namespace g4;

extern "C" {

int granite4_gemv_fp8w(const uint16_t* d_a, const uint8_t* d_w, float scale, int N, int K,
                       uint16_t* d_out) {
  const uint8_t* const w[3] = {d_w, nullptr, nullptr};
  const float s[3] = {scale, 0.0f, 0.0f};
  uint16_t* const o[3] = {d_out, nullptr, nullptr};
  const int n[3] = {N, 0, 0};
  return gemv_out(kProNone, d_a, nullptr, 0.0f, w, s, o, n, K, "granite4_gemv_fp8w");
}

int granite4_gemv_fp8w_resid(const uint16_t* d_a, const uint8_t* d_w, float scale,
                             const uint16_t* d_residual, float resid_scale, int N, int K,
                             uint16_t* d_out) {
  if (d_a == nullptr || d_w == nullptr || d_residual == nullptr || d_out == nullptr || !al16(d_a) ||
      !al16(d_w) || !gemv_k_ok(K) || N <= 0 || !std::isfinite(scale) ||
      !std::isfinite(resid_scale)) {
    std::fprintf(stderr, "granite4: granite4_gemv_fp8w_resid: invalid arguments\n");
    return -1;
  }
  GemvArgs a{};
  a.x = d_a;
  a.w[0] = d_w;
  a.s[0] = scale;
  a.o[0] = d_out;
  a.residual = d_residual;
  a.rs = resid_scale;
  a.seg1 = a.seg2 = a.N = N;
  a.K = K;
  return launch_gemv<kProNone, kEpiResid>(
      a, static_cast<unsigned>((N + kRows - 1) / kRows), "granite4_gemv_fp8w_resid");
}

int granite4_gemv_qkv(const uint16_t* d_a, const uint8_t* d_wq, const uint8_t* d_wk,
                      const uint8_t* d_wv, float sq, float sk, float sv, int Nq, int Nk, int Nv,
                      int K, uint16_t* d_q, uint16_t* d_k, uint16_t* d_v) {
  const uint8_t* const w[3] = {d_wq, d_wk, d_wv};
  const float s[3] = {sq, sk, sv};
  uint16_t* const o[3] = {d_q, d_k, d_v};
  const int n[3] = {Nq, Nk, Nv};
  return gemv_out(kProNone, d_a, nullptr, 0.0f, w, s, o, n, K, "granite4_gemv_qkv");
}

int granite4_gemv_rmsnorm_qkv(const uint16_t* d_x, const uint16_t* d_gamma, float eps,
                              const uint8_t* d_wq, const uint8_t* d_wk, const uint8_t* d_wv,
                              float sq, float sk, float sv, int Nq, int Nk, int Nv, int K,
                              uint16_t* d_q, uint16_t* d_k, uint16_t* d_v) {
  const uint8_t* const w[3] = {d_wq, d_wk, d_wv};
  const float s[3] = {sq, sk, sv};
  uint16_t* const o[3] = {d_q, d_k, d_v};
  const int n[3] = {Nq, Nk, Nv};
  return gemv_out(kProNorm, d_x, d_gamma, eps, w, s, o, n, K, "granite4_gemv_rmsnorm_qkv");
}

int granite4_kernel_silu_gate_up(const uint8_t* d_wg, const uint8_t* d_wu, const uint16_t* d_x,
                                 float scale_g, float scale_u, int N, int K, uint16_t* d_out) {
  return gemv_swiglu(kProNone, d_x, nullptr, 0.0f, d_wg, d_wu, scale_g, scale_u, N, K, d_out,
                     "granite4_kernel_silu_gate_up");
}

int granite4_gemv_rmsnorm_silu_gate_up(const uint16_t* d_x, const uint16_t* d_gamma, float eps,
                                       const uint8_t* d_wg, const uint8_t* d_wu, float scale_g,
                                       float scale_u, int N, int K, uint16_t* d_out) {
  return gemv_swiglu(kProNorm, d_x, d_gamma, eps, d_wg, d_wu, scale_g, scale_u, N, K, d_out,
                     "granite4_gemv_rmsnorm_silu_gate_up");
}

}  // extern "C"
