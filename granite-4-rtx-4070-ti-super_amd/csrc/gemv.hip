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
// Layout: 256-thread workgroups, 16 weight rows each (4 per wave); lane l
// streams bytes [16 l + 1024 j, +16) of its wave's rows (16-byte loads,
// non-temporal: each weight byte is read once per step) with the next step's
// loads in flight, and reads the matching 16 activations from LDS (f32). The
// first weight loads are issued before the prologue, so the norm's latency
// overlaps them. Sums: per-lane f32 partials, then a DPP wave reduction.

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

constexpr int kRowsPerWave = 4;
constexpr int kRowsPerBlock = 4 * kRowsPerWave;
constexpr int kMaxK = 16384;  // LDS activation f32 [K]: 64 KB at most

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

// Weight row r of the workgroup's 16 (swiglu: rows 0..7 gate, 8..15 up of the
// same 8 act columns, wave w holding gate c, c+1 and up c, c+1).
template <int EPI>
__device__ __forceinline__ const uint8_t* row_ptr(const GemvArgs& a, int wave, int j, int& n) {
  if (EPI == kEpiSwiglu) {
    const int c = blockIdx.x * 8 + 2 * wave + (j & 1);
    n = c;
    if (c >= a.I) return nullptr;
    return (j < 2 ? a.w[0] : a.w[1]) + static_cast<size_t>(c) * a.K;
  }
  const int r = blockIdx.x * kRowsPerBlock + wave * kRowsPerWave + j;
  n = r;
  if (r >= a.N) return nullptr;
  if (r < a.seg1) return a.w[0] + static_cast<size_t>(r) * a.K;
  if (r < a.seg2) return a.w[1] + static_cast<size_t>(r - a.seg1) * a.K;
  return a.w[2] + static_cast<size_t>(r - a.seg2) * a.K;
}

template <int PRO, int EPI>
__global__ __launch_bounds__(256) void gemv_kernel(GemvArgs a) {
  extern __shared__ float s_a[];  // activation, f32 [K]
  __shared__ double s_ss[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int K = a.K;
  const int steps = (K + 1023) / 1024;
  const uint8_t* rows[kRowsPerWave];
  int ns[kRowsPerWave];
#pragma unroll
  for (int j = 0; j < kRowsPerWave; ++j) rows[j] = row_ptr<EPI>(a, wave, j, ns[j]);

  // First step's weight loads, before the prologue.
  uint4 wcur[kRowsPerWave];
  const auto load_step = [&](int st, uint4 (&dst)[kRowsPerWave]) {
    const int k0 = st * 1024 + 16 * lane;
#pragma unroll
    for (int j = 0; j < kRowsPerWave; ++j)
      dst[j] = (rows[j] != nullptr && k0 < K) ? ld_u4_nt(rows[j] + k0) : make_uint4(0u, 0u, 0u, 0u);
  };
  load_step(0, wcur);

  // Prologue: the activation into LDS as f32.
  if (PRO == kProNorm) {
    double ss = 0.0;
    for (int k = 8 * threadIdx.x; k < K; k += 8 * 256) {
      const uint4 v = *reinterpret_cast<const uint4*>(a.x + k);
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float lo = lo_bf16(w[e]), hi = hi_bf16(w[e]);
        ss += static_cast<double>(lo * lo);
        ss += static_cast<double>(hi * hi);
      }
    }
    ss = wave_sum(ss);
    if (lane == 0) s_ss[wave] = ss;
    __syncthreads();
    ss = s_ss[0] + s_ss[1] + s_ss[2] + s_ss[3];
    const float r = 1.0f / sqrtf(static_cast<float>(ss / K) + a.eps);
    for (int k = 8 * threadIdx.x; k < K; k += 8 * 256) {
      const uint4 v = *reinterpret_cast<const uint4*>(a.x + k);
      const uint4 g = *reinterpret_cast<const uint4*>(a.gamma + k);
      const uint32_t xv[4] = {v.x, v.y, v.z, v.w}, gv[4] = {g.x, g.y, g.z, g.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t y = pack_bf16_hw(lo_bf16(xv[e]) * r * lo_bf16(gv[e]),
                                        hi_bf16(xv[e]) * r * hi_bf16(gv[e]));
        s_a[k + 2 * e] = lo_bf16(y);
        s_a[k + 2 * e + 1] = hi_bf16(y);
      }
    }
  } else {
    for (int k = 8 * threadIdx.x; k < K; k += 8 * 256) {
      const uint4 v = *reinterpret_cast<const uint4*>(a.x + k);
      const uint32_t xv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        s_a[k + 2 * e] = lo_bf16(xv[e]);
        s_a[k + 2 * e + 1] = hi_bf16(xv[e]);
      }
    }
  }
  __syncthreads();

  float acc[kRowsPerWave] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int st = 0; st < steps; ++st) {
    uint4 wnext[kRowsPerWave];
    if (st + 1 < steps) load_step(st + 1, wnext);
    const int k0 = st * 1024 + 16 * lane;
    if (k0 < K) {
      float av[16];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 f = *reinterpret_cast<const float4*>(s_a + k0 + 4 * q);
        av[4 * q] = f.x;
        av[4 * q + 1] = f.y;
        av[4 * q + 2] = f.z;
        av[4 * q + 3] = f.w;
      }
#pragma unroll
      for (int j = 0; j < kRowsPerWave; ++j) {
        float wf[16];
        fp8x16_to_f32(wcur[j], wf);
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[j] = fmaf(wf[e], av[e], acc[j]);
      }
    }
    if (st + 1 < steps) {
#pragma unroll
      for (int j = 0; j < kRowsPerWave; ++j) wcur[j] = wnext[j];
    }
  }
#pragma unroll
  for (int j = 0; j < kRowsPerWave; ++j) acc[j] = wave_sum_f32(acc[j]);
  if (lane != 0) return;

  if (EPI == kEpiSwiglu) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int c = ns[t];
      if (c >= a.I) continue;
      const float g = a.s[0] * acc[t];
      const float u = a.s[1] * acc[2 + t];
      a.o[0][c] = static_cast<uint16_t>(f32_to_bf16(silu_mul(g, u)));
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < kRowsPerWave; ++j) {
    const int n = ns[j];
    if (n >= a.N) continue;
    if (EPI == kEpiResid) {
      const float y = a.s[0] * acc[j];
      const float res = __uint_as_float(static_cast<uint32_t>(a.residual[n]) << 16);
      a.o[0][n] = static_cast<uint16_t>(f32_to_bf16(res + a.rs * y));
    } else {
      const int seg = n < a.seg1 ? 0 : (n < a.seg2 ? 1 : 2);
      const int base = seg == 0 ? 0 : (seg == 1 ? a.seg1 : a.seg2);
      a.o[seg][n - base] = static_cast<uint16_t>(f32_to_bf16(a.s[seg] * acc[j]));
    }
  }
}

bool gemv_k_ok(int K) { return K > 0 && K % 16 == 0 && K <= kMaxK; }
bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <int PRO, int EPI>
int launch_gemv(const GemvArgs& a, unsigned grid, const char* what) {
  hipLaunchKernelGGL((gemv_kernel<PRO, EPI>), grid, 256, static_cast<size_t>(a.K) * sizeof(float),
                     stream(), a);
  return launch_status(what);
}

int gemv_out(int pro, const uint16_t* x, const uint16_t* gamma, float eps,
             const uint8_t* const (&w)[3], const float (&s)[3], uint16_t* const (&o)[3],
             const int (&n)[3], int K, const char* what) {
  const int N = n[0] + n[1] + n[2];
  if (x == nullptr || !al16(x) || !gemv_k_ok(K) || N <= 0 ||
      (pro == kProNorm && (gamma == nullptr || !al16(gamma) || !std::isfinite(eps))) ||
      static_cast<long long>(N) * K >= (1LL << 40)) {
    std::fprintf(stderr, "granite4: %s: invalid arguments (K %% 16 == 0, K <= %d)\n", what, kMaxK);
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
  const unsigned grid = static_cast<unsigned>((N + kRowsPerBlock - 1) / kRowsPerBlock);
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
    std::fprintf(stderr, "granite4: %s: invalid arguments (K %% 16 == 0, K <= %d)\n", what, kMaxK);
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
  const unsigned grid = static_cast<unsigned>((N + 7) / 8);
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
      a, static_cast<unsigned>((N + kRowsPerBlock - 1) / kRowsPerBlock), "granite4_gemv_fp8w_resid");
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
