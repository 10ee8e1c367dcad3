// gemm.hip - FP8 x FP8 GEMM on the gfx950 matrix cores, with the reference
// prefill GEMM's epilogues and the layer epilogues fused into it.
//
// C[m][n] = a_scale * w_scale(n) * sum_k A[m][k] * W[n][k], A fp8 e4m3 codes
// [M][K] (row pitch lda bytes; the FP8 output of add+RMSNorm / SwiGLU with
// its per-tensor scale), W fp8 e4m3 [N][K] row-major with per-tensor scales
// by column segment (scale0 / scale1 / scale2 split at seg1 / seg2, as the
// reference's GemmEpilogue, prefill_gemm.h:12-28). Products of two e4m3
// values are exact in f32; the sum runs in f32 in the matrix cores' order.
//
// Epilogues (the reference's GemmOut kinds, prefill_gemm.cu:69-89, plus the
// layer ops fused in):
//   bf16      out[m][n] = bf16(y)
//   f32       out[m][n] = y
//   residual  out[m][n] = bf16(residual[m][n] + resid_scale * y)  (in place)
//   swiglu    W = [gate rows 0..I-1 ; up rows I..2I-1] (the reference's gate|up
//             weight, forward_gpu.cu:2837); act[m][i] = bf16(silu(g) * u) with
//             g, u the f32 GEMM values (prefill_gemm.cu:1194-1203 applied to
//             the kF32 output without storing it), plus each workgroup's
//             max |act| for the per-tensor FP8 scale of the encode pass.
//
// Layout: 256-thread workgroups on 128 x 128 output tiles (swiglu: 64 act
// columns = 64 gate + 64 up weight rows), 4 waves in 2 x 2, each wave 4 x 4
// v_mfma_f32_16x16x128_f8f6f4 tiles. K advances 128 bytes per stage through
// two LDS buffers (rows padded to 144 bytes: the 16 rows a fragment read
// touches fall on distinct banks); the next stage's global loads are in
// flight while the current one is multiplied. The grid is persistent (at
// most the resident workgroups and the 1024 partial slots); tiles run M
// fastest, so the workgroups sharing a weight tile run together.
//
// Fragment layout: lane l holds row (l % 16) of A and row (l % 16) of W (a
// column of W^T), 32 bytes at k offset 32 * (l / 16) of the 128-byte step;
// A and B take the same k slice per (lane group, byte), so the contraction
// does not depend on the matrix cores' internal k order. The 16 x 16 f32
// result: lane l holds rows 4 (l / 16) + i, column l % 16.

#include "g4_common.h"
#include "g4_hw.h"
#include "g4_math.h"
#include "granite4_layerops.h"

#include <cmath>
#include <cstdio>

namespace g4 {
namespace {

constexpr int kGBM = 128;                 // output rows per tile
constexpr int kGBN = 128;                 // weight rows per tile
constexpr int kGBK = 128;                 // k bytes per stage
constexpr int kGPitch = kGBK + 16;        // LDS row pitch, bytes
constexpr int kGStage = (kGBM + kGBN) * kGPitch;

enum : int {
  kEpiBf16 = GRANITE4_GEMM_BF16,
  kEpiF32 = GRANITE4_GEMM_F32,
  kEpiResidual = GRANITE4_GEMM_RESIDUAL,
  kEpiSwiglu = 3
};

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

struct GemmArgs {
  const uint8_t* A;
  int lda;
  float a_scale;
  const uint8_t* W;
  int M, N, K;  // N: weight rows (swiglu: 2I)
  int I;        // swiglu: act columns
  Granite4GemmEpilogue ep;
  float* partials;  // swiglu: [gridDim.x] max |act|
  int mt, nt;       // tile counts along M and N
};

__device__ __forceinline__ float epi_scale(const Granite4GemmEpilogue& ep, int n) {
  return n < ep.seg1 ? ep.scale0 : (n < ep.seg2 ? ep.scale1 : ep.scale2);
}

// Weight row behind tile row r (0..127) of N tile tn, or -1 past the end.
template <int EPI>
__device__ __forceinline__ int w_row(const GemmArgs& a, int tn, int r) {
  if (EPI == kEpiSwiglu) {
    const int c = tn * 64 + (r & 63);
    if (c >= a.I) return -1;
    return r < 64 ? c : a.I + c;
  }
  const int n = tn * kGBN + r;
  return n < a.N ? n : -1;
}

// Tile row of the wave's B fragment ni (swiglu: ni 0, 1 gate; 2, 3 the
// matching up rows, so one lane holds g and u of the same act element).
template <int EPI>
__device__ __forceinline__ int b_row(int wn, int ni) {
  if (EPI == kEpiSwiglu) return ni < 2 ? wn * 32 + ni * 16 : 64 + wn * 32 + (ni - 2) * 16;
  return wn * 64 + ni * 16;
}

struct StageRegs {
  uint4 a[4], w[4];
};

template <int EPI>
__device__ __forceinline__ void stage_load(const GemmArgs& a, int m0, int tn, int k0,
                                           StageRegs& r) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = threadIdx.x + 256 * i;  // 16-byte chunk of the 128 x 128 tile
    const int row = c >> 3, col = (c & 7) * 16;
    const int m = m0 + row;
    r.a[i] = m < a.M ? *reinterpret_cast<const uint4*>(a.A + static_cast<size_t>(m) * a.lda + k0 + col)
                     : make_uint4(0u, 0u, 0u, 0u);
    const int n = w_row<EPI>(a, tn, row);
    r.w[i] = n >= 0 ? *reinterpret_cast<const uint4*>(a.W + static_cast<size_t>(n) * a.K + k0 + col)
                    : make_uint4(0u, 0u, 0u, 0u);
  }
}

__device__ __forceinline__ void stage_store(uint8_t* st, const StageRegs& r) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = threadIdx.x + 256 * i;
    const int row = c >> 3, col = (c & 7) * 16;
    *reinterpret_cast<uint4*>(st + row * kGPitch + col) = r.a[i];
    *reinterpret_cast<uint4*>(st + (kGBM + row) * kGPitch + col) = r.w[i];
  }
}

__device__ __forceinline__ v8i frag(const uint8_t* p) {
  const uint4 x = *reinterpret_cast<const uint4*>(p);
  const uint4 y = *reinterpret_cast<const uint4*>(p + 16);
  v8i f;
  f[0] = static_cast<int>(x.x);
  f[1] = static_cast<int>(x.y);
  f[2] = static_cast<int>(x.z);
  f[3] = static_cast<int>(x.w);
  f[4] = static_cast<int>(y.x);
  f[5] = static_cast<int>(y.y);
  f[6] = static_cast<int>(y.z);
  f[7] = static_cast<int>(y.w);
  return f;
}

template <int EPI>
__global__ __launch_bounds__(256) void gemm_fp8_kernel(GemmArgs a) {
  __shared__ __align__(16) uint8_t s_tile[2 * kGStage];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int ktiles = a.K / kGBK;
  const int tiles = a.mt * a.nt;
  const int fr = lane & 15;          // fragment row
  const int fk = (lane >> 4) * 32;   // fragment k offset
  float amax = 0.0f;

  for (int tile = blockIdx.x; tile < tiles; tile += gridDim.x) {
    const int tm = tile % a.mt, tn = tile / a.mt;
    const int m0 = tm * kGBM;
    v4f acc[4][4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

    StageRegs r;
    stage_load<EPI>(a, m0, tn, 0, r);
    __syncthreads();  // the previous tile's readers are done with both buffers
    stage_store(s_tile, r);
    __syncthreads();
    for (int kt = 0; kt < ktiles; ++kt) {
      const bool more = kt + 1 < ktiles;
      if (more) stage_load<EPI>(a, m0, tn, (kt + 1) * kGBK, r);
      const uint8_t* st = s_tile + (kt & 1) * kGStage;
      v8i af[4], bf[4];
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) af[mi] = frag(st + (wm * 64 + mi * 16 + fr) * kGPitch + fk);
#pragma unroll
      for (int ni = 0; ni < 4; ++ni)
        bf[ni] = frag(st + (kGBM + b_row<EPI>(wn, ni) + fr) * kGPitch + fk);
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
          acc[mi][ni] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(af[mi], bf[ni], acc[mi][ni],
                                                                         0, 0, 0, 0, 0, 0);
      if (more) stage_store(s_tile + ((kt + 1) & 1) * kGStage, r);
      __syncthreads();
    }

    // Epilogue: lane holds rows m0 + wm*64 + mi*16 + 4*(lane/16) + i.
    const Granite4GemmEpilogue& ep = a.ep;
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = m0 + wm * 64 + mi * 16 + 4 * (lane >> 4) + i;
        if (m >= a.M) continue;
        if (EPI == kEpiSwiglu) {
#pragma unroll
          for (int ni = 0; ni < 2; ++ni) {
            const int c = tn * 64 + wn * 32 + ni * 16 + fr;
            if (c >= a.I) continue;
            const float g = acc[mi][ni][i] * (a.a_scale * ep.scale0);
            const float u = acc[mi][ni + 2][i] * (a.a_scale * ep.scale1);
            const uint32_t h = f32_to_bf16(silu_mul(g, u));
            ep.out_bf16[static_cast<size_t>(m) * ep.ldc + c] = static_cast<uint16_t>(h);
            amax = fmaxf(amax, __uint_as_float((h & 0x7fffu) << 16));
          }
        } else {
#pragma unroll
          for (int ni = 0; ni < 4; ++ni) {
            const int n = tn * kGBN + wn * 64 + ni * 16 + fr;
            if (n >= a.N) continue;
            const float y = acc[mi][ni][i] * (a.a_scale * epi_scale(ep, n));
            const size_t off = static_cast<size_t>(m) * ep.ldc + n;
            if (EPI == kEpiF32) {
              ep.out_f32[off] = y;
            } else if (EPI == kEpiBf16) {
              ep.out_bf16[off] = static_cast<uint16_t>(f32_to_bf16(y));
            } else {
              const float res = __uint_as_float(static_cast<uint32_t>(ep.residual[off]) << 16);
              ep.out_bf16[off] = static_cast<uint16_t>(f32_to_bf16(res + ep.resid_scale * y));
            }
          }
        }
      }
    }
  }
  if (EPI == kEpiSwiglu) write_partial(a.partials, amax);
}

bool gemm_args_ok(const uint8_t* A, int lda, const uint8_t* W, int M, int N, int K) {
  return A != nullptr && W != nullptr && M > 0 && N > 0 && K > 0 && K % kGBK == 0 && lda >= K &&
         lda % 16 == 0 && (reinterpret_cast<uintptr_t>(A) & 15u) == 0 &&
         (reinterpret_cast<uintptr_t>(W) & 15u) == 0 &&
         static_cast<long long>(M) * lda < (1LL << 40);
}

template <int EPI>
unsigned gemm_grid(long long tiles, int cap) {
  const int resident = resident_blocks(reinterpret_cast<const void*>(gemm_fp8_kernel<EPI>), 256);
  long long g = tiles;
  if (resident > 0 && g > resident) g = resident;
  if (g > cap) g = cap;
  return static_cast<unsigned>(g > 0 ? g : 1);
}

}  // namespace
}  // namespace g4

using namespace g4;

extern "C" {

int granite4_gemm_fp8(int out, const uint8_t* A, int lda, float a_scale, const uint8_t* W, int M,
                      int N, int K, const Granite4GemmEpilogue* ep) {
  if (!gemm_args_ok(A, lda, W, M, N, K) || ep == nullptr || ep->ldc < N ||
      !std::isfinite(a_scale) ||
      (out == GRANITE4_GEMM_F32 ? ep->out_f32 == nullptr : ep->out_bf16 == nullptr) ||
      (out == GRANITE4_GEMM_RESIDUAL && ep->residual == nullptr) || out < 0 || out > 2) {
    std::fprintf(stderr, "granite4: granite4_gemm_fp8: invalid arguments (K %% 128 == 0, lda %% 16 == 0)\n");
    return -1;
  }
  GemmArgs a{};
  a.A = A;
  a.lda = lda;
  a.a_scale = a_scale;
  a.W = W;
  a.M = M;
  a.N = N;
  a.K = K;
  a.ep = *ep;
  a.mt = (M + kGBM - 1) / kGBM;
  a.nt = (N + kGBN - 1) / kGBN;
  const long long tiles = static_cast<long long>(a.mt) * a.nt;
  const hipStream_t st = stream();
  switch (out) {
    case GRANITE4_GEMM_BF16:
      hipLaunchKernelGGL(gemm_fp8_kernel<kEpiBf16>, gemm_grid<kEpiBf16>(tiles, INT_MAX), 256, 0, st, a);
      break;
    case GRANITE4_GEMM_F32:
      hipLaunchKernelGGL(gemm_fp8_kernel<kEpiF32>, gemm_grid<kEpiF32>(tiles, INT_MAX), 256, 0, st, a);
      break;
    default:
      hipLaunchKernelGGL(gemm_fp8_kernel<kEpiResidual>, gemm_grid<kEpiResidual>(tiles, INT_MAX), 256,
                         0, st, a);
      break;
  }
  return launch_status("granite4_gemm_fp8");
}

int granite4_gemm_fp8_swiglu(const uint8_t* A, int lda, float a_scale, const uint8_t* W_gu, int M,
                             int I, int K, float gate_scale, float up_scale, uint16_t* act,
                             uint8_t* codes, float* d_scale, void* d_work) {
  if (!gemm_args_ok(A, lda, W_gu, M, 2 * I, K) || act == nullptr || I % 8 != 0 ||
      !std::isfinite(a_scale) || !std::isfinite(gate_scale) || !std::isfinite(up_scale) ||
      d_work == nullptr || (codes != nullptr && d_scale == nullptr) ||
      static_cast<long long>(M) * I >= INT_MAX) {
    std::fprintf(stderr, "granite4: granite4_gemm_fp8_swiglu: invalid arguments\n");
    return -1;
  }
  GemmArgs a{};
  a.A = A;
  a.lda = lda;
  a.a_scale = a_scale;
  a.W = W_gu;
  a.M = M;
  a.N = 2 * I;
  a.K = K;
  a.I = I;
  a.ep.scale0 = gate_scale;
  a.ep.scale1 = up_scale;
  a.ep.out_bf16 = act;
  a.ep.ldc = I;
  a.mt = (M + kGBM - 1) / kGBM;
  a.nt = (I + 63) / 64;
  a.partials = work_partials(d_work);
  const long long tiles = static_cast<long long>(a.mt) * a.nt;
  const unsigned grid = gemm_grid<kEpiSwiglu>(tiles, kMaxPartials);
  hipLaunchKernelGGL(gemm_fp8_kernel<kEpiSwiglu>, grid, 256, 0, stream(), a);
  if (launch_status("granite4_gemm_fp8_swiglu") != 0) return -1;
  if (codes == nullptr) return 0;
  return launch_encode_bf16(act, M, I, work_partials(d_work), static_cast<int>(grid), codes, d_scale)
             ? 0
             : -1;
}

}  // extern "C"
