// gemm.hip - FP8 x FP8 GEMM on the gfx950 matrix cores, with the reference
// prefill GEMM's epilogues and the layer epilogues fused into it.
//
// C[m][n] = a_scale * w_scale(n) * sum_k A[m][k] * W[n][k], A fp8 e4m3 codes
// [M][K] (row pitch lda bytes; the FP8 output of add+RMSNorm / SwiGLU with
// its per-tensor scale, read from device memory as those ops write it), W fp8 e4m3 [N][K] row-major with per-tensor scales
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
// G4_GEMM_STAGES LDS buffers (32 KB each; 16-byte chunks XOR-swizzled by
// row) filled by direct-to-LDS global loads (global_load_lds_dwordx4), so the
// next stage streams in without staging registers while the current one is
// multiplied. Measured: two stages with two workgroups per CU beat three or
// four stages with one (M = 8192: 2.38 vs 1.47-1.52 PFLOP/s on the down
// projection) and the register-staged form (1.79). Where the 128 x 64 tiles
// give each CU at most one (a short prompt's O and down projections), the
// workgroup takes six stages instead (T=512 down 64.5 -> 58.5 us), three
// where two share a CU. The grid is persistent (at
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
#include <cstdlib>
#include <type_traits>

namespace g4 {
namespace {

constexpr int kGBM = 128;                 // output rows per tile
constexpr int kGBN = 128;                 // weight rows per tile
constexpr int kGBK = 128;                 // k bytes per stage
constexpr int kGStage = (kGBM + kGBN) * kGBK;  // bytes per pipeline stage
#ifndef G4_GEMM_STAGES
#define G4_GEMM_STAGES 2
#endif
constexpr int kGStages = G4_GEMM_STAGES;
constexpr int kEP = 68;  // f32 pitch of the epilogue's LDS staging rows

enum : int {
  kEpiBf16 = GRANITE4_GEMM_BF16,
  kEpiF32 = GRANITE4_GEMM_F32,
  kEpiResidual = GRANITE4_GEMM_RESIDUAL,
  kEpiSwiglu = 3
};

typedef int v8i __attribute__((ext_vector_type(8)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

struct GemmArgs {
  const uint8_t* A;
  int lda;
  const float* a_scale;  // device: the activation's per-tensor scale
  const uint8_t* W;
  int M, N, K;  // N: weight rows (swiglu: 2I)
  int I;        // swiglu: act columns
  Granite4GemmEpilogue ep;
  float* partials;  // swiglu: [gridDim.x] max |act|
  int mt, nt;       // tile counts along M and N
  bool vec_out;     // 16-byte output rows (pitch and width multiples of 8)
  bool xcd_order;   // tiles renumbered per XCD (xcd_tile0)
  // Skinny kBf16 only (gemm_rows_split): when seg_out[0] is set, column n of
  // segment s (ep.seg1 / ep.seg2 bounds) goes to seg_out[s][m * seg_ld[s] +
  // n - start of s] instead of ep.out_bf16.
  uint16_t* seg_out[3];
  int seg_ld[3];
};

// Workgroups are handed to the 8 XCDs round-robin by id (id % 8), each XCD
// with its own L2. The first tile of workgroup b is renumbered so that
// consecutive tile numbers - the M tiles of one weight column, which read the
// same W rows - run on one XCD and share its L2 instead of each XCD fetching
// the column: b -> (b % 8) * (g / 8) + b / 8 over the first 8 * floor(g / 8)
// workgroups (g the grid), the identity on the rest. Tile t + g keeps the
// same XCD as tile t.
__device__ __forceinline__ int xcd_tile0(bool on) {
  const int b = blockIdx.x, g = gridDim.x, full = g & ~7;
  if (!on || b >= full) return b;
  return (b & 7) * (full >> 3) + (b >> 3);
}

__device__ __forceinline__ float epi_scale(const Granite4GemmEpilogue& ep, int n) {
  return n < ep.seg1 ? ep.scale0 : (n < ep.seg2 ? ep.scale1 : ep.scale2);
}

// Weight row behind tile row r (0..127) of N tile tn, or -1 past the end.
template <int EPI, int TN = kGBN>
__device__ __forceinline__ int w_row(const GemmArgs& a, int tn, int r) {
  if (EPI == kEpiSwiglu) {
    const int c = tn * 64 + (r & 63);
    if (c >= a.I) return -1;
    return r < 64 ? c : a.I + c;
  }
  const int n = tn * TN + r;
  return n < a.N ? n : -1;
}

// Tile row of the wave's B fragment ni (swiglu: ni 0, 1 gate; 2, 3 the
// matching up rows, so one lane holds g and u of the same act element).
template <int EPI, int TN = kGBN>
__device__ __forceinline__ int b_row(int wn, int ni) {
  if (EPI == kEpiSwiglu) return ni < 2 ? wn * 32 + ni * 16 : 64 + wn * 32 + (ni - 2) * 16;
  return wn * (TN / 2) + ni * 16;
}

// Stage layout: [A 128 rows][W 128 rows] x 128 bytes, the eight 16-byte
// chunks of row r stored at chunk position c ^ (r & 7) (the 16 rows a
// fragment read touches spread over the banks without padding). A stage is
// filled by direct-to-LDS loads: 16-byte slot s of a region is written by
// lane s % 64 of the wave instruction covering slots (s / 64) * 64.., so the
// lane loads the global chunk that slot s stands for. Rows past M / N load a
// valid row instead (their results are never stored).
typedef __attribute__((address_space(3))) void* lds_ptr;

// Chunk position of 16-byte chunk c of tile row r: c ^ chunk_swz(r).
__device__ __forceinline__ int chunk_swz(int r) { return r & 7; }
// The bf16-A kernel's A rows: c ^ ((r >> 1) & 7). Measured against r & 7
// (A/B on one box): T=8192 down + residual 1716 -> 1611 us, T=512 215.6 ->
// 203 us; the FP8 kernel's fragments show no difference (bank-conflict
// counts equal, times within 1.5 %).
__device__ __forceinline__ int bw_chunk_swz(int r) { return (r >> 1) & 7; }

template <int EPI, int TN = kGBN>
__device__ __forceinline__ void stage_issue(const GemmArgs& a, int m0, int tn, int k0,
                                            uint8_t* st, int tid) {
  const int wave = tid >> 6;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int slot = i * 256 + tid;
    const int row = slot >> 3, c = (slot & 7) ^ chunk_swz(row);
    const int m = min(m0 + row, a.M - 1);
    __builtin_amdgcn_global_load_lds(a.A + static_cast<size_t>(m) * a.lda + k0 + 16 * c,
                                     (lds_ptr)(st + (i * 256 + wave * 64) * 16), 16,
                                     0, 0);
  }
#pragma unroll
  for (int i = 0; i < TN / 32; ++i) {
    const int slot = i * 256 + tid;
    const int row = slot >> 3, c = (slot & 7) ^ chunk_swz(row);
    int n = w_row<EPI, TN>(a, tn, row);
    if (n < 0) n = 0;
    __builtin_amdgcn_global_load_lds(a.W + static_cast<size_t>(n) * a.K + k0 + 16 * c,
                                     (lds_ptr)(st + kGBM * kGBK + (i * 256 + wave * 64) * 16),
                                     16, 0, 0);
  }
}

// LDS byte address of a pointer into the workgroup's LDS.
__device__ __forceinline__ uint32_t lds_addr(const uint8_t* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_ptr)(p)));
}

// 16-byte LDS read issued as assembly: the compiler's wait insertion would
// otherwise wait for every direct-to-LDS load in flight (it cannot tell the
// stage being read from the stages being filled). The caller waits with
// lds_reads_done() before using the result.
__device__ __forceinline__ v4u lds_read16(uint32_t addr) {
  v4u v;
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr) : "memory");
  return v;
}
__device__ __forceinline__ void lds_reads_done() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
// Waits until at most N of the wave's LDS reads are still in flight.
template <int N>
__device__ __forceinline__ void lds_reads_left() {
  if constexpr (N == 0) asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  else if constexpr (N == 1) asm volatile("s_waitcnt lgkmcnt(1)" ::: "memory");
  else if constexpr (N == 2) asm volatile("s_waitcnt lgkmcnt(2)" ::: "memory");
  else if constexpr (N == 3) asm volatile("s_waitcnt lgkmcnt(3)" ::: "memory");
  else if constexpr (N == 4) asm volatile("s_waitcnt lgkmcnt(4)" ::: "memory");
  else if constexpr (N == 6) asm volatile("s_waitcnt lgkmcnt(6)" ::: "memory");
  else if constexpr (N == 8) asm volatile("s_waitcnt lgkmcnt(8)" ::: "memory");
  else if constexpr (N == 9) asm volatile("s_waitcnt lgkmcnt(9)" ::: "memory");
  else if constexpr (N == 10) asm volatile("s_waitcnt lgkmcnt(10)" ::: "memory");
  else if constexpr (N == 11) asm volatile("s_waitcnt lgkmcnt(11)" ::: "memory");
  else static_assert(N < 0, "add the count");
}

// Fragment of tile row r of a region at LDS address `region`: chunks
// 2 * (lane / 16) and + 1 of the row, as two 16-byte reads.
__device__ __forceinline__ void frag_issue(uint32_t region, int r, int lane, v4u& x, v4u& y) {
  const int c0 = 2 * (lane >> 4);
  const uint32_t row = region + static_cast<uint32_t>(r * kGBK);
  x = lds_read16(row + 16u * static_cast<uint32_t>(c0 ^ chunk_swz(r)));
  y = lds_read16(row + 16u * static_cast<uint32_t>((c0 + 1) ^ chunk_swz(r)));
}

__device__ __forceinline__ v8i frag_of(const v4u& x, const v4u& y) {
  v8i f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[i] = static_cast<int>(x[i]);
    f[i + 4] = static_cast<int>(y[i]);
  }
  return f;
}

__device__ __forceinline__ void wave_lds_wait() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Two bf16 RNE conversions in one v_cvt_pk_bf16_f32 (equal to the integer
// rounding for every non-NaN value).
__device__ __forceinline__ uint32_t pack_bf16_rne(float lo, float hi) { return pack_bf16_hw(lo, hi); }

// Waits until at most `later` stages' loads (LPS per thread each) are in
// flight (vmcnt counts a thread's loads in issue order).
template <int N>
__device__ __forceinline__ void vm_wait() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  if constexpr (N == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  else if constexpr (N == 6) asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
  else if constexpr (N == 8) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  else if constexpr (N == 12) asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
  else if constexpr (N == 16) asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
  else if constexpr (N == 18) asm volatile("s_waitcnt vmcnt(18)" ::: "memory");
  else if constexpr (N == 24) asm volatile("s_waitcnt vmcnt(24)" ::: "memory");
  else if constexpr (N == 30) asm volatile("s_waitcnt vmcnt(30)" ::: "memory");
  else if constexpr (N == 32) asm volatile("s_waitcnt vmcnt(32)" ::: "memory");
  else if constexpr (N == 40) asm volatile("s_waitcnt vmcnt(40)" ::: "memory");
  else static_assert(N < 0, "add the count");
}
template <int LPS>
__device__ __forceinline__ void stage_wait_n(int later) {
  if (later >= 5) vm_wait<5 * LPS>();
  else if (later == 4) vm_wait<4 * LPS>();
  else if (later == 3) vm_wait<3 * LPS>();
  else if (later == 2) vm_wait<2 * LPS>();
  else if (later == 1) vm_wait<LPS>();
  else vm_wait<0>();
}

// Epilogue of one output tile through LDS: each wave writes its f32 values
// (y = acc * (a_scale * w_scale(n)), or silu(g) * u) 32 rows at a time into
// its own region and reads them back row-contiguous, so a lane owns 8
// consecutive columns and every global access is 16 bytes (or, where the
// output pitch or width is not a multiple of 8, element by element). The
// residual was prefetched at the tile's start (a load after a store would
// wait for the store: the vector memory counter covers both).
template <int EPI, int kIters, int kWCols, bool kBarrier = true>
__device__ __forceinline__ void tile_epilogue(const GemmArgs& a, const v4f (&acc)[4][4],
                                              float a_scale, uint8_t* s_tile, int m0, int col0,
                                              int n_end, const uint4* res, float& amax) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave >> 1;
  const int fr = lane & 15;
  constexpr int kLanesPerRow = kWCols / 8;
  constexpr int kRowsPerIter = 64 / kLanesPerRow;
  if (kBarrier) __builtin_amdgcn_s_barrier();  // every wave is past its last fragment read
  float* const sv = reinterpret_cast<float*>(s_tile) + wave * (32 * kEP);
  const Granite4GemmEpilogue& ep = a.ep;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int mj = 0; mj < 2; ++mj) {
      const int mi = 2 * h + mj;
#pragma unroll
      for (int ni = 0; ni < kWCols / 16; ++ni) {
        const int col = ni * 16 + fr;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float v;
          if (EPI == kEpiSwiglu) {
            const float g = acc[mi][ni][i] * (a_scale * ep.scale0);
            const float u = acc[mi][ni + 2][i] * (a_scale * ep.scale1);
            v = silu_mul(g, u);
          } else {
            v = acc[mi][ni][i] * (a_scale * epi_scale(ep, col0 + col));
          }
          sv[(mj * 16 + 4 * (lane >> 4) + i) * kEP + col] = v;
        }
      }
    }
    wave_lds_wait();
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
      const int rl = it * kRowsPerIter + lane / kLanesPerRow;
      const int ch = lane % kLanesPerRow;
      const int m = m0 + wm * 64 + h * 32 + rl;
      const int n = col0 + ch * 8;
      const float4 lo = *reinterpret_cast<const float4*>(sv + rl * kEP + ch * 8);
      const float4 hi = *reinterpret_cast<const float4*>(sv + rl * kEP + ch * 8 + 4);
      if (m >= a.M || n >= n_end) continue;
      const float y[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
      const size_t off = static_cast<size_t>(m) * ep.ldc + n;
      if (EPI != kEpiSwiglu && !a.vec_out) {
        // Element by element (an output pitch or width that is not a
        // multiple of 8): the same arithmetic per element.
        for (int e = 0; e < 8 && n + e < n_end; ++e) {
          if (EPI == kEpiF32) {
            ep.out_f32[off + e] = y[e];
          } else if (EPI == kEpiResidual) {
            const float r = bf16_to_f32(ep.residual[off + e]);
            ep.out_bf16[off + e] = static_cast<uint16_t>(f32_to_bf16(r + ep.resid_scale * y[e]));
          } else {
            ep.out_bf16[off + e] = static_cast<uint16_t>(f32_to_bf16(y[e]));
          }
        }
        continue;
      }
      if (EPI == kEpiF32) {
        *reinterpret_cast<float4*>(ep.out_f32 + off) = lo;
        *reinterpret_cast<float4*>(ep.out_f32 + off + 4) = hi;
        continue;
      }
      uint32_t w[4];
      if (EPI == kEpiResidual) {
        const uint4 r = res[h * kIters + it];
        const uint32_t rw[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
        for (int e = 0; e < 4; ++e)
          w[e] = pack_bf16_rne(lo_bf16(rw[e]) + ep.resid_scale * y[2 * e],
                               hi_bf16(rw[e]) + ep.resid_scale * y[2 * e + 1]);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = pack_bf16_rne(y[2 * e], y[2 * e + 1]);
      }
      if (EPI == kEpiSwiglu) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          amax = fmaxf(amax, fmaxf(lo_bf16(w[e] & 0x7fff7fffu), hi_bf16(w[e] & 0x7fff7fffu)));
      }
      *reinterpret_cast<uint4*>(ep.out_bf16 + off) = make_uint4(w[0], w[1], w[2], w[3]);
    }
    wave_lds_wait();  // reads done before the next half's writes
  }
}

// TN: weight rows per tile, 128, or 64 where 128 x 128 tiles cannot fill the
// CUs (a short prompt's O and down projections: 128 tiles at M = 512); each
// wave then owns 64 x 32 outputs (4 x 2 MFMA tiles).
// ST: pipeline stages (kGStages, or more where one workgroup per CU leaves
// it the LDS).
// KS = 2: K split inside the workgroup. Two 4-wave halves (512 threads) run
// K tiles [0, kh) and [kh, ktiles) through their own ST stages, meeting at
// every barrier (half 1 idles through its last step when ktiles is odd);
// half 1 then hands its accumulators to half 0 through LDS, which adds them
// (the sum of two f32 partial sums) and runs the epilogue. Two waves per
// SIMD instead of one where a short prompt gives each CU one tile.
template <int EPI, int TN = kGBN, int ST = kGStages, int KS = 1>
__global__ __launch_bounds__(256 * KS) void gemm_fp8_kernel(GemmArgs a) {
  static_assert(TN == kGBN || (TN == 64 && EPI != kEpiSwiglu), "tile width");
  static_assert(KS == 1 || (KS == 2 && EPI != kEpiSwiglu), "split K: plain epilogues only");
  constexpr int kNI = TN / 32;  // MFMA tiles per wave along N
  constexpr int kStage = (kGBM + TN) * kGBK;
  __shared__ __align__(16) uint8_t s_tile[KS * ST * kStage];
  constexpr int kLps = 4 + TN / 32;  // loads per thread per stage
  const int tid = threadIdx.x & 255;
  const int half = KS == 2 ? static_cast<int>(threadIdx.x >> 8) : 0;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int ktiles = a.K / kGBK;
  const int kh = KS == 2 ? (ktiles + 1) / 2 : ktiles;  // steps of the K loop
  const int kbeg = half * kh;
  const int kn = KS == 2 ? min(kh, ktiles - kbeg) : ktiles;  // this half's K tiles
  uint8_t* const sbase = s_tile + half * ST * kStage;
  const int tiles = a.mt * a.nt;
  const int fr = lane & 15;          // fragment row
  const float a_scale = *a.a_scale;
  float amax = 0.0f;
  static_assert(ST >= 2 && ST <= 6, "pipeline depth");
  // Epilogue geometry: the wave's output block is 64 rows x kWCols columns.
  constexpr int kWCols = EPI == kEpiSwiglu ? 32 : TN / 2;
  constexpr int kLanesPerRow = kWCols / 8;
  constexpr int kRowsPerIter = 64 / kLanesPerRow;
  constexpr int kIters = 32 / kRowsPerIter;
  static_assert(4 * 32 * kEP * 4 <= ST * kStage, "epilogue staging fits the stage buffers");

  for (int tile = xcd_tile0(a.xcd_order); tile < tiles; tile += gridDim.x) {
    const int tm = tile % a.mt, tn = tile / a.mt;
    const int m0 = tm * kGBM;
    v4f acc[4][4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

    // This wave's output columns [col0, col0 + kWCols) (act columns for swiglu).
    const int col0 = EPI == kEpiSwiglu ? tn * 64 + wn * 32 : tn * TN + wn * (TN / 2);
    const int n_end = EPI == kEpiSwiglu ? a.I : a.N;
    uint4 res[EPI == kEpiResidual ? 2 * kIters : 1];
    if (EPI == kEpiResidual && half == 0) {
#pragma unroll
      for (int j = 0; j < 2 * kIters; ++j) {
        const int h = j / kIters, it = j % kIters;
        const int m = m0 + wm * 64 + h * 32 + it * kRowsPerIter + lane / kLanesPerRow;
        const int n = col0 + (lane % kLanesPerRow) * 8;
        res[j] = (m < a.M && n < n_end)
                     ? *reinterpret_cast<const uint4*>(a.ep.residual + static_cast<size_t>(m) * a.ep.ldc + n)
                     : make_uint4(0u, 0u, 0u, 0u);
      }
    }

    __syncthreads();  // the previous tile's readers are done with every buffer
#pragma unroll
    for (int sidx = 0; sidx < ST - 1; ++sidx)
      if (sidx < kn) stage_issue<EPI, TN>(a, m0, tn, (kbeg + sidx) * kGBK, sbase + sidx * kStage, tid);
    for (int kt = 0; kt < kh; ++kt) {
      // Stages issued after kt so far: min(kStages - 2, kn - 1 - kt).
      const int later = min(ST - 2, kn - 1 - kt);
      stage_wait_n<kLps>(later);
      // Stage kt landed for every wave (each waited for its own loads);
      // stage kt - 1's reads are done (waited before its MFMAs). No fence:
      // a workgroup-scope release would wait for the stages still in flight.
      __builtin_amdgcn_s_barrier();
      if (kt + ST - 1 < kn)
        stage_issue<EPI, TN>(a, m0, tn, (kbeg + kt + ST - 1) * kGBK,
                             sbase + ((kt + ST - 1) % ST) * kStage, tid);
      if (KS == 2 && kt >= kn) continue;  // half 1's idle last step (odd ktiles)
      const uint32_t st = lds_addr(sbase + (kt % ST) * kStage);
      v4u ax[4], ay[4], bx[kNI], by[kNI];
      // B's fragments first, then A's row blocks in order: row block mi's
      // MFMAs start once its two reads (and B's) have landed, while the
      // later blocks' reads are still in flight (LDS reads complete in order).
#pragma unroll
      for (int ni = 0; ni < kNI; ++ni)
        frag_issue(st + kGBM * kGBK, b_row<EPI, TN>(wn, ni) + fr, lane, bx[ni], by[ni]);
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) frag_issue(st, wm * 64 + mi * 16 + fr, lane, ax[mi], ay[mi]);
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) {
        if (mi == 0) lds_reads_left<6>();
        else if (mi == 1) lds_reads_left<4>();
        else if (mi == 2) lds_reads_left<2>();
        else lds_reads_left<0>();
        // The fragments pass through the wait: no use can move above it.
        asm volatile("" : "+v"(ax[mi]), "+v"(ay[mi]));
        if (mi == 0) {
#pragma unroll
          for (int j = 0; j < kNI; ++j) asm volatile("" : "+v"(bx[j]), "+v"(by[j]));
        }
#pragma unroll
        for (int ni = 0; ni < kNI; ++ni)
          acc[mi][ni] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
              frag_of(ax[mi], ay[mi]), frag_of(bx[ni], by[ni]), acc[mi][ni], 0, 0, 0, 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);  // keep the block's MFMAs ahead of the next wait
      }
    }

    if constexpr (KS == 2) {
      // Half 1's accumulators to half 0 through half 1's stage buffers
      // (16 bytes per lane and MFMA tile, lane-contiguous).
      __builtin_amdgcn_s_barrier();  // every wave is past its last fragment read
      v4f* const xa = reinterpret_cast<v4f*>(s_tile + ST * kStage) + wave * (4 * kNI * 64) + lane;
      if (half == 1) {
#pragma unroll
        for (int mi = 0; mi < 4; ++mi)
#pragma unroll
          for (int ni = 0; ni < kNI; ++ni) xa[(mi * kNI + ni) * 64] = acc[mi][ni];
      }
      wave_lds_wait();
      __builtin_amdgcn_s_barrier();
      if (half == 1) continue;  // the next tile's first barrier waits for half 0's epilogue
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int ni = 0; ni < kNI; ++ni) acc[mi][ni] += xa[(mi * kNI + ni) * 64];
    }
    tile_epilogue<EPI, kIters, kWCols, KS == 1>(a, acc, a_scale, s_tile, m0, col0, n_end, res,
                                                amax);
  }
  if (EPI == kEpiSwiglu) write_partial(a.partials, amax);
}

// ---------------------------------------------------------------------------
// bf16 A x fp8 W (the reference's prefill_gemm, prefill_gemm.h:34-39):
// C[m][n] = w_scale(n) * sum_k A[m][k] * W[n][k], A bf16 [M][lda], W e4m3
// [N][K]. Each product bf16 x e4m3 is exact in f32; the sum runs in f32 in
// the matrix cores' order (v_mfma_f32_16x16x32_bf16).
//
// Same tiling, persistent grid and epilogue as gemm_fp8_kernel; K advances
// 64 elements per stage. A stage holds A as 128 rows x 128 bytes (the bf16
// k-slice, eight 16-byte chunks XOR-swizzled by (row / 2) % 8) and W raw as 128 rows
// x 64 bytes (four chunks, swizzled by (row / 2) % 4), both filled by
// direct-to-LDS loads. Each wave converts its W fragments from e4m3 to bf16
// as it reads them (exact: an e4m3 value has at most 4 significant bits, so
// its bf16 is the top half of its f32): one conversion and one byte permute
// per two elements. A stage whose second 32-element half lies past K (K % 64
// == 32) loads valid bytes there and skips that half's MFMAs.
constexpr int kBwK = 64;                          // k elements per stage
constexpr int kBwARow = 2 * kBwK;                 // A bytes per tile row per stage
constexpr int kBwWRow = kBwK;                     // W bytes per tile row per stage
constexpr int kBwStage = kGBM * kBwARow + kGBN * kBwWRow;  // 24 KB

typedef __bf16 bf16x8_g __attribute__((ext_vector_type(8)));

template <int EPI>
__device__ __forceinline__ void bw_stage_issue(const GemmArgs& a, int m0, int tn, int k0,
                                               uint8_t* st) {
  const int wave = threadIdx.x >> 6;
  const uint16_t* A = reinterpret_cast<const uint16_t*>(a.A);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int slot = i * 256 + threadIdx.x;
    const int row = slot >> 3, c = (slot & 7) ^ bw_chunk_swz(row);
    const int m = min(m0 + row, a.M - 1);
    const int k = k0 + 8 * c < a.K ? k0 + 8 * c : 0;  // past K: a valid chunk, unused
    __builtin_amdgcn_global_load_lds(A + static_cast<size_t>(m) * a.lda + k,
                                     (lds_ptr)(st + (i * 256 + wave * 64) * 16), 16, 0, 0);
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int slot = i * 256 + threadIdx.x;
    const int row = slot >> 2, c = (slot & 3) ^ ((row >> 1) & 3);
    int n = w_row<EPI>(a, tn, row);
    if (n < 0) n = 0;
    const int k = k0 + 16 * c < a.K ? k0 + 16 * c : 0;
    __builtin_amdgcn_global_load_lds(a.W + static_cast<size_t>(n) * a.K + k,
                                     (lds_ptr)(st + kGBM * kBwARow + (i * 256 + wave * 64) * 16),
                                     16, 0, 0);
  }
}

__device__ __forceinline__ uint2 lds_read8(uint32_t addr) {
  uint2 v;
  asm volatile("ds_read_b64 %0, %1" : "=v"(v) : "v"(addr) : "memory");
  return v;
}

// Eight e4m3 codes -> eight bf16 (exact), in element order.
__device__ __forceinline__ bf16x8_g fp8x8_to_bf16(uint2 q) {
  uint32_t w[4];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t x = h ? q.y : q.x;
    const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(x), false);
    const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(x), true);
    w[2 * h] = __builtin_amdgcn_perm(__float_as_uint(lo[1]), __float_as_uint(lo[0]), 0x07060302u);
    w[2 * h + 1] = __builtin_amdgcn_perm(__float_as_uint(hi[1]), __float_as_uint(hi[0]), 0x07060302u);
  }
  const v4u u = {w[0], w[1], w[2], w[3]};
  return __builtin_bit_cast(bf16x8_g, u);
}

template <int EPI, bool kLateRes = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void gemm_bf16w_kernel(GemmArgs a) {
  __shared__ __align__(16) uint8_t s_tile[2 * kBwStage];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int ktiles = (a.K + kBwK - 1) / kBwK;
  const int tiles = a.mt * a.nt;
  const int fr = lane & 15;
  float amax = 0.0f;
  constexpr int kWCols = 64;
  constexpr int kLanesPerRow = kWCols / 8;
  constexpr int kRowsPerIter = 64 / kLanesPerRow;
  constexpr int kIters = 32 / kRowsPerIter;
  static_assert(4 * 32 * kEP * 4 <= 2 * kBwStage, "epilogue staging fits the stage buffers");

  for (int tile = xcd_tile0(a.xcd_order); tile < tiles; tile += gridDim.x) {
    const int tm = tile % a.mt, tn = tile / a.mt;
    const int m0 = tm * kGBM;
    v4f acc[4][4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    const int col0 = tn * kGBN + wn * 64;
    const int n_end = a.N;
    // The residual of the tile's outputs: loaded at the tile's start (its wait
    // overlaps the first stage's), or, kLateRes, after the K loop. Held across
    // the loop its 32 registers leave one wave per SIMD: with more tiles than
    // CUs (T=8192 down + residual: 1437 -> 1150 us) the second wave is worth
    // more than the round trip; with one tile per workgroup (T=512: 175 vs
    // 189 us) it is not.
    uint4 res[EPI == kEpiResidual ? 2 * kIters : 1];
    const auto load_res = [&] {
#pragma unroll
      for (int j = 0; j < 2 * kIters; ++j) {
        const int h = j / kIters, it = j % kIters;
        const int m = m0 + wm * 64 + h * 32 + it * kRowsPerIter + lane / kLanesPerRow;
        const int n = col0 + (lane % kLanesPerRow) * 8;
        res[j] = (a.vec_out && m < a.M && n < n_end)
                     ? *reinterpret_cast<const uint4*>(a.ep.residual + static_cast<size_t>(m) * a.ep.ldc + n)
                     : make_uint4(0u, 0u, 0u, 0u);
      }
    };
    if (EPI == kEpiResidual && !kLateRes) load_res();

    __syncthreads();  // the previous tile's readers are done with both buffers
    bw_stage_issue<EPI>(a, m0, tn, 0, s_tile);
    for (int kt = 0; kt < ktiles; ++kt) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      // Stage kt landed for every wave; stage kt - 1's reads are done.
      __builtin_amdgcn_s_barrier();
      if (kt + 1 < ktiles) bw_stage_issue<EPI>(a, m0, tn, (kt + 1) * kBwK, s_tile + ((kt + 1) & 1) * kBwStage);
      const uint32_t st = lds_addr(s_tile + (kt & 1) * kBwStage);
      const uint32_t sw = st + kGBM * kBwARow;
      const int halves = a.K - kt * kBwK >= kBwK ? 2 : 1;  // wave-uniform
      // Both 32-element halves' reads go out first (W's fragments, then A's
      // row blocks, per half), and each row block's MFMAs start once its
      // reads have landed: the second half's reads overlap the first half's
      // MFMAs (LDS reads complete in order).
      v4u ax[2][4];
      uint2 bq[2][4];
      const uint32_t wh = 8u * static_cast<uint32_t>((lane >> 4) & 1);
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        if (s >= halves) break;
        const int ca = 4 * s + (lane >> 4);            // A chunk: elements 32 s + 8 (lane / 16)
        const int cw = 2 * s + (lane >> 5);            // W chunk: bytes 32 s + 8 (lane / 16)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) {
          const int r = wn * 64 + ni * 16 + fr;
          bq[s][ni] = lds_read8(sw + static_cast<uint32_t>(r * kBwWRow) +
                                16u * static_cast<uint32_t>(cw ^ ((r >> 1) & 3)) + wh);
        }
#pragma unroll
        for (int mi = 0; mi < 4; ++mi) {
          const int r = wm * 64 + mi * 16 + fr;
          ax[s][mi] = lds_read16(st + static_cast<uint32_t>(r * kBwARow) +
                                 16u * static_cast<uint32_t>(ca ^ bw_chunk_swz(r)));
        }
      }
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        if (s >= halves) break;
        const bool more = s == 0 && halves == 2;  // the second half's 8 reads are behind
        bf16x8_g bf[4];
#pragma unroll
        for (int mi = 0; mi < 4; ++mi) {
          if (more) {
            if (mi == 0) lds_reads_left<11>();
            else if (mi == 1) lds_reads_left<10>();
            else if (mi == 2) lds_reads_left<9>();
            else lds_reads_left<8>();
          } else {
            if (mi == 0) lds_reads_left<3>();
            else if (mi == 1) lds_reads_left<2>();
            else if (mi == 2) lds_reads_left<1>();
            else lds_reads_left<0>();
          }
          asm volatile("" : "+v"(ax[s][mi]));
          if (mi == 0) {
#pragma unroll
            for (int j = 0; j < 4; ++j) asm volatile("" : "+v"(bq[s][j]));
#pragma unroll
            for (int ni = 0; ni < 4; ++ni) bf[ni] = fp8x8_to_bf16(bq[s][ni]);
          }
          const bf16x8_g af = __builtin_bit_cast(bf16x8_g, ax[s][mi]);
#pragma unroll
          for (int ni = 0; ni < 4; ++ni)
            acc[mi][ni] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, bf[ni], acc[mi][ni], 0, 0, 0);
          __builtin_amdgcn_sched_barrier(0);  // keep the block's MFMAs ahead of the next wait
        }
      }
    }
    if (EPI == kEpiResidual && kLateRes) load_res();
    tile_epilogue<EPI, kIters, kWCols>(a, acc, 1.0f, s_tile, m0, col0, n_end, res, amax);
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

bool gemm_args_ok(const uint8_t* A, int lda, const uint8_t* W, int M, int N, int K) {
  return A != nullptr && W != nullptr && M > 0 && N > 0 && K > 0 && K % kGBK == 0 && lda >= K &&
         lda % 16 == 0 && (reinterpret_cast<uintptr_t>(A) & 15u) == 0 &&
         (reinterpret_cast<uintptr_t>(W) & 15u) == 0 &&
         static_cast<long long>(M) * lda < (1LL << 40);
}

// Whether XCD-ordered tiles (xcd_tile0) cut the L2 fills of a launch of g
// workgroups over mt M tiles. Per round each XCD runs g / 8 tiles; the A rows
// and W rows it fetches grow with the block of tiles it covers, bm M tiles x
// bn N tiles, as bm + bn. XCD order gives each XCD whole columns, bm = mt
// (up to g / 8); the plain order gives it every 8th tile: one M tile (mt <= 8)
// or mt / 8 of them, spread over g / 8 or g / mt columns. Measured: T = 512
// gate|up 88 -> 77 us with XCD order (4 x 16 against 1 x 64), T = 8192 the
// plain order's 8 x 8 beats XCD order's 64 x 1 by 14-17 %.
bool gemm_xcd_order(int mt, unsigned g) {
  if (g < 16) return false;
  const long long per = g / 8;
  const long long xbm = mt < per ? mt : per, xbn = (per + mt - 1) / mt;
  const long long pbm = mt <= 8 ? 1 : mt / 8, pbn = mt <= 8 ? per : (g + mt - 1) / mt;
  return xbm + xbn < pbm + pbn;
}


// ---------------------------------------------------------------------------
// Skinny GEMM, M <= 16 rows (a batched decode step's sessions, a short
// chunk): the 128-row tiles above would leave 120 of 128 MFMA rows idle and
// stream each weight tile through LDS. Here a workgroup of NW waves owns 16
// weight rows (swiglu: 16 gate + the matching 16 up rows) and all M rows,
// one 16 x 16 MFMA tile; its NW waves split K into NW parts, each streaming
// its part of the 16 rows straight from global memory into the MFMA
// fragments (lane l: row l % 16, the fragment's bytes at k offset
// (l / 16) * 32 of a 128-element step, for bf16 activations split over
// four MFMAs), U steps of loads in flight. A rows past M and
// weight rows past N read row M - 1 / N - 1 (their outputs are not
// stored). The NW partial tiles are summed in wave order through LDS, and
// wave 0 stores the tile with the epilogue of the large kernels (same
// y = acc * (a_scale * w_scale(n)), residual and SwiGLU arithmetic). The f32
// sum's order differs from the large kernels' (K in NW parts); both are
// held to the same parity bar.
// ---------------------------------------------------------------------------
constexpr int kSkinnyMaxM = 16;

template <bool F8A, int EPI, int U, int NW>
__global__ __launch_bounds__(NW * 64) void gemm_skinny_kernel(GemmArgs a) {
  __shared__ v4f s_acc[2][NW - 1][64];  // waves 1..NW-1's partial tiles (gate / up)
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int fr = lane & 15, fq = lane >> 4;
  constexpr int kStepK = 128;  // k elements per step (bf16 A: four MFMAs)
  const int steps = a.K / kStepK;
  const int s0 = wave * steps / NW, s1 = (wave + 1) * steps / NW;
  const int arow = min(fr, a.M - 1);
  constexpr int kTiles = EPI == kEpiSwiglu ? 2 : 1;
  const int ncols = EPI == kEpiSwiglu ? a.I : a.N;
  const int ntile = (ncols + 15) / 16;
  float amax = 0.0f;
  const float a_scale = F8A ? *a.a_scale : 1.0f;
  for (int tile = blockIdx.x; tile < ntile; tile += gridDim.x) {
    const int c = min(tile * 16 + fr, ncols - 1);
    // this lane's weight rows: column c (gate row c and up row I + c for swiglu)
    const uint8_t* wrow[kTiles];
    wrow[0] = a.W + static_cast<size_t>(c) * a.K;
    if (EPI == kEpiSwiglu) wrow[kTiles - 1] = a.W + static_cast<size_t>(a.I + c) * a.K;
    v4f acc[kTiles];
#pragma unroll
    for (int t = 0; t < kTiles; ++t) acc[t] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    for (int sb = s0; sb < s1; sb += U) {
      if constexpr (F8A) {
        v4u wx[U][kTiles], wy[U][kTiles], ax[U], ay[U];
        const uint8_t* arow_p = a.A + static_cast<size_t>(arow) * a.lda;
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int k = min(sb + u, s1 - 1) * kStepK + 32 * fq;
#pragma unroll
          for (int t = 0; t < kTiles; ++t) {
            wx[u][t] = *reinterpret_cast<const v4u*>(wrow[t] + k);
            wy[u][t] = *reinterpret_cast<const v4u*>(wrow[t] + k + 16);
          }
          ax[u] = *reinterpret_cast<const v4u*>(arow_p + k);
          ay[u] = *reinterpret_cast<const v4u*>(arow_p + k + 16);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          if (sb + u >= s1) break;
#pragma unroll
          for (int t = 0; t < kTiles; ++t)
            acc[t] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                frag_of(ax[u], ay[u]), frag_of(wx[u][t], wy[u][t]), acc[t], 0, 0, 0, 0, 0, 0);
        }
      } else {
        // A step's 128 k elements as four MFMAs: lane group fq reads the
        // 32 contiguous weight bytes 32 fq .. 32 fq + 31 of the step (and the
        // same 32 activations), and feeds bytes 8 j .. 8 j + 7 to MFMA j as
        // its k slot fq. A and B take the same k assignment, so each MFMA sums
        // products of matching k; the four cover the step.
        v4u wx[U][kTiles], wy[U][kTiles], ax[U][4];
        const uint16_t* arow_p = reinterpret_cast<const uint16_t*>(a.A) + static_cast<size_t>(arow) * a.lda;
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int k = min(sb + u, s1 - 1) * kStepK + 32 * fq;
#pragma unroll
          for (int t = 0; t < kTiles; ++t) {
            wx[u][t] = *reinterpret_cast<const v4u*>(wrow[t] + k);
            wy[u][t] = *reinterpret_cast<const v4u*>(wrow[t] + k + 16);
          }
#pragma unroll
          for (int j = 0; j < 4; ++j) ax[u][j] = *reinterpret_cast<const v4u*>(arow_p + k + 8 * j);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          if (sb + u >= s1) break;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const bf16x8_g af = __builtin_bit_cast(bf16x8_g, ax[u][j]);
#pragma unroll
            for (int t = 0; t < kTiles; ++t) {
              const v4u& wv = j < 2 ? wx[u][t] : wy[u][t];
              const uint2 wq = (j & 1) ? make_uint2(wv[2], wv[3]) : make_uint2(wv[0], wv[1]);
              acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, fp8x8_to_bf16(wq), acc[t], 0, 0, 0);
            }
          }
        }
      }
    }
    if constexpr (!F8A) {
      // K % 128: the remaining 32-element steps, by the last wave.
      if (wave == NW - 1) {
        const uint16_t* arow_p = reinterpret_cast<const uint16_t*>(a.A) + static_cast<size_t>(arow) * a.lda;
        for (int k0 = steps * kStepK; k0 < a.K; k0 += 32) {
          const int k = k0 + 8 * fq;
          const bf16x8_g af = __builtin_bit_cast(bf16x8_g, *reinterpret_cast<const v4u*>(arow_p + k));
#pragma unroll
          for (int t = 0; t < kTiles; ++t)
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                af, fp8x8_to_bf16(*reinterpret_cast<const uint2*>(wrow[t] + k)), acc[t], 0, 0, 0);
        }
      }
    }
    // the quarters summed in wave order: wave 0 + 1 + 2 + 3
    if (wave > 0) {
#pragma unroll
      for (int t = 0; t < kTiles; ++t) s_acc[t][wave - 1][lane] = acc[t];
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int t = 0; t < kTiles; ++t)
#pragma unroll
        for (int w = 0; w < NW - 1; ++w) acc[t] += s_acc[t][w][lane];
      // lane l holds C[4 (l / 16) + i][16 tile + l % 16]
      const int n = tile * 16 + fr;
      const Granite4GemmEpilogue& ep = a.ep;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = 4 * fq + i;
        if (m >= a.M || n >= ncols) continue;
        const size_t off = static_cast<size_t>(m) * ep.ldc + n;
        if constexpr (EPI == kEpiSwiglu) {
          const float g = acc[0][i] * (a_scale * ep.scale0);
          const float u = acc[kTiles - 1][i] * (a_scale * ep.scale1);
          const uint32_t b = pack_bf16_rne(silu_mul(g, u), 0.0f) & 0xffffu;
          ep.out_bf16[off] = static_cast<uint16_t>(b);
          amax = fmaxf(amax, bf16_to_f32(static_cast<uint16_t>(b & 0x7fffu)));
        } else {
          const float y = acc[0][i] * (a_scale * epi_scale(ep, n));
          if (EPI == kEpiF32) {
            ep.out_f32[off] = y;
          } else if (EPI == kEpiResidual) {
            const float r = bf16_to_f32(ep.residual[off]);
            ep.out_bf16[off] = static_cast<uint16_t>(pack_bf16_rne(r + ep.resid_scale * y, 0.0f));
          } else if (a.seg_out[0] != nullptr) {
            const int sg = n < ep.seg1 ? 0 : (n < ep.seg2 ? 1 : 2);
            const int n0 = sg == 0 ? 0 : (sg == 1 ? ep.seg1 : ep.seg2);
            a.seg_out[sg][static_cast<size_t>(m) * a.seg_ld[sg] + n - n0] =
                static_cast<uint16_t>(pack_bf16_rne(y, 0.0f));
          } else {
            ep.out_bf16[off] = static_cast<uint16_t>(pack_bf16_rne(y, 0.0f));
          }
        }
      }
    }
    __syncthreads();  // s_acc is reused by the next tile
  }
  if (EPI == kEpiSwiglu && wave == 0) {
    // only wave 0 stores outputs, so it alone holds the workgroup's max |act|
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
    if (lane == 0) a.partials[blockIdx.x] = amax;
  }
}

constexpr int kSkinnyU = 4;
// Waves per skinny workgroup. Measured on the 40-layer batched decode step
// (FP8 / bf16 ms): 4 waves 8.94-9.20 / 9.38-9.64, 8 waves 8.89-8.90 /
// 9.41, 16 waves 8.96-8.97 / 9.87.
constexpr int kSkinnyWaves = 8;

// Launches the skinny kernel for M <= kSkinnyMaxM; grid: one workgroup per
// 16 output columns, at most `cap` (the partial slots for swiglu).
template <bool F8A, int EPI>
unsigned launch_skinny(const GemmArgs& a, int cap) {
  const int ncols = EPI == kEpiSwiglu ? a.I : a.N;
  const long long ntile = (ncols + 15) / 16;
  const unsigned grid = static_cast<unsigned>(ntile < cap ? ntile : cap);
  hipLaunchKernelGGL((gemm_skinny_kernel<F8A, EPI, kSkinnyU, kSkinnyWaves>), grid, kSkinnyWaves * 64, 0, stream(), a);
  return grid;
}

template <int EPI, int TN = kGBN, int ST = kGStages, int KS = 1>
unsigned gemm_grid(long long tiles, int cap) {
  const int resident =
      resident_blocks(reinterpret_cast<const void*>(gemm_fp8_kernel<EPI, TN, ST, KS>), 256 * KS);
  long long g = tiles;
  if (resident > 0 && g > resident) g = resident;
  if (g > cap) g = cap;
  return static_cast<unsigned>(g > 0 ? g : 1);
}

}  // namespace

// One skinny GEMM (M <= 16) over a weight block of three row segments
// (ep.seg1, ep.seg2 bounds, scale0..2 their scales) with each segment's bf16
// output in a buffer of its own: the batched decode step's q|k|v, whose
// three row blocks the multi-row RoPE append reads. fp8: A is e4m3 codes with
// the device scale a_scale (granite4_gemm_fp8's operands), else bf16
// (granite4_prefill_gemm's). Not exported: layer_steps.hip calls it.
int gemm_rows_split(bool fp8, const void* A, int lda, const float* a_scale, const uint8_t* W,
                    int M, int N, int K, const Granite4GemmEpilogue& ep, uint16_t* const out[3],
                    const int ld[3]) {
  const bool ok = fp8 ? gemm_args_ok(static_cast<const uint8_t*>(A), lda, W, M, N, K) && a_scale != nullptr
                      : (A != nullptr && W != nullptr && K > 0 && K % 32 == 0 && lda >= K && lda % 8 == 0 &&
                         aligned16(A) && aligned16(W));
  if (!ok || M <= 0 || M > kSkinnyMaxM || N <= 0 || ep.seg1 <= 0 || ep.seg2 < ep.seg1 ||
      ep.seg2 > N || out[0] == nullptr || out[1] == nullptr || out[2] == nullptr ||
      ld[0] < ep.seg1 || ld[1] < ep.seg2 - ep.seg1 || ld[2] < N - ep.seg2) {
    std::fprintf(stderr, "granite4: gemm_rows_split: invalid arguments\n");
    return -1;
  }
  GemmArgs a{};
  a.A = static_cast<const uint8_t*>(A);
  a.lda = lda;
  a.a_scale = a_scale;
  a.W = W;
  a.M = M;
  a.N = N;
  a.K = K;
  a.ep = ep;
  for (int i = 0; i < 3; ++i) {
    a.seg_out[i] = out[i];
    a.seg_ld[i] = ld[i];
  }
  if (fp8) launch_skinny<true, kEpiBf16>(a, INT_MAX);
  else launch_skinny<false, kEpiBf16>(a, INT_MAX);
  return launch_status("gemm_rows_split");
}

}  // namespace g4

using namespace g4;

extern "C" {

int granite4_gemm_fp8(int out, const uint8_t* A, int lda, const float* d_a_scale, const uint8_t* W,
                      int M, int N, int K, const Granite4GemmEpilogue* ep) {
  if (!gemm_args_ok(A, lda, W, M, N, K) || ep == nullptr || ep->ldc < N || N % 8 != 0 ||
      ep->ldc % 8 != 0 || !aligned16(ep->out_bf16) || !aligned16(ep->out_f32) ||
      !aligned16(ep->residual) ||
      d_a_scale == nullptr ||
      (out == GRANITE4_GEMM_F32 ? ep->out_f32 == nullptr : ep->out_bf16 == nullptr) ||
      (out == GRANITE4_GEMM_RESIDUAL && ep->residual == nullptr) || out < 0 || out > 2) {
    std::fprintf(stderr,
                 "granite4: granite4_gemm_fp8: invalid arguments (K %% 128 == 0, lda %% 16 == 0, "
                 "N %% 8 == 0, ldc %% 8 == 0, 16-byte aligned outputs)\n");
    return -1;
  }
  GemmArgs a{};
  a.A = A;
  a.lda = lda;
  a.a_scale = d_a_scale;
  a.W = W;
  a.M = M;
  a.N = N;
  a.K = K;
  a.ep = *ep;
  a.mt = (M + kGBM - 1) / kGBM;
  a.vec_out = true;
  // 128 x 64 tiles where 128 x 128 ones would leave CUs idle.
  const bool narrow = static_cast<long long>(a.mt) * ((N + kGBN - 1) / kGBN) < kCUs;
  a.nt = narrow ? (N + 63) / 64 : (N + kGBN - 1) / kGBN;
  const long long tiles = static_cast<long long>(a.mt) * a.nt;
  const hipStream_t st = stream();
  const auto go = [&](auto kern, unsigned grid, int threads = 256) {
    a.xcd_order = gemm_xcd_order(a.mt, grid);
    hipLaunchKernelGGL(kern, grid, threads, 0, st, a);
  };
  // 128 x 64 tiles: six stages where every tile has a CU of its own (one
  // workgroup per CU, 144 KB of LDS), three where two share one (72 KB
  // each), two otherwise.
  const int deep = !narrow ? 2 : (tiles <= kCUs ? 6 : (tiles <= 2 * kCUs ? 3 : 2));
  const auto run = [&](auto e_tag) {
    constexpr int E = decltype(e_tag)::value;
    if (M <= kSkinnyMaxM) launch_skinny<true, E>(a, INT_MAX);
    else if (!narrow) go(gemm_fp8_kernel<E>, gemm_grid<E>(tiles, INT_MAX));
    else if (deep == 6) go(gemm_fp8_kernel<E, 64, 3, 2>, gemm_grid<E, 64, 3, 2>(tiles, INT_MAX), 512);
    else if (deep == 3) go(gemm_fp8_kernel<E, 64, 3>, gemm_grid<E, 64, 3>(tiles, INT_MAX));
    else go(gemm_fp8_kernel<E, 64>, gemm_grid<E, 64>(tiles, INT_MAX));
  };
  switch (out) {
    case GRANITE4_GEMM_BF16: run(std::integral_constant<int, kEpiBf16>{}); break;
    case GRANITE4_GEMM_F32: run(std::integral_constant<int, kEpiF32>{}); break;
    default: run(std::integral_constant<int, kEpiResidual>{}); break;
  }
  return launch_status("granite4_gemm_fp8");
}

int granite4_prefill_gemm(int out, const uint16_t* A, int lda, const uint8_t* W, int M, int N,
                          int K, const Granite4GemmEpilogue* ep, float* ws, size_t ws_bytes) {
  (void)ws;
  (void)ws_bytes;
  // The reference's requirements (prefill_gemm.cu:1264-1271): K % 32 == 0,
  // lda % 8 == 0, even N and ldc, 16-byte aligned A and W.
  if (A == nullptr || W == nullptr || ep == nullptr || M <= 0 || N <= 0 || K <= 0 || K % 32 != 0 ||
      lda % 8 != 0 || lda < K || (N & 1) != 0 || (ep->ldc & 1) != 0 || ep->ldc < N ||
      !aligned16(A) || !aligned16(W) || out < 0 || out > 2 ||
      (out == GRANITE4_GEMM_F32 ? ep->out_f32 == nullptr : ep->out_bf16 == nullptr) ||
      (out == GRANITE4_GEMM_RESIDUAL && ep->residual == nullptr) ||
      static_cast<long long>(M) * lda >= (1LL << 40) ||
      static_cast<long long>(N) * K >= (1LL << 40)) {
    std::fprintf(stderr,
                 "granite4: granite4_prefill_gemm: invalid arguments (K %% 32 == 0, lda %% 8 == 0, "
                 "even N and ldc, 16-byte aligned A and W)\n");
    return -1;
  }
  GemmArgs a{};
  a.A = reinterpret_cast<const uint8_t*>(A);
  a.lda = lda;
  a.W = W;
  a.M = M;
  a.N = N;
  a.K = K;
  a.ep = *ep;
  a.mt = (M + kGBM - 1) / kGBM;
  a.nt = (N + kGBN - 1) / kGBN;
  const void* outp = out == GRANITE4_GEMM_F32 ? static_cast<const void*>(ep->out_f32)
                                              : static_cast<const void*>(ep->out_bf16);
  a.vec_out = N % 8 == 0 && ep->ldc % 8 == 0 && aligned16(outp) &&
              (out != GRANITE4_GEMM_RESIDUAL || aligned16(ep->residual));
  const long long tiles = static_cast<long long>(a.mt) * a.nt;
  const hipStream_t st = stream();
  const auto grid = [&](const void* k) {
    const int resident = resident_blocks(k, 256);
    long long g = tiles;
    if (resident > 0 && g > resident) g = resident;
    const unsigned gu = static_cast<unsigned>(g > 0 ? g : 1);
    a.xcd_order = gemm_xcd_order(a.mt, gu);
    return gu;
  };
  if (M <= kSkinnyMaxM) {
    if (out == GRANITE4_GEMM_BF16) launch_skinny<false, kEpiBf16>(a, INT_MAX);
    else if (out == GRANITE4_GEMM_F32) launch_skinny<false, kEpiF32>(a, INT_MAX);
    else launch_skinny<false, kEpiResidual>(a, INT_MAX);
    return launch_status("granite4_prefill_gemm");
  }
  switch (out) {
    case GRANITE4_GEMM_BF16:
      hipLaunchKernelGGL(gemm_bf16w_kernel<kEpiBf16>,
                         grid(reinterpret_cast<const void*>(gemm_bf16w_kernel<kEpiBf16>)), 256, 0,
                         st, a);
      break;
    case GRANITE4_GEMM_F32:
      hipLaunchKernelGGL(gemm_bf16w_kernel<kEpiF32>,
                         grid(reinterpret_cast<const void*>(gemm_bf16w_kernel<kEpiF32>)), 256, 0, st,
                         a);
      break;
    default: {
      // More tiles than the early-residual form keeps resident: the late form.
      const void* early = reinterpret_cast<const void*>(gemm_bf16w_kernel<kEpiResidual, false>);
      const int resident = resident_blocks(early, 256);
      if (resident > 0 && tiles > resident) {
        const void* late = reinterpret_cast<const void*>(gemm_bf16w_kernel<kEpiResidual, true>);
        hipLaunchKernelGGL((gemm_bf16w_kernel<kEpiResidual, true>), grid(late), 256, 0, st, a);
      } else {
        hipLaunchKernelGGL((gemm_bf16w_kernel<kEpiResidual, false>), grid(early), 256, 0, st, a);
      }
      break;
    }
  }
  return launch_status("granite4_prefill_gemm");
}

size_t granite4_prefill_gemm_workspace_bytes(int M, int N) {
  (void)M;
  (void)N;
  return 0;
}

int granite4_gemm_fp8_swiglu(const uint8_t* A, int lda, const float* d_a_scale,
                             const uint8_t* W_gu, int M, int I, int K, float gate_scale,
                             float up_scale, uint16_t* act, uint8_t* codes, float* d_scale,
                             void* d_work) {
  if (!gemm_args_ok(A, lda, W_gu, M, 2 * I, K) || act == nullptr || I % 8 != 0 || !aligned16(act) ||
      d_a_scale == nullptr || !std::isfinite(gate_scale) || !std::isfinite(up_scale) ||
      d_work == nullptr || (codes != nullptr && d_scale == nullptr) ||
      static_cast<long long>(M) * I >= INT_MAX) {
    std::fprintf(stderr, "granite4: granite4_gemm_fp8_swiglu: invalid arguments\n");
    return -1;
  }
  GemmArgs a{};
  a.A = A;
  a.lda = lda;
  a.a_scale = d_a_scale;
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
  a.vec_out = true;
  a.partials = work_partials(d_work);
  const long long tiles = static_cast<long long>(a.mt) * a.nt;
  unsigned grid;
  if (M <= kSkinnyMaxM) {
    grid = launch_skinny<true, kEpiSwiglu>(a, kMaxPartials);
  } else {
    grid = gemm_grid<kEpiSwiglu>(tiles, kMaxPartials);
    a.xcd_order = gemm_xcd_order(a.mt, grid);
    hipLaunchKernelGGL(gemm_fp8_kernel<kEpiSwiglu>, grid, 256, 0, stream(), a);
  }
  if (launch_status("granite4_gemm_fp8_swiglu") != 0) return -1;
  if (codes == nullptr) return 0;
  return launch_encode_bf16(act, M, I, work_partials(d_work), static_cast<int>(grid), codes, d_scale)
             ? 0
             : -1;
}

int granite4_gemm_fp8_residual_rmsnorm_fp8(const uint8_t* A, int lda, const float* d_a_scale,
                                           const uint8_t* W, int M, int H, int K, float w_scale,
                                           uint16_t* hidden, float resid_scale,
                                           const uint16_t* gamma, float eps, uint8_t* codes,
                                           float* d_scale, void* d_work) {
  if (hidden == nullptr || gamma == nullptr || codes == nullptr || d_scale == nullptr ||
      d_work == nullptr || !std::isfinite(w_scale) || !std::isfinite(resid_scale)) {
    std::fprintf(stderr, "granite4: granite4_gemm_fp8_residual_rmsnorm_fp8: invalid arguments\n");
    return -1;
  }
  Granite4GemmEpilogue ep{};
  ep.scale0 = ep.scale1 = ep.scale2 = w_scale;
  ep.seg1 = ep.seg2 = H;
  ep.out_bf16 = hidden;
  ep.residual = hidden;
  ep.resid_scale = resid_scale;
  ep.ldc = H;
  if (granite4_gemm_fp8(GRANITE4_GEMM_RESIDUAL, A, lda, d_a_scale, W, M, H, K, &ep) != 0) return -1;
  // The norm reads only the updated residual (no branch): 2 B read + 1 B
  // written per element after the GEMM's in-place 2 B + 2 B.
  return granite4_add_rmsnorm_fp8(hidden, nullptr, 1.0f, gamma, eps, M, H, nullptr, codes, d_scale,
                                  d_work);
}

}  // extern "C"
