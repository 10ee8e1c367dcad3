// norm.hip - fused residual add + RMSNorm for gfx950, with bf16 or FP8 e4m3
// output.
//
// Arithmetic (bit-for-bit the reference's, kernels_phase2.cu:51-132 and the
// residual epilogue forward_gpu.cu:992-994):
//   x      = bf16(float(res) + mult * float(branch))        (two roundings, no FMA)
//   r      = 1 / sqrt(float(sum(x^2) in double / cols) + eps)
//   y      = bf16((x * r) * w)
// Each x^2 of a bf16 value is exact in f32; the row sum is accumulated in f64
// per lane, then reduced across lanes with DPP (g4_wave.h) and across the
// row's waves through LDS in a fixed order.
//
// Layout: one row is 4096 bf16 = 512 16-byte vectors. WPR waves share a row
// (WPR = 1: 8 vectors per lane held in VGPRs; WPR = 4: 2 per lane) and a
// 256-thread workgroup holds 4 / WPR rows. Every wave-wide load is 1 KiB
// contiguous. All loads of a lane (x, branch, gamma) are issued before any
// store, so an in-place residual (res_out == res) does not serialise them.
//
// FP8 output (granite4_add_rmsnorm_fp8): the per-tensor scale depends on the
// maximum over the whole [rows][cols] tensor, so two launches run back to
// back. Pass 1 writes res' and one partial max |y| per workgroup into the
// workspace (plain stores to distinct addresses: no same-address atomics,
// which serialise across the 8 XCDs); its grid is capped at kMaxPartials
// workgroups that loop over row groups. Pass 2 reduces the partials, re-reads
// res' (2 B / element, usually still in the 256 MB Infinity Cache),
// recomputes r and y exactly as pass 1 did, and writes the codes.
#include "g4_common.h"
#include "g4_hw.h"
#include "g4_math.h"
#include "g4_sync.h"
#include "g4_wave.h"
#include "granite4_layerops.h"

#include <cstdlib>
#include <mutex>
#include <type_traits>

static_assert(g4::kMaxPartials == GRANITE4_FP8_MAX_PARTIALS, "workspace layout");
static_assert(GRANITE4_FP8_WORK_BYTES(0) == g4::kWorkRowOff, "workspace layout");
static_assert(g4::kMaxPartials <= g4::kBlock * g4::kSyncSlotsPerThread,
              "grid_max: workgroup 0 polls every slot of the largest grid");

namespace g4 {
namespace {

typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));

enum : int { kOutBf16 = 0, kOutAmax = 1, kOutFp8 = 2 };

struct NormArgs {
  const uint16_t* x;       // residual stream (or the plain RMSNorm input)
  const uint16_t* branch;  // NULL: no residual add
  float mult;
  const uint16_t* w;
  float eps;
  int rows, cols;
  uint16_t* res_out;  // NULL: res' not stored
  uint16_t* normed;   // kOutBf16
  uint8_t* codes;     // kOutFp8
  float* scale_out;   // kOutFp8
  float* partials;    // kOutAmax writes [gridDim.x]; kOutFp8 reads [n_partials]
  int n_partials;
  float* row_r;       // kOutAmax writes each row's 1 / rms, the encode pass reads it
  double inv_nvec;    // 1 / (cols / 8)
};

__device__ __forceinline__ Fp8Enc fp8_scale_of(float amax) { return fp8_enc_of(fp8_scale_for(amax)); }

// The lane's share of one row of a row group (4 / WPR rows per 256-thread
// workgroup): res' (x + mult * branch, bf16; stored when res_out is given),
// the gamma vectors, and the row's r = 1 / rms. Every thread of the
// workgroup must call it (it synchronises when WPR > 1).
template <int VPL, int WPR>
struct NormRow {
  V8 xv[VPL], wv[VPL], bv[VPL];
  bool ok[VPL];
  size_t base;
  int row, part, lane;
  bool live;
  float r;
};

// First half of norm_row_front: the row's indices and its loads (x, branch,
// gamma).
template <int VPL, int WPR>
__device__ __forceinline__ void norm_row_load(const NormArgs& a, int rg, NormRow<VPL, WPR>& t) {
  constexpr int RPB = 4 / WPR;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int row = rg * RPB + wave / WPR;
  const int part = wave % WPR;
  const bool live = row < a.rows;
  const int nvec = a.cols >> 3;
  const size_t base = live ? static_cast<size_t>(row) * static_cast<size_t>(a.cols) : 0;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int vi = (j * WPR + part) * 64 + lane;
    t.ok[j] = live && vi < nvec;
    t.xv[j] = V8{{0u, 0u, 0u, 0u}};
    t.bv[j] = V8{{0u, 0u, 0u, 0u}};
    t.wv[j] = V8{{0u, 0u, 0u, 0u}};
    if (t.ok[j]) {
      // x and branch stream; res' goes out through the caches, where the FP8
      // op's encode pass re-reads it.
      t.xv[j] = ld8_nt(a.x + base + 8 * vi);
      if (a.branch != nullptr) t.bv[j] = ld8_nt(a.branch + base + 8 * vi);
      t.wv[j] = ld8(a.w + 8 * vi);
    }
  }
  t.base = base;
  t.row = row;
  t.part = part;
  t.lane = lane;
  t.live = live;
}

// Second half: res' = x + mult * branch (bf16; stored when res_out is given)
// and the row's r = 1 / rms. Every thread of the workgroup must call it (it
// synchronises when WPR > 1).
// NT_RES: res' stored non-temporally (a single-launch form never reads it
// back; the two-launch form's encode pass does, through the caches).
template <int VPL, int WPR, bool NT_RES = false>
__device__ __forceinline__ void norm_row_finish(const NormArgs& a, NormRow<VPL, WPR>& t) {
  const int wave = threadIdx.x >> 6;
  double ss = 0.0;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    if (a.branch != nullptr) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float lo = lo_bf16(t.xv[j].w[e]) + a.mult * lo_bf16(t.bv[j].w[e]);
        const float hi = hi_bf16(t.xv[j].w[e]) + a.mult * hi_bf16(t.bv[j].w[e]);
        t.xv[j].w[e] = pack_bf16_hw(lo, hi);
      }
      if (t.ok[j] && a.res_out != nullptr) {
        const int vi = (j * WPR + t.part) * 64 + t.lane;
        if (NT_RES) st8_nt(a.res_out + t.base + 8 * vi, t.xv[j]);
        else st8(a.res_out + t.base + 8 * vi, t.xv[j]);
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float lo = lo_bf16(t.xv[j].w[e]), hi = hi_bf16(t.xv[j].w[e]);
      ss += static_cast<double>(lo * lo);
      ss += static_cast<double>(hi * hi);
    }
  }
  ss = wave_sum(ss);
  if (WPR > 1) {
    __shared__ double s_part[kBlock / 64];
    if (t.lane == 0) s_part[wave] = ss;
    __syncthreads();
    const int w0 = (wave / WPR) * WPR;
    ss = s_part[w0];
#pragma unroll
    for (int k = 1; k < WPR; ++k) ss += s_part[w0 + k];
    __syncthreads();  // s_part is reused by the next row group
  }
  t.r = 1.0f / sqrtf(static_cast<float>(ss / a.cols) + a.eps);
}

// The lane's share of one row of a row group (4 / WPR rows per 256-thread
// workgroup): res', the gamma vectors, and the row's r = 1 / rms.
template <int VPL, int WPR, bool NT_RES = false>
__device__ __forceinline__ void norm_row_front(const NormArgs& a, int rg, NormRow<VPL, WPR>& t) {
  norm_row_load<VPL, WPR>(a, rg, t);
  norm_row_finish<VPL, WPR, NT_RES>(a, t);
}

// One row group of the workgroup; MODE kOutAmax folds into *m.
template <int VPL, int WPR, int MODE>
__device__ __forceinline__ void norm_rows(const NormArgs& a, int rg, const Fp8Enc& f, float* m_acc) {
  NormRow<VPL, WPR> t;
  norm_row_front<VPL, WPR>(a, rg, t);
  const V8 (&xv)[VPL] = t.xv;
  const V8 (&wv)[VPL] = t.wv;
  const bool (&ok)[VPL] = t.ok;
  const size_t base = t.base;
  const int row = t.row, part = t.part, lane = t.lane;
  const bool live = t.live;
  const float r = t.r;
  if (MODE == kOutAmax && live && part == 0 && lane == 0) a.row_r[row] = r;

  if (MODE == kOutBf16) {
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      if (!ok[j]) continue;
      V8 y;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        y.w[e] = pack_bf16_hw(lo_bf16(xv[j].w[e]) * r * lo_bf16(wv[j].w[e]),
                              hi_bf16(xv[j].w[e]) * r * hi_bf16(wv[j].w[e]));
      const int vi = (j * WPR + part) * 64 + lane;
      st8_nt(a.normed + base + 8 * vi, y);
    }
    return;
  }
  if (MODE == kOutAmax) {
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t y = pack_bf16_hw(lo_bf16(xv[j].w[e]) * r * lo_bf16(wv[j].w[e]),
                                        hi_bf16(xv[j].w[e]) * r * hi_bf16(wv[j].w[e]));
        m = fmaxf(m, lo_bf16(y & 0x7fff7fffu));
        m = fmaxf(m, hi_bf16(y & 0x7fff7fffu));
      }
    }
    *m_acc = fmaxf(*m_acc, m);
    return;
  }
  // kOutFp8
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    if (!ok[j]) continue;
    uint32_t c[2] = {0u, 0u};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t y = pack_bf16_hw(lo_bf16(xv[j].w[e]) * r * lo_bf16(wv[j].w[e]),
                                      hi_bf16(xv[j].w[e]) * r * hi_bf16(wv[j].w[e]));
      const uint32_t pair = fp8x2_encode_scaled(lo_bf16(y), hi_bf16(y), f.s, f.inv, f.fast);
      c[e >> 1] |= pair << (16 * (e & 1));
    }
    const int vi = (j * WPR + part) * 64 + lane;
    st_u32x2_nt(a.codes + base + 8 * vi, c[0], c[1]);
  }
}

template <int VPL, int WPR, int MODE>
__global__ __launch_bounds__(kBlock) void norm_kernel(NormArgs a) {
  // The arguments of the row loads fetched in one scalar round trip.
  asm volatile("" ::"s"(a.x), "s"(a.branch), "s"(a.w), "s"(a.rows), "s"(a.cols), "s"(a.mult),
               "s"(a.res_out), "s"(a.normed), "s"(a.eps));
  constexpr int RPB = 4 / WPR;
  const int nrg = (a.rows + RPB - 1) / RPB;
  Fp8Enc f = fp8_enc_of(0.0f);
  if (MODE == kOutFp8) {
    f = fp8_scale_of(reduce_partials(a.partials, a.n_partials));
    if (blockIdx.x == 0 && threadIdx.x == 0) *a.scale_out = f.s;
  }
  float m = 0.0f;
  for (int rg = blockIdx.x; rg < nrg; rg += gridDim.x) norm_rows<VPL, WPR, MODE>(a, rg, f, &m);
  if (MODE == kOutAmax) write_partial(a.partials, m);
}

// FP8 pass 2 of the vector path: element-wise over [rows][cols / 8] vectors.
// Each row's 1 / rms comes from pass 1 (row_r), so y = bf16((x * r) * w) is
// recomputed bit-identically without a row reduction, and the pass streams
// at full occupancy. x is re-read with cached loads: pass 1 wrote it just
// before (it is usually still in the Infinity Cache).
struct NormEncRaw {
  V8 x, b, w;
  float r;
};

__global__ __launch_bounds__(kBlock) void norm_encode_kernel(NormArgs a) {
  const int nvec = a.cols >> 3;
  const auto load = [&](int v) {
    NormEncRaw t;
    const int row = div_fast(v, nvec, a.inv_nvec);
    const size_t off = 8ull * static_cast<unsigned>(v);
    t.x = ld8(a.x + off);
    if (a.branch != nullptr) t.b = ld8_nt(a.branch + off);
    t.w = ld8(a.w + 8 * (v - row * nvec));
    t.r = a.row_r[row];
    return t;
  };
  auto sw = sweep_begin<4>(a.rows * nvec, load);
  // The partials' reduction overlaps the first loads.
  const Fp8Enc f = fp8_scale_of(reduce_partials(a.partials, a.n_partials));
  if (blockIdx.x == 0 && threadIdx.x == 0) *a.scale_out = f.s;
  const auto body = [&](auto fast_tag) {
    return [&, fast_tag](int v, const NormEncRaw& t) {
      uint32_t x[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) x[e] = t.x.w[e];
      if (a.branch != nullptr) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          x[e] = pack_bf16_hw(lo_bf16(x[e]) + a.mult * lo_bf16(t.b.w[e]),
                              hi_bf16(x[e]) + a.mult * hi_bf16(t.b.w[e]));
      }
      uint32_t y[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        y[e] = pack_bf16_hw(lo_bf16(x[e]) * t.r * lo_bf16(t.w.w[e]),
                            hi_bf16(x[e]) * t.r * hi_bf16(t.w.w[e]));
      const uint2 c = fp8x8_encode_bf16<decltype(fast_tag)::value>(y, f);
      st_u32x2_nt(a.codes + 8ull * static_cast<unsigned>(v), c.x, c.y);
    };
  };
  if (f.fast) sweep_run(sw, load, body(std::true_type{}));
  else sweep_run(sw, load, body(std::false_type{}));
}

// Any-shape fallback: one workgroup per row, element loops, two passes over
// the row (the second re-reads it from cache). Same arithmetic and reduction
// order as above at the wave level.
template <int MODE>
__device__ void norm_generic_row(const NormArgs& a, int row, const Fp8Enc& f, float* m_acc) {
  const size_t base = static_cast<size_t>(row) * static_cast<size_t>(a.cols);
  auto load_x = [&](int c) {
    const float x = bf16_to_f32(a.x[base + c]);
    if (a.branch == nullptr) return x;
    return bf16_to_f32(f32_to_bf16(x + a.mult * bf16_to_f32(a.branch[base + c])));
  };
  double ss = 0.0;
  for (int c = threadIdx.x; c < a.cols; c += kBlock) {
    const float x = load_x(c);
    if (a.branch != nullptr && a.res_out != nullptr) a.res_out[base + c] = f32_to_bf16(x);
    ss += static_cast<double>(x * x);
  }
  __shared__ double s_part[kBlock / 64];
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) s_part[threadIdx.x >> 6] = ss;
  __syncthreads();
  ss = (s_part[0] + s_part[1]) + (s_part[2] + s_part[3]);
  __syncthreads();
  const float r = 1.0f / sqrtf(static_cast<float>(ss / a.cols) + a.eps);
  // The same thread reads back what it wrote above, so res_out aliasing res
  // needs no extra barrier: recompute from the inputs when res' was not stored.
  auto x_again = [&](int c) {
    if (a.branch != nullptr && a.res_out != nullptr) return bf16_to_f32(a.res_out[base + c]);
    return load_x(c);
  };
  if (MODE == kOutBf16) {
    for (int c = threadIdx.x; c < a.cols; c += kBlock)
      a.normed[base + c] = static_cast<uint16_t>(f32_to_bf16(x_again(c) * r * bf16_to_f32(a.w[c])));
    return;
  }
  if (MODE == kOutAmax) {
    float m = 0.0f;
    for (int c = threadIdx.x; c < a.cols; c += kBlock)
      m = fmaxf(m, bf16_to_f32(f32_to_bf16(x_again(c) * r * bf16_to_f32(a.w[c])) & 0x7fffu));
    *m_acc = fmaxf(*m_acc, m);
    return;
  }
  for (int c = threadIdx.x; c < a.cols; c += kBlock) {
    const float y = bf16_to_f32(f32_to_bf16(x_again(c) * r * bf16_to_f32(a.w[c])));
    a.codes[base + c] = static_cast<uint8_t>(fp8_encode_scaled(y, f.s, f.inv, f.fast));
  }
}

template <int MODE>
__global__ __launch_bounds__(kBlock) void norm_generic_kernel(NormArgs a) {
  Fp8Enc f = fp8_enc_of(0.0f);
  if (MODE == kOutFp8) {
    f = fp8_scale_of(reduce_partials(a.partials, a.n_partials));
    if (blockIdx.x == 0 && threadIdx.x == 0) *a.scale_out = f.s;
  }
  float m = 0.0f;
  for (int row = blockIdx.x; row < a.rows; row += gridDim.x) norm_generic_row<MODE>(a, row, f, &m);
  if (MODE == kOutAmax) write_partial(a.partials, m);
}

// Row held in slot h by this workgroup, or -1. In round h the grid takes
// rows h * grid + blockIdx.x. When the rows are n >= 2 full rounds of a grid
// of a multiple of 4 workgroups (and a slot is left), the last round is
// weighted by the workgroup's age on its CU: the dispatcher fills each CU with
// workgroups b, b + grid / 4, b + grid / 2, b + 3 grid / 4, and the SIMD
// arbiter favours the oldest waves, so (measured at 8192 rows on 1024
// workgroups) the oldest quarter loads its rows ~12 % faster than the mean and
// the youngest ~12 % slower. Quarter 3 then holds n - 1 rows, quarters 1 and 2
// n, quarter 0 n + 1: round n - 1 covers the first three quarters, round n
// the first. Measured at T=8192 (three rounds, one box): 54.5-55.0 ->
// 53.4-53.6 us.
__device__ __forceinline__ int norm_held_row(int rows, int slots, int h) {
  const int G = gridDim.x, b = blockIdx.x;
  const int n = rows / G;
  if (G % 4 == 0 && n >= 2 && n * G == rows && n + 1 <= slots) {
    const int q = G / 4;
    if (h < n - 1) return h * G + b;
    if (h == n - 1) return b < 3 * q ? (n - 1) * G + b : -1;
    if (h == n) return b < q ? (n - 1) * G + 3 * q + b : -1;
    return -1;
  }
  const int r = b + h * G;
  return r < rows ? r : -1;
}

// Single-launch FP8 form for tensors that fit one resident grid: each
// 256-thread workgroup (four waves per row, as the two-launch form's first
// pass, so y and the amax are bit-identical to it) holds up to HR rows'
// y = bf16(res' * r * w) in VGPRs and HL more in LDS, the workgroups agree on
// max |y| with one grid synchronisation, and each encodes what it holds. HBM
// traffic: x (+ branch) read once, res' and codes written once, against a
// second read of res' in the two-launch form, and one launch instead of two.
template <int VPL, int HR, int HL>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(VPL >= 4 ? 1 : 4)))
void norm_fp8_fused_kernel(NormArgs a, GridSync gs) {
  static_assert(kBlock == kSyncThreads, "grid_max assumes kSyncThreads-thread workgroups");
  // Every argument of the first loads fetched in one scalar round trip.
  asm volatile("" ::"s"(a.x), "s"(a.branch), "s"(a.w), "s"(a.rows), "s"(a.cols), "s"(a.mult),
               "s"(a.res_out), "s"(a.eps), "s"(gs.gen), "s"(gs.slots), "s"(gs.result),
               "s"(gs.blocks));
  __shared__ uint4 s_y[HL > 0 ? HL : 1][VPL][kBlock];
  G4_TRACE_MARK(gs, 0);
  const unsigned tag = grid_sync_tag(gs);
  V8 y[HR > 0 ? HR : 1][VPL];
  // max |y| on the bf16 bit patterns, two per v_pk_max_u16 (for
  // non-negative bf16 values the unsigned order of the patterns is the
  // numeric order); a lane that saw a NaN pattern (above 0x7f80 once the
  // sign is cleared) recomputes its maximum with fmaxf, which skips NaN.
  u16x2_t mk = {0, 0};
  const auto row_of = [&](int h) { return norm_held_row(a.rows, HR + HL, h); };
#pragma unroll
  for (int h = 0; h < HR + HL; ++h) {
    const int rg = row_of(h);  // uniform over the workgroup
    if (rg < 0) break;
    NormRow<VPL, 4> t;
    norm_row_front<VPL, 4, true>(a, rg, t);
    if (h == 0) G4_TRACE_MARK(gs, 1);
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      V8 yv;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        yv.w[e] = pack_bf16_hw(lo_bf16(t.xv[j].w[e]) * t.r * lo_bf16(t.wv[j].w[e]),
                               hi_bf16(t.xv[j].w[e]) * t.r * hi_bf16(t.wv[j].w[e]));
        // lanes past the row's end hold zeros (x and w load as 0)
        mk = __builtin_elementwise_max(mk, __builtin_bit_cast(u16x2_t, yv.w[e] & 0x7fff7fffu));
      }
      if (h < HR) y[h < HR ? h : 0][j] = yv;
      else s_y[h >= HR ? h - HR : 0][j][threadIdx.x] = make_uint4(yv.w[0], yv.w[1], yv.w[2], yv.w[3]);
    }
  }
  const uint32_t mb = mk[0] > mk[1] ? mk[0] : mk[1];
  float m = __uint_as_float(mb << 16);
  if (__builtin_expect(mb > 0x7f80u, 0)) {
    m = 0.0f;
#pragma unroll
    for (int h = 0; h < HR + HL; ++h) {
      if (row_of(h) < 0) break;
#pragma unroll
      for (int j = 0; j < VPL; ++j) {
        uint32_t w4[4];
        if (h < HR) {
#pragma unroll
          for (int e = 0; e < 4; ++e) w4[e] = y[h < HR ? h : 0][j].w[e];
        } else {
          const uint4 q = s_y[h >= HR ? h - HR : 0][j][threadIdx.x];
          w4[0] = q.x;
          w4[1] = q.y;
          w4[2] = q.z;
          w4[3] = q.w;
        }
#pragma unroll
        for (int e = 0; e < 4; ++e)
          m = fmaxf(m, fmaxf(lo_bf16(w4[e] & 0x7fff7fffu), hi_bf16(w4[e] & 0x7fff7fffu)));
      }
    }
  }
  G4_TRACE_MARK(gs, 2);
  const Fp8Enc f = fp8_scale_of(grid_max(m, gs, tag));
  G4_TRACE_MARK(gs, 3);
  if (blockIdx.x == 0 && threadIdx.x == 0) *a.scale_out = f.s;
  const int part = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int nvec = a.cols >> 3;
  const auto encode = [&](auto fast_tag) {
#pragma unroll
    for (int h = 0; h < HR + HL; ++h) {
      const int rg = row_of(h);
      if (rg < 0) break;
      const size_t base = static_cast<size_t>(rg) * static_cast<size_t>(a.cols);
#pragma unroll
      for (int j = 0; j < VPL; ++j) {
        const int vi = (j * 4 + part) * 64 + lane;
        if (vi >= nvec) continue;
        V8 yv;
        if (h < HR) {
          yv = y[h < HR ? h : 0][j];
        } else {
          const uint4 q = s_y[h >= HR ? h - HR : 0][j][threadIdx.x];
          yv = V8{{q.x, q.y, q.z, q.w}};
        }
        const uint2 c = fp8x8_encode_bf16<decltype(fast_tag)::value>(yv.w, f);
        st_u32x2_nt(a.codes + base + 8 * vi, c.x, c.y);
      }
    }
  };
  if (f.fast) encode(std::true_type{});
  else encode(std::false_type{});
  G4_TRACE_MARK(gs, 4);
}

// Held rows per workgroup of the two single-launch forms: VGPRs only, and
// VGPRs + LDS for row counts beyond the first's reach.
#ifndef G4_NORM_DEEP_HR
#define G4_NORM_DEEP_HR 8
#endif
#ifndef G4_NORM_DEEP_HL
#define G4_NORM_DEEP_HL 4
#endif
constexpr int kNormHold = 4;
constexpr int kNormDeepHR = G4_NORM_DEEP_HR;
constexpr int kNormDeepHL = G4_NORM_DEEP_HL;

// Waves per row. Four waves per 4096-wide row (2 vectors per lane, 54-62
// VGPRs, full occupancy) measured faster than one wave per row (8 vectors per
// lane, 142-152 VGPRs, 3 waves per SIMD) at every size: T=8192 FP8 70 vs 76 µs,
// T=32768 bf16 stress 5.62 vs 5.52 TB/s. Every width the vector path takes
// (nvec <= 512) runs four waves per row.

// Grid of a norm launch: one workgroup per row group, capped at kMaxPartials
// for the FP8 passes (their workgroups loop over row groups).
unsigned norm_grid(int MODE, int row_groups) {
  if (MODE == kOutBf16) return static_cast<unsigned>(row_groups);
  return static_cast<unsigned>(row_groups < kMaxPartials ? row_groups : kMaxPartials);
}

// Whether the row-vector kernels (and the element-wise FP8 encode pass) take
// this shape; otherwise the any-shape fallback runs.
bool norm_vector_path(int rows, int cols) {
  return cols % 8 == 0 && cols / 8 <= 8 * 64 && static_cast<long long>(rows) * cols < INT_MAX;
}

template <int MODE>
int launch_norm(NormArgs& a, const char* what) {
  const int nvec = a.cols / 8;
  const bool vec = norm_vector_path(a.rows, a.cols);
  const hipStream_t st = stream();
  if (MODE == kOutFp8 && vec) {
    a.inv_nvec = 1.0 / nvec;
    const long long vectors = static_cast<long long>(a.rows) * nvec;
    const long long want = (vectors + 4LL * kBlock - 1) / (4LL * kBlock);
    const unsigned grid = static_cast<unsigned>(want < kPersistBlocks ? want : kPersistBlocks);
    hipLaunchKernelGGL(norm_encode_kernel, grid, kBlock, 0, st, a);
  } else if (vec) {
    const unsigned grid = norm_grid(MODE, a.rows);
    if (MODE == kOutAmax) a.n_partials = static_cast<int>(grid);
    if (nvec <= 256) hipLaunchKernelGGL((norm_kernel<1, 4, MODE>), grid, kBlock, 0, st, a);
    else if (nvec <= 512) hipLaunchKernelGGL((norm_kernel<2, 4, MODE>), grid, kBlock, 0, st, a);
    else hipLaunchKernelGGL((norm_kernel<4, 4, MODE>), grid, kBlock, 0, st, a);
  } else {
    const unsigned grid = norm_grid(MODE, a.rows);
    if (MODE == kOutAmax) a.n_partials = static_cast<int>(grid);
    hipLaunchKernelGGL((norm_generic_kernel<MODE>), grid, kBlock, 0, st, a);
  }
  return launch_status(what);
}

// Launches norm_fp8_fused_kernel<VPL, HR, HL> for the row width when every
// row fits the resident grid's holds; false (nothing launched) otherwise.
template <int HR, int HL>
bool launch_fused_vpl(const NormArgs& a, const GridSync& gs, int nvec) {
  const auto go = [&](auto kern) {
    const int resident = resident_blocks(reinterpret_cast<const void*>(kern), kBlock);
    const int cap = resident < kMaxPartials ? resident : kMaxPartials;
    if (cap <= 0 || a.rows > static_cast<long long>(cap) * (HR + HL)) return false;
    const unsigned grid = static_cast<unsigned>(a.rows < cap ? a.rows : cap);
    GridSync g = gs;
    g.blocks = static_cast<int>(grid);
    launch_grid_sync(kern, grid, kBlock, stream(), a, g);
    return true;
  };
  if (nvec <= 256) return go(norm_fp8_fused_kernel<1, HR, HL>);
  if (nvec <= 512) return go(norm_fp8_fused_kernel<2, HR, HL>);
  return go(norm_fp8_fused_kernel<4, HR, HL>);
}

// Launches the single-launch FP8 form when the shape takes the four-waves-
// per-row vector path (as the two-launch form would) and the rows fit the
// resident grid; returns false (nothing launched) otherwise.
bool launch_norm_fp8_fused(const uint16_t* x, const uint16_t* branch, float mult, const uint16_t* w,
                           float eps, int rows, int cols, uint16_t* res_out, uint8_t* codes,
                           float* scale, void* work) {
  const int nvec = cols / 8;
  if (fp8_launch_mode() == 1 || !norm_vector_path(rows, cols))
    return false;
  NormArgs a{x, branch, mult, w, eps, rows, cols, res_out, nullptr, codes, scale, nullptr, 0,
             nullptr, 0.0};
  const GridSync gs{work_slots(work), work_gen(work), work_result(work), 0, work_err(work),
                    fp8_sync_spin_limit()};
  return launch_fused_vpl<kNormHold, 0>(a, gs, nvec) ||
         launch_fused_vpl<kNormDeepHR, kNormDeepHL>(a, gs, nvec);
}

bool norm_args_ok(const void* x, const void* w, float eps, int rows, int cols) {
  return x != nullptr && w != nullptr && std::isfinite(eps) && eps >= 0.0f && rows > 0 &&
         cols > 0 && fits_int(static_cast<long long>(rows) * cols);
}

int rmsnorm_ref_api(const uint16_t* d_x, const uint16_t* d_w, float eps, int rows, int cols,
                    uint16_t* d_out, int max_rows, const char* what) {
  // kernels_phase2.cu:910-936: eps must be finite and > 0.
  if (!norm_args_ok(d_x, d_w, eps, rows, cols) || eps <= 0.0f || d_out == nullptr ||
      rows > max_rows) {
    std::fprintf(stderr, "granite4: %s: invalid arguments\n", what);
    return -1;
  }
  NormArgs a{d_x, nullptr, 1.0f, d_w, eps, rows, cols, nullptr, d_out, nullptr, nullptr, nullptr, 0, nullptr, 0.0};
  return launch_norm<kOutBf16>(a, what);
}

int add_rmsnorm_fp8_impl(const uint16_t* d_res, const uint16_t* d_branch, float resid_mult,
                         const uint16_t* d_w, float eps, int rows, int cols, uint16_t* d_res_out,
                         uint8_t* d_codes, float* d_scale, void* d_work, const char* what) {
  if (!norm_args_ok(d_res, d_w, eps, rows, cols) || !std::isfinite(resid_mult) ||
      d_codes == nullptr || d_scale == nullptr || d_work == nullptr) {
    std::fprintf(stderr, "granite4: %s: invalid arguments\n", what);
    return -1;
  }
  uint16_t* res_out = d_branch != nullptr ? d_res_out : nullptr;
  if (launch_norm_fp8_fused(d_res, d_branch, resid_mult, d_w, eps, rows, cols, res_out, d_codes,
                            d_scale, d_work))
    return launch_status(what);
  NormArgs p1{d_res, d_branch, resid_mult, d_w, eps, rows, cols,
              res_out, nullptr, nullptr, nullptr, work_partials(d_work), 0,
              work_row_r(d_work), 0.0};
  if (launch_norm<kOutAmax>(p1, "granite4_add_rmsnorm_fp8 (amax)") != 0) return -1;
  // Pass 2 reads the stored residual when there is one (it may alias d_res).
  NormArgs p2 = p1;
  if (res_out != nullptr) {
    p2.x = res_out;
    p2.branch = nullptr;
  }
  p2.res_out = nullptr;
  p2.codes = d_codes;
  p2.scale_out = d_scale;
  return launch_norm<kOutFp8>(p2, "granite4_add_rmsnorm_fp8 (encode)");
}

}  // namespace

// ---------------------------------------------------------------------------
// Static scratch for granite4_add_rmsnorm_fp8_noalloc: the FP8 workspace
// (partials, synchronisation slots, generation / error / result words, one
// f32 1 / rms per row) for up to kNoAllocMaxRows rows, in device memory the
// code object reserves, so the entry point never allocates. Each GPU holds
// its own copy (at its own address) until the process ends; every call on a
// GPU shares it, so calls that overlap on one GPU race.
constexpr int kNoAllocMaxRows = 65536;
constexpr size_t kNoAllocScratchBytes = kWorkRowOff + 4u * kNoAllocMaxRows;  // 274,688 B
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;

// The device address of the current device's `scratch` (the host-side name
// is only a stand-in), looked up once per device with that device current.
// Nothing is launched: the array is zero-initialised when the code object is
// loaded onto the device, which is the start state the synchronisation area
// needs (slots, generation and error word), so a first use under graph
// capture records no clearing node. The per-row and partial areas need no
// clearing: each call writes them before reading them. nullptr (with a
// message) on failure.
void* static_scratch(const char* what) {
  static std::mutex mu;
  static void* ptrs[kMaxDevices] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    (void)hipGetLastError();
    std::fprintf(stderr, "granite4: %s: no usable current device\n", what);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (ptrs[dev] != nullptr) return ptrs[dev];
  void* ptr = nullptr;
  const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess || ptr == nullptr) {
    (void)hipGetLastError();
    std::fprintf(stderr, "granite4: %s: hipGetSymbolAddress(scratch) failed: %s\n", what,
                 hipGetErrorString(e));
    return nullptr;
  }
  ptrs[dev] = ptr;
  return ptr;
}

}  // namespace g4

using namespace g4;

extern "C" {

int granite4_kernel_rmsnorm(const uint16_t* d_x, const uint16_t* d_w, float eps, int rows,
                            int cols, uint16_t* d_out) {
  return rmsnorm_ref_api(d_x, d_w, eps, rows, cols, d_out, INT_MAX, "granite4_kernel_rmsnorm");
}

int granite4_kernel_rmsnorm_batched(const uint16_t* d_x, const uint16_t* d_w, float eps,
                                    int rows, int cols, uint16_t* d_out) {
  return rmsnorm_ref_api(d_x, d_w, eps, rows, cols, d_out, kMaxVerifyRows,
                         "granite4_kernel_rmsnorm_batched");
}

int granite4_add_rmsnorm(const uint16_t* d_res, const uint16_t* d_branch, float resid_mult,
                         const uint16_t* d_w, float eps, int rows, int cols, uint16_t* d_res_out,
                         uint16_t* d_normed) {
  if (!norm_args_ok(d_res, d_w, eps, rows, cols) || !std::isfinite(resid_mult) ||
      d_normed == nullptr) {
    std::fprintf(stderr, "granite4: granite4_add_rmsnorm: invalid arguments\n");
    return -1;
  }
  NormArgs a{d_res, d_branch, resid_mult, d_w, eps, rows, cols,
             d_branch != nullptr ? d_res_out : nullptr, d_normed, nullptr, nullptr, nullptr, 0, nullptr,
             0.0};
  return launch_norm<kOutBf16>(a, "granite4_add_rmsnorm");
}

int granite4_add_rmsnorm_fp8(const uint16_t* d_res, const uint16_t* d_branch, float resid_mult,
                             const uint16_t* d_w, float eps, int rows, int cols,
                             uint16_t* d_res_out, uint8_t* d_codes, float* d_scale,
                             void* d_work) {
  return add_rmsnorm_fp8_impl(d_res, d_branch, resid_mult, d_w, eps, rows, cols, d_res_out, d_codes,
                              d_scale, d_work, "granite4_add_rmsnorm_fp8");
}

int granite4_add_rmsnorm_fp8_noalloc(const uint16_t* d_res, const uint16_t* d_branch,
                                     float resid_mult, const uint16_t* d_w, float eps, int rows,
                                     int cols, uint16_t* d_res_out, uint8_t* d_codes,
                                     float* d_scale) {
  if (rows > kNoAllocMaxRows) {
    std::fprintf(stderr,
                 "granite4: granite4_add_rmsnorm_fp8_noalloc: %d rows exceed the static "
                 "scratch's maximum of %d (use granite4_add_rmsnorm_fp8 with a workspace)\n",
                 rows, kNoAllocMaxRows);
    return -1;
  }
  void* work = static_scratch("granite4_add_rmsnorm_fp8_noalloc");
  if (work == nullptr) return -1;
  return add_rmsnorm_fp8_impl(d_res, d_branch, resid_mult, d_w, eps, rows, cols, d_res_out, d_codes,
                              d_scale, work, "granite4_add_rmsnorm_fp8_noalloc");
}

}  // extern "C"
