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
// Layout: 256-thread workgroups of 8 weight rows (4 for the smaller forms
// without a norm prologue; swiglu: half gate rows, half the matching up
// rows). The workgroup walks its rows in order with G4_GEMV_DEPTH
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
#include "rope_unit.h"

#include <cmath>
#include <cstdio>

namespace g4 {
namespace {

// Prologues: none; the RMSNorm of x; the embedding row of the token at
// *d_pos (x = bf16(emb_mult * emb[token]), also stored to x_out, the
// residual stream) followed by the RMSNorm.
enum : int { kProNone = 0, kProNorm = 1, kProEmbedNorm = 2 };
enum : int { kEpiOut = 0, kEpiResid = 1, kEpiSwiglu = 2, kEpiRope = 3 };

#ifndef G4_GEMV_DEPTH
#define G4_GEMV_DEPTH 4
#endif
constexpr int kDepth = G4_GEMV_DEPTH;     // rows of loads in flight
// The RoPE forms (768 workgroups for the 8B q|k|v: 3 per CU) issue all 8
// rows before the norm prologue: one round trip to the weights instead of
// two. Measured (rocprof kernel durations, 40-layer steps): norm + q|k|v +
// RoPE 7.47 -> 7.28 us per call; 6 rows in flight 7.47.
#ifndef G4_GEMV_ROPE_DEPTH
#define G4_GEMV_ROPE_DEPTH 8
#endif
constexpr int kRopeDepth = G4_GEMV_ROPE_DEPTH;
constexpr int kMaxChunks = 4;             // 1024-byte chunks per wave per row: K <= 16384
constexpr int kMaxK = 4 * kMaxChunks * 1024;

struct GemvArgs {
  const uint16_t* x;      // activation, or the residual row to normalise
  const uint16_t* gamma;  // norm weight (kProNorm)
  float eps;
  double inv_k;           // 1 / K when K is a power of two, else 0
  const uint8_t* w[3];    // weight segments [n_i][K]
  float s[3];             // their scales
  uint16_t* o[3];         // their outputs (kEpiOut); o[0] = out / act otherwise
  int seg1, seg2, N;      // rows [0, seg1) from w[0], [seg1, seg2) from w[1], the rest w[2]
  int K;
  const uint16_t* residual;  // kEpiResid (may alias o[0])
  float rs;
  int I;                  // kEpiSwiglu: act columns (w[0] gate, w[1] up)
  // kEpiRope: segments 0 and 1 (q, k heads of 128 rows) rotated at *d_pos
  const float* cos_t;
  const float* sin_t;
  int max_pos;
  const int* d_pos;
  // kProEmbedNorm: x is row tokens[*d_pos] of the table x (vocab rows; a
  // token outside [0, vocab) gives a zero row), times emb_mult.
  const int32_t* tokens;
  int vocab;
  float emb_mult;
  uint16_t* x_out;
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

// Sum of squares of the 16 bf16 in w[8], in double, as a pairwise tree
// (each square of a bf16 is exact in f32, so only the additions round; the
// tree keeps the dependent chain 4 additions long instead of 16).
__device__ __forceinline__ double sumsq16(const uint32_t (&w)[8]) {
  double d[16];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float lo = lo_bf16(w[e]), hi = hi_bf16(w[e]);
    d[2 * e] = static_cast<double>(lo * lo);
    d[2 * e + 1] = static_cast<double>(hi * hi);
  }
#pragma unroll
  for (int w2 = 8; w2 > 0; w2 >>= 1)
#pragma unroll
    for (int i = 0; i < w2; ++i) d[i] = d[2 * i] + d[2 * i + 1];
  return d[0];
}

// mean = ss / K as the reference computes it (double division): a multiply
// by the exact 1 / K when K is a power of two (inv_k != 0).
__device__ __forceinline__ double mean_of(double ss, int K, double inv_k) {
  return inv_k != 0.0 ? ss * inv_k : ss / K;
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

// Weight row r (0 .. kRows - 1) of the workgroup, or nullptr past the end (n:
// its output index). swiglu: the first half gate rows, the second half the up
// rows of the same act columns.
// kEpiRope (kRows = 2 half): the rotated segments [0, seg2) go 64 / half
// blocks per head, block j of a head holding dims half j .. half j + half - 1
// (rows r < half) and their RoPE partners 64 + half j .. (rows r >= half), so
// each rotation pair is in one workgroup; the rows past seg2 (v) follow in
// order.
template <int EPI, int kRows>
__device__ __forceinline__ int out_row(const GemvArgs& a, int r) {
  if (EPI == kEpiRope) {
    constexpr int half = kRows / 2;
    const int nrot = a.seg2 / kRows;
    if (static_cast<int>(blockIdx.x) < nrot) {
      const int h = blockIdx.x / (64 / half), j = blockIdx.x % (64 / half);
      return h * 128 + half * j + (r % half) + (r >= half ? 64 : 0);
    }
    return a.seg2 + (blockIdx.x - nrot) * kRows + r;
  }
  return blockIdx.x * kRows + r;
}

template <int EPI, int kRows>
__device__ __forceinline__ const uint8_t* row_ptr(const GemvArgs& a, int r, int& n) {
  if (EPI == kEpiSwiglu) {
    const int c = blockIdx.x * (kRows / 2) + (r % (kRows / 2));
    n = c;
    if (c >= a.I) return nullptr;
    return (r < kRows / 2 ? a.w[0] : a.w[1]) + static_cast<size_t>(c) * a.K;
  }
  const int i = out_row<EPI, kRows>(a, r);
  n = i;
  if (i >= a.N) return nullptr;
  if (i < a.seg1) return a.w[0] + static_cast<size_t>(i) * a.K;
  if (i < a.seg2) return a.w[1] + static_cast<size_t>(i - a.seg1) * a.K;
  return a.w[2] + static_cast<size_t>(i - a.seg2) * a.K;
}

// Row r's offset (in rows) from row 0 within its segment when every row of
// the workgroup lies in one segment: r, or the head-paired order in
// kEpiRope's rotated segments. (The swiglu form, whose halves come from two
// matrices, has a fast path of its own.)
template <int EPI, int kRows>
__device__ __forceinline__ int row_offset(const GemvArgs& a, int r) {
  // kEpiRope: head-paired rows in the rotated segments, plain order for v
  if (EPI == kEpiRope && static_cast<int>(blockIdx.x) < a.seg2 / kRows)
    return (r % (kRows / 2)) + (r >= kRows / 2 ? 64 : 0);
  return r;
}

template <int EPI, int kRows>
__device__ __forceinline__ bool rows_in_one_segment(const GemvArgs& a) {
  if (EPI == kEpiSwiglu) return false;
  const int first = out_row<EPI, kRows>(a, 0);
  const int last = out_row<EPI, kRows>(a, kRows - 1);
  if (last >= a.N || last - first != row_offset<EPI, kRows>(a, kRows - 1)) return false;
  const int sf = first < a.seg1 ? 0 : (first < a.seg2 ? 1 : 2);
  const int sl = last < a.seg1 ? 0 : (last < a.seg2 ? 1 : 2);
  return sf == sl;
}

// Workgroup barrier for LDS exchanges only (waits for this wave's LDS
// operations, not for its weight loads in flight).
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <int PRO, int EPI, int kChunks, int kRows>
__global__ __launch_bounds__(256) void gemv_kernel(GemvArgs a) {
  __shared__ double s_ss[4];
  __shared__ float s_part[4][kRows];
  // Every kernel argument the prologue needs, fetched together: otherwise the
  // compiler loads them where each is first used, one dependent scalar-cache
  // miss after another before the first weight load.
  asm volatile("" ::"s"(a.N), "s"(a.K), "s"(a.seg1), "s"(a.seg2), "s"(a.I), "s"(a.w[0]),
               "s"(a.w[1]), "s"(a.w[2]), "s"(a.x), "s"(a.gamma), "s"(a.d_pos));
  if (PRO == kProEmbedNorm) asm volatile("" ::"s"(a.tokens), "s"(a.vocab), "s"(a.emb_mult), "s"(a.x_out));
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
  if (EPI == kEpiSwiglu && static_cast<int>(blockIdx.x + 1) * (kRows / 2) <= a.I) {
    // Every act column of the workgroup exists: gate rows c0 .. c0 + kRows / 2
    // - 1, then the same up rows.
    const int c0 = blockIdx.x * (kRows / 2);
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
      const int c = c0 + r % (kRows / 2);
      rows[r] = (r < kRows / 2 ? a.w[0] : a.w[1]) + static_cast<size_t>(c) * a.K;
      ns[r] = c;
      live[r] = true;
    }
  } else if (rows_in_one_segment<EPI, kRows>(a)) {
    // Every row of the workgroup exists and lies in one weight segment (all
    // but the last workgroup of a segment): row r at a fixed offset from the
    // first, straight-line address arithmetic.
    int n0;
    const uint8_t* p0 = row_ptr<EPI, kRows>(a, 0, n0);
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
      const int off = row_offset<EPI, kRows>(a, r);
      rows[r] = p0 + static_cast<size_t>(off) * a.K;
      ns[r] = n0 + off;
      live[r] = true;
    }
  } else {
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
      rows[r] = row_ptr<EPI, kRows>(a, r, ns[r]);
      live[r] = rows[r] != nullptr;
      if (!live[r]) rows[r] = a.w[0];
    }
  }

  // Rows of weights stream in order, kDepth rows in flight; the 4 waves read
  // each row together (4 contiguous quarters), so the workgroup's accesses
  // stay within a few contiguous rows at any time. Every load is
  // unconditional (out-of-range data is zeroed before use).
  // Measured: 8 rows in flight instead of 4 in the 8-row forms cost 14 us
  // per decode step (all 8 in flight before the SwiGLU form's norm: no
  // change, 18.7 vs 18.8 us per call).
  constexpr int kDep = EPI == kEpiRope ? kRopeDepth : kDepth;
  constexpr int kD = kRows < kDep ? kRows : kDep;
  uint4 buf[kD][kChunks];
  const auto load_row = [&](int r, uint4 (&dst)[kChunks]) {
#pragma unroll
    for (int c = 0; c < kChunks; ++c) dst[c] = ld_u4_nt(rows[r] + koff[c]);
  };
  // Prologue loads: the lane's activations (and norm weights) first, then
  // the first kDepth weight rows, all issued before any is used (vmcnt is in
  // order: x is waited for while the rows are still in flight, so the norm
  // overlaps the weight fetch). Without the scheduling barrier the compiler
  // unpacks x between the row loads and the wait holds the later rows back
  // by a round trip.
  float av[kChunks][16];
  uint4 xr[kChunks][2], gr[kChunks][2];
  // kEpiRope's position, loaded first as a vector load (a scalar load would
  // be scheduled after the weight rows, and its wait would hold the norm).
  int rpos = 0;
  if (EPI == kEpiRope) {
    int z;
    asm volatile("v_mov_b32 %0, 0" : "=v"(z));
    rpos = a.d_pos[z];
  }
  if (PRO == kProEmbedNorm) {
    // The token's row depends on two loads (position, token): the weight
    // rows go out first, then the row and gamma.
#pragma unroll
    for (int r = 0; r < kD; ++r) load_row(r, buf[r]);
    // The token through the scalar cache (its wait counts scalar loads only,
    // not the weight rows issued above, which a vector load would queue
    // behind). A negative position reads no token (a zero row).
    const int pos_s = __builtin_amdgcn_readfirstlane(rpos);
    int tok = -1;
    if (pos_s >= 0) {
      const int32_t* tp = a.tokens + pos_s;
      asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(tok) : "s"(tp) : "memory");
    }
    const bool valid = tok >= 0 && tok < a.vocab;
    const uint32_t vmask = valid ? 0xffffffffu : 0u;
    const uint16_t* xrow = a.x + static_cast<size_t>(valid ? tok : 0) * K;
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
      xr[c][0] = *reinterpret_cast<const uint4*>(xrow + koff[c]);
      xr[c][1] = *reinterpret_cast<const uint4*>(xrow + koff[c] + 8);
      gr[c][0] = *reinterpret_cast<const uint4*>(a.gamma + koff[c]);
      gr[c][1] = *reinterpret_cast<const uint4*>(a.gamma + koff[c] + 8);
    }
    // bf16(emb_mult * e) per element, as the embedding kernel computes it;
    // workgroup 0 stores the row (the residual stream of the step).
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        uint32_t w4[4] = {xr[c][h].x, xr[c][h].y, xr[c][h].z, xr[c][h].w};
#pragma unroll
        for (int e = 0; e < 4; ++e)
          w4[e] = pack_bf16_hw(a.emb_mult * lo_bf16(w4[e]), a.emb_mult * hi_bf16(w4[e])) & vmask;
        xr[c][h] = make_uint4(w4[0], w4[1], w4[2], w4[3]);
      }
      if (blockIdx.x == 0 && cin[c]) {
        *reinterpret_cast<uint4*>(a.x_out + koff[c]) = xr[c][0];
        *reinterpret_cast<uint4*>(a.x_out + koff[c] + 8) = xr[c][1];
      }
    }
  } else {
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
      xr[c][0] = *reinterpret_cast<const uint4*>(a.x + koff[c]);
      xr[c][1] = *reinterpret_cast<const uint4*>(a.x + koff[c] + 8);
      if (PRO == kProNorm) {
        gr[c][0] = *reinterpret_cast<const uint4*>(a.gamma + koff[c]);
        gr[c][1] = *reinterpret_cast<const uint4*>(a.gamma + koff[c] + 8);
      }
    }
#pragma unroll
    for (int r = 0; r < kD; ++r) load_row(r, buf[r]);
  }
  __builtin_amdgcn_sched_barrier(0);
  // kEpiRope: this thread's cos / sin (as output row threadIdx.x % 8), loaded
  // unconditionally from a clamped position, used in the epilogue.
  // kEpiResid: the residual of this thread's output row (threads < kRows),
  // loaded now so the epilogue does not wait a round trip for it.
  uint32_t res_bits = 0;
  if (EPI == kEpiResid) {
    const int n = min(static_cast<int>(blockIdx.x * kRows + threadIdx.x % kRows), a.N - 1);
    res_bits = a.residual[n];
  }
  float rc = 0.0f, rsn = 0.0f;
  static_assert(PRO != kProEmbedNorm || EPI == kEpiRope, "the embed prologue reads *d_pos");
  if (EPI == kEpiRope) {
    const int i = out_row<EPI, kRows>(a, threadIdx.x % kRows) % 128;
    const long long cp = static_cast<long long>(min(max(rpos, 0), a.max_pos - 1)) * 64 + (i & 63);
    rc = a.cos_t[cp];
    rsn = a.sin_t[cp];
  }
  if (PRO != kProNone) {
    double ss = 0.0;
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
      if (!cin[c]) continue;
      const uint32_t w[8] = {xr[c][0].x, xr[c][0].y, xr[c][0].z, xr[c][0].w,
                             xr[c][1].x, xr[c][1].y, xr[c][1].z, xr[c][1].w};
      ss += sumsq16(w);
    }
    ss = wave_sum(ss);
    if (lane == 0) s_ss[wave] = ss;
    lds_barrier();
    ss = s_ss[0] + s_ss[1] + s_ss[2] + s_ss[3];
    const float rr = 1.0f / sqrtf(static_cast<float>(mean_of(ss, K, a.inv_k)) + a.eps);
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
      const uint4 g0 = gr[c][0], g1 = gr[c][1];
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
    const int slot = r % kD;
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
    if (r + kD < kRows) load_row(r + kD, buf[slot]);
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
  const int n = out_row<EPI, kRows>(a, r);
  if (n >= a.N) return;
  if (EPI == kEpiRope && n < a.seg2) {
    // y = bf16(s tot) for this row and its partner (r ^ 4), then the append
    // kernels' rotation (rotate8: a c + b' s, b' the partner, negated in the
    // first half of the head) and bf16. A position outside the table leaves
    // the output unwritten, as the append kernels leave q_rot.
    const int seg = n < a.seg1 ? 0 : 1;
    const int base = seg == 0 ? 0 : a.seg1;
    const int p = r ^ (kRows / 2);
    const float tp = (s_part[0][p] + s_part[1][p]) + (s_part[2][p] + s_part[3][p]);
    const float ya = bf16_to_f32(f32_to_bf16(a.s[seg] * tot));
    const float yp = bf16_to_f32(f32_to_bf16(a.s[seg] * tp));
    const float b = r < kRows / 2 ? -yp : yp;
    if (rpos >= 0 && rpos < a.max_pos) a.o[seg][n - base] = static_cast<uint16_t>(f32_to_bf16(ya * rc + b * rsn));
    return;
  }
  if (EPI == kEpiResid) {
    const float y = a.s[0] * tot;
    const float res = __uint_as_float(res_bits << 16);
    a.o[0][n] = static_cast<uint16_t>(f32_to_bf16(res + a.rs * y));
  } else {
    const int seg = n < a.seg1 ? 0 : (n < a.seg2 ? 1 : 2);
    const int base = seg == 0 ? 0 : (seg == 1 ? a.seg1 : a.seg2);
    a.o[seg][n - base] = static_cast<uint16_t>(f32_to_bf16(a.s[seg] * tot));
  }
}

// ---------------------------------------------------------------------------
// Decode q|k|v GEMV with the RMSNorm prologue and RoPE + the quantised KV
// write as its epilogue: one 1024-thread workgroup per head (128 weight rows:
// Hq query heads, then Hk key heads, then Hk value heads), each wave reading
// whole rows (chunk c of a row = lane bytes [16 l + 1024 c, +16)). The head's
// 128 outputs gather in LDS as bf16 and one 16-lane row applies rope_unit to
// them, exactly as the append kernel does to a stored q|k|v row.
//
// Sums in the order of gemv_kernel (one partial per 1024-byte chunk, reduced
// across lanes, then (c0 + c1) + (c2 + c3)), and the norm's sum of squares in
// the same order, so the outputs are bit-identical to
// granite4_gemv_rmsnorm_qkv followed by granite4_rope_append_at_pos.
// ---------------------------------------------------------------------------
constexpr int kHeadWaves = 16;
constexpr int kHeadRowsPerWave = 128 / kHeadWaves;

template <int BITS, int GROUP>
__global__ __launch_bounds__(1024) void gemv_qkv_rope_kernel(GemvArgs g, RopeArgs ra) {
  __shared__ uint16_t s_head[128];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int u = blockIdx.x;  // head unit
  const int Hq = ra.Hq, Hk = ra.Hk;
  const int seg = u < Hq ? 0 : (u < Hq + Hk ? 1 : 2);
  const int h = seg == 0 ? u : (seg == 1 ? u - Hq : u - Hq - Hk);
  const uint8_t* wbase = g.w[seg] + static_cast<size_t>(h) * 128 * 4096;
  const float scale = g.s[seg];

  // Weights: rows 8 wave .. 8 wave + 7 of the head, 2 rows in flight.
  uint4 buf[2][4];
  const auto load_row = [&](int j, uint4 (&dst)[4]) {
    const uint8_t* row = wbase + static_cast<size_t>(kHeadRowsPerWave * wave + j) * 4096;
#pragma unroll
    for (int c = 0; c < 4; ++c) dst[c] = ld_u4_nt(row + 1024 * c + 16 * lane);
  };
  load_row(0, buf[0]);
  load_row(1, buf[1]);

  // Norm prologue over the whole row (K = 4096): chunk c = bytes 1024 c + 16 l
  // of the bf16 row, as wave c of gemv_kernel holds them.
  uint32_t av[4][8];  // the lane's normalised activations, bf16 pairs
  {
    uint4 xr[4][2], gr[4][2];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int k = 1024 * c + 16 * lane;
      xr[c][0] = *reinterpret_cast<const uint4*>(g.x + k);
      xr[c][1] = *reinterpret_cast<const uint4*>(g.x + k + 8);
      gr[c][0] = *reinterpret_cast<const uint4*>(g.gamma + k);
      gr[c][1] = *reinterpret_cast<const uint4*>(g.gamma + k + 8);
    }
    double ssc[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint32_t w[8] = {xr[c][0].x, xr[c][0].y, xr[c][0].z, xr[c][0].w,
                             xr[c][1].x, xr[c][1].y, xr[c][1].z, xr[c][1].w};
      ssc[c] = wave_sum(sumsq16(w));
    }
    const double ss = ssc[0] + ssc[1] + ssc[2] + ssc[3];
    const float rr = 1.0f / sqrtf(static_cast<float>(ss * (1.0 / 4096)) + g.eps);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint32_t xv[8] = {xr[c][0].x, xr[c][0].y, xr[c][0].z, xr[c][0].w,
                              xr[c][1].x, xr[c][1].y, xr[c][1].z, xr[c][1].w};
      const uint32_t gv[8] = {gr[c][0].x, gr[c][0].y, gr[c][0].z, gr[c][0].w,
                              gr[c][1].x, gr[c][1].y, gr[c][1].z, gr[c][1].w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        av[c][e] = pack_bf16_hw(lo_bf16(xv[e]) * rr * lo_bf16(gv[e]),
                                hi_bf16(xv[e]) * rr * hi_bf16(gv[e]));
      }
    }
  }

#pragma unroll
  for (int j = 0; j < kHeadRowsPerWave; ++j) {
    float part[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float wf[16];
      fp8x16_to_f32(buf[j & 1][c], wf);
      float sum = 0.0f;
#pragma unroll
      for (int e = 0; e < 16; ++e)
        sum = fmaf(wf[e], (e & 1) ? hi_bf16(av[c][e >> 1]) : lo_bf16(av[c][e >> 1]), sum);
      part[c] = sum;
    }
    if (j + 2 < kHeadRowsPerWave) load_row(j + 2, buf[j & 1]);
#pragma unroll
    for (int c = 0; c < 4; ++c) part[c] = wave_sum_f32(part[c]);
    if (lane == 0)
      s_head[kHeadRowsPerWave * wave + j] =
          static_cast<uint16_t>(f32_to_bf16(scale * ((part[0] + part[1]) + (part[2] + part[3]))));
  }
  __syncthreads();
  if (threadIdx.x >= 16) return;
  const int lane16 = threadIdx.x;
  rope_unit<BITS, GROUP>(ra, 0, u, lane16, [&](const uint16_t*) {
    const uint4 v = *reinterpret_cast<const uint4*>(s_head + 8 * lane16);
    return V8{{v.x, v.y, v.z, v.w}};
  });
}

bool gemv_k_ok(int K) { return K >= 64 && K % 64 == 0 && K <= kMaxK; }
bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Chunks per wave per row: K / 4 bytes in 1024-byte chunks. Rows per
// workgroup: 16, or 8 when 16 would leave fewer than two workgroups per CU.
#ifndef G4_GEMV_ROPE_ROWS
#define G4_GEMV_ROPE_ROWS 8
#endif
constexpr int kRopeRows = G4_GEMV_ROPE_ROWS;

template <int PRO, int EPI>
int launch_gemv(const GemvArgs& a, const char* what) {
  const int ch = (a.K / 4 + 1023) / 1024;
  const long long outputs = EPI == kEpiSwiglu ? 2LL * a.I : a.N;
  // Rows per workgroup: 8 (swiglu: 4 gate + 4 up rows), or 4 for the forms
  // without a norm prologue whose outputs number fewer than 8192 (O, q|k|v,
  // down). Measured per call (40-layer graphs, medians over interleaved
  // rounds), against the earlier 16 rows for 8192 outputs and up:
  //   norm + gate/up + SwiGLU   19.5 -> 18.3-18.9 us (4 rows: 27)
  //   gate|up plain             19.5 -> 18.0-18.3
  //   O + residual               5.68 -> 5.31 (4 rows)
  //   q|k|v                      6.76 -> 6.41 (4 rows)
  //   down + residual           11.81 -> 11.63 (4 rows)
  // More workgroups hide the weight stream's latency better; the norm forms
  // keep 8 (with 4 their per-workgroup row norm costs more than it hides:
  // q|k|v 7.18 -> 7.39), as the RoPE form must (head-paired rows).
  const int rows = EPI == kEpiRope ? kRopeRows
                   : (PRO == kProNone && EPI != kEpiSwiglu && outputs < 8192 ? 4 : 8);
  const unsigned grid = static_cast<unsigned>(EPI == kEpiSwiglu ? (a.I + rows / 2 - 1) / (rows / 2)
                                                                 : (a.N + rows - 1) / rows);
  const hipStream_t st = stream();
  const auto go = [&](auto kern) { hipLaunchKernelGGL(kern, grid, 256, 0, st, a); };
  if constexpr ((PRO == kProNone && EPI != kEpiSwiglu) || EPI == kEpiRope) {
    if (rows == 4) {
      if (ch <= 1) go(gemv_kernel<PRO, EPI, 1, 4>);
      else if (ch == 2) go(gemv_kernel<PRO, EPI, 2, 4>);
      else go(gemv_kernel<PRO, EPI, 4, 4>);
      return launch_status(what);
    }
  }
  if (ch <= 1) go(gemv_kernel<PRO, EPI, 1, 8>);
  else if (ch == 2) go(gemv_kernel<PRO, EPI, 2, 8>);
  else go(gemv_kernel<PRO, EPI, 4, 8>);
  return launch_status(what);
}

int gemv_out(int pro, const uint16_t* x, const uint16_t* gamma, float eps,
             const uint8_t* const (&w)[3], const float (&s)[3], uint16_t* const (&o)[3],
             const int (&n)[3], int K, const char* what) {
  const long long N = static_cast<long long>(n[0]) + n[1] + n[2];
  if (x == nullptr || !al16(x) || !gemv_k_ok(K) || N <= 0 || N > INT_MAX || n[0] < 0 ||
      n[1] < 0 || n[2] < 0 ||
      (pro == kProNorm && (gamma == nullptr || !al16(gamma) || !std::isfinite(eps))) ||
      N * K >= (1LL << 40)) {
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
  a.N = static_cast<int>(N);
  a.K = K;
  a.inv_k = (K & (K - 1)) == 0 ? 1.0 / K : 0.0;
  return pro == kProNorm ? launch_gemv<kProNorm, kEpiOut>(a, what)
                         : launch_gemv<kProNone, kEpiOut>(a, what);
}

// q|k|v with RoPE on q and k (Hq, Hk heads of 128): kRows 8, head-paired rows.
int gemv_qkv_rope(int pro, const uint16_t* x, const uint16_t* gamma, float eps,
                  const uint8_t* wq, const uint8_t* wk, const uint8_t* wv, float sq, float sk,
                  float sv, const float* cos_t, const float* sin_t, int max_pos, const int* d_pos,
                  int Hq, int Hk, int K, uint16_t* q_rot, uint16_t* k_rot, uint16_t* v,
                  const char* what) {
  if (x == nullptr || !al16(x) || !gemv_k_ok(K) || Hq <= 0 || Hk <= 0 || cos_t == nullptr ||
      sin_t == nullptr || max_pos <= 0 || d_pos == nullptr || wq == nullptr || wk == nullptr ||
      wv == nullptr || !al16(wq) || !al16(wk) || !al16(wv) || q_rot == nullptr ||
      k_rot == nullptr || v == nullptr || !std::isfinite(sq) || !std::isfinite(sk) ||
      !std::isfinite(sv) || (pro == kProNorm && (gamma == nullptr || !al16(gamma) || !std::isfinite(eps))) ||
      static_cast<long long>(Hq + 2 * Hk) * 128 * K >= (1LL << 40)) {
    std::fprintf(stderr, "granite4: %s: invalid arguments\n", what);
    return -1;
  }
  GemvArgs a{};
  a.x = x;
  a.gamma = gamma;
  a.eps = eps;
  a.w[0] = wq;
  a.w[1] = wk;
  a.w[2] = wv;
  a.s[0] = sq;
  a.s[1] = sk;
  a.s[2] = sv;
  a.o[0] = q_rot;
  a.o[1] = k_rot;
  a.o[2] = v;
  a.seg1 = Hq * 128;
  a.seg2 = (Hq + Hk) * 128;
  a.N = (Hq + 2 * Hk) * 128;
  a.K = K;
  a.inv_k = (K & (K - 1)) == 0 ? 1.0 / K : 0.0;
  a.cos_t = cos_t;
  a.sin_t = sin_t;
  a.max_pos = max_pos;
  a.d_pos = d_pos;
  return pro == kProNorm ? launch_gemv<kProNorm, kEpiRope>(a, what)
                         : launch_gemv<kProNone, kEpiRope>(a, what);
}

// The first layer's q|k|v with the embedding of the step's token as the
// prologue (kProEmbedNorm): gemv_qkv_rope's arguments plus the table.
int gemv_embed_qkv_rope(const int32_t* tokens, const uint16_t* emb, int vocab, float emb_mult,
                        uint16_t* hidden_out, const uint16_t* gamma, float eps, const uint8_t* wq,
                        const uint8_t* wk, const uint8_t* wv, float sq, float sk, float sv,
                        const float* cos_t, const float* sin_t, int max_pos, const int* d_pos,
                        int Hq, int Hk, int K, uint16_t* q_rot, uint16_t* k_rot, uint16_t* v,
                        const char* what) {
  if (tokens == nullptr || emb == nullptr || !al16(emb) || vocab <= 0 || !std::isfinite(emb_mult) ||
      hidden_out == nullptr || !al16(hidden_out) || gamma == nullptr || !al16(gamma) ||
      !std::isfinite(eps) || !gemv_k_ok(K) || Hq <= 0 || Hk <= 0 || cos_t == nullptr ||
      sin_t == nullptr || max_pos <= 0 || d_pos == nullptr || wq == nullptr || wk == nullptr ||
      wv == nullptr || !al16(wq) || !al16(wk) || !al16(wv) || q_rot == nullptr ||
      k_rot == nullptr || v == nullptr || !std::isfinite(sq) || !std::isfinite(sk) ||
      !std::isfinite(sv) || static_cast<long long>(Hq + 2 * Hk) * 128 * K >= (1LL << 40) ||
      static_cast<long long>(vocab) * K >= (1LL << 40)) {
    std::fprintf(stderr, "granite4: %s: invalid arguments\n", what);
    return -1;
  }
  GemvArgs a{};
  a.x = emb;
  a.gamma = gamma;
  a.eps = eps;
  a.w[0] = wq;
  a.w[1] = wk;
  a.w[2] = wv;
  a.s[0] = sq;
  a.s[1] = sk;
  a.s[2] = sv;
  a.o[0] = q_rot;
  a.o[1] = k_rot;
  a.o[2] = v;
  a.seg1 = Hq * 128;
  a.seg2 = (Hq + Hk) * 128;
  a.N = (Hq + 2 * Hk) * 128;
  a.K = K;
  a.inv_k = (K & (K - 1)) == 0 ? 1.0 / K : 0.0;
  a.cos_t = cos_t;
  a.sin_t = sin_t;
  a.max_pos = max_pos;
  a.d_pos = d_pos;
  a.tokens = tokens;
  a.vocab = vocab;
  a.emb_mult = emb_mult;
  a.x_out = hidden_out;
  return launch_gemv<kProEmbedNorm, kEpiRope>(a, what);
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
  a.N = static_cast<int>(N);
  a.K = K;
  a.inv_k = (K & (K - 1)) == 0 ? 1.0 / K : 0.0;
  return pro == kProNorm ? launch_gemv<kProNorm, kEpiSwiglu>(a, what)
                         : launch_gemv<kProNone, kEpiSwiglu>(a, what);
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
  a.inv_k = (K & (K - 1)) == 0 ? 1.0 / K : 0.0;
  return launch_gemv<kProNone, kEpiResid>(a, "granite4_gemv_fp8w_resid");
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

int granite4_gemv_qkv_rope(const uint16_t* d_a, const uint8_t* d_wq, const uint8_t* d_wk,
                           const uint8_t* d_wv, float sq, float sk, float sv, const float* cos_tbl,
                           const float* sin_tbl, int max_pos, const int* d_pos, int Hq, int Hk,
                           int K, uint16_t* d_q_rot, uint16_t* d_k_rot, uint16_t* d_v) {
  return gemv_qkv_rope(kProNone, d_a, nullptr, 0.0f, d_wq, d_wk, d_wv, sq, sk, sv, cos_tbl,
                       sin_tbl, max_pos, d_pos, Hq, Hk, K, d_q_rot, d_k_rot, d_v,
                       "granite4_gemv_qkv_rope");
}

int granite4_gemv_embed_rmsnorm_qkv_rope(const int32_t* d_tokens, const uint16_t* d_emb,
                                         int vocab, float emb_mult, uint16_t* d_hidden_out,
                                         const uint16_t* d_gamma, float eps, const uint8_t* d_wq,
                                         const uint8_t* d_wk, const uint8_t* d_wv, float sq,
                                         float sk, float sv, const float* cos_tbl,
                                         const float* sin_tbl, int max_pos, const int* d_pos,
                                         int Hq, int Hk, int K, uint16_t* d_q_rot,
                                         uint16_t* d_k_rot, uint16_t* d_v) {
  return gemv_embed_qkv_rope(d_tokens, d_emb, vocab, emb_mult, d_hidden_out, d_gamma, eps, d_wq,
                             d_wk, d_wv, sq, sk, sv, cos_tbl, sin_tbl, max_pos, d_pos, Hq, Hk, K,
                             d_q_rot, d_k_rot, d_v, "granite4_gemv_embed_rmsnorm_qkv_rope");
}

int granite4_gemv_rmsnorm_qkv_rope(const uint16_t* d_x, const uint16_t* d_gamma, float eps,
                                   const uint8_t* d_wq, const uint8_t* d_wk, const uint8_t* d_wv,
                                   float sq, float sk, float sv, const float* cos_tbl,
                                   const float* sin_tbl, int max_pos, const int* d_pos, int Hq,
                                   int Hk, int K, uint16_t* d_q_rot, uint16_t* d_k_rot,
                                   uint16_t* d_v) {
  return gemv_qkv_rope(kProNorm, d_x, d_gamma, eps, d_wq, d_wk, d_wv, sq, sk, sv, cos_tbl,
                       sin_tbl, max_pos, d_pos, Hq, Hk, K, d_q_rot, d_k_rot, d_v,
                       "granite4_gemv_rmsnorm_qkv_rope");
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

int granite4_gemv_rmsnorm_qkv_rope_append(const uint16_t* d_x, const uint16_t* d_gamma,
                                          float eps, const uint8_t* d_wq, const uint8_t* d_wk,
                                          const uint8_t* d_wv, float sq, float sk, float sv,
                                          const float* cos_tbl, const float* sin_tbl, int max_pos,
                                          const int* d_pos, const int* d_pt, int Hq, int Hk,
                                          int bits, int group, uint16_t* q_rot, void* cache_k,
                                          void* cache_v, float* k_scale, float* v_scale,
                                          int stride) {
  RopeArgs ra;
  // q / k / v point at the weights only to pass the builder's null checks:
  // the head rows come from the GEMV, not from memory.
  const uint16_t* dummy = d_x;
  if (d_x == nullptr || d_gamma == nullptr || !al16(d_x) || !al16(d_gamma) || d_wq == nullptr ||
      d_wk == nullptr || d_wv == nullptr || !al16(d_wq) || !al16(d_wk) || !al16(d_wv) ||
      !std::isfinite(eps) || !std::isfinite(sq) || !std::isfinite(sk) || !std::isfinite(sv) ||
      !rope_args_at_pos(ra, dummy, dummy, dummy, cos_tbl, sin_tbl, max_pos, d_pos, d_pt, Hq, Hk,
                        128, bits, group, q_rot, cache_k, cache_v, k_scale, v_scale, stride)) {
    std::fprintf(stderr, "granite4: granite4_gemv_rmsnorm_qkv_rope_append: invalid arguments\n");
    return -1;
  }
  GemvArgs g{};
  g.x = d_x;
  g.gamma = d_gamma;
  g.eps = eps;
  g.w[0] = d_wq;
  g.w[1] = d_wk;
  g.w[2] = d_wv;
  g.s[0] = sq;
  g.s[1] = sk;
  g.s[2] = sv;
  g.K = 4096;
  const unsigned grid = static_cast<unsigned>(Hq + 2 * Hk);
  const hipStream_t st = stream();
  const int grp = bits == 16 ? 128 : group;
  const auto go = [&](auto kern) { hipLaunchKernelGGL(kern, grid, 1024, 0, st, g, ra); };
  switch (bits * 1000 + grp) {
    case 16128: go(gemv_qkv_rope_kernel<16, 128>); break;
    case 8128: go(gemv_qkv_rope_kernel<8, 128>); break;
    case 8064: go(gemv_qkv_rope_kernel<8, 64>); break;
    case 8032: go(gemv_qkv_rope_kernel<8, 32>); break;
    case 4128: go(gemv_qkv_rope_kernel<4, 128>); break;
    case 4064: go(gemv_qkv_rope_kernel<4, 64>); break;
    case 4032: go(gemv_qkv_rope_kernel<4, 32>); break;
    case 5128: go(gemv_qkv_rope_kernel<5, 128>); break;
    case 5064: go(gemv_qkv_rope_kernel<5, 64>); break;
    default: go(gemv_qkv_rope_kernel<5, 32>); break;
  }
  return launch_status("granite4_gemv_rmsnorm_qkv_rope_append");
}

}  // extern "C"
