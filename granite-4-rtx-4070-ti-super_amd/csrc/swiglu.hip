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
#include "g4_sync.h"
#include "g4_wave.h"
#include "granite4_layerops.h"

#include <type_traits>

namespace g4 {
namespace {

enum : int { kOutBf16 = 0, kOutAmax = 1, kOutFp8 = 2 };

typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));

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


// Raw gate and up vectors of one 8-element output vector, as loaded: bf16
// (one 16-byte load each) or f32 (two 16-byte loads each).
template <bool F32IN>
struct GuRaw {
  V8 g, u;
};
template <>
struct GuRaw<true> {
  float4 g0, g1, u0, u1;
};

// Vector v (8 elements) of the [rows][I / 8] output: act offset 8 v, gate
// offset 8 v + r I (the row stride of gu is 2I), up offset one I further.
// Loads only: the caller issues all of a step's loads before unpacking any,
// so they are in flight together.
template <bool F32IN, bool NT>
__device__ __forceinline__ GuRaw<F32IN> load_gu(const SwArgs& a, int v, int nv) {
  const int r = div_fast(v, nv, a.inv_nv);
  const long long gofs = 8LL * v + static_cast<long long>(r) * a.I;
  GuRaw<F32IN> x;
  if constexpr (F32IN) {
    const float* p = static_cast<const float*>(a.gu) + gofs;
    x.g0 = ld_f4_nt(p);
    x.g1 = ld_f4_nt(p + 4);
    x.u0 = ld_f4_nt(p + a.I);
    x.u1 = ld_f4_nt(p + a.I + 4);
  } else {
    const uint16_t* p = static_cast<const uint16_t*>(a.gu) + gofs;
    x.g = ld8_t<NT>(p);
    x.u = ld8_t<NT>(p + a.I);
  }
  return x;
}

// act of element e (0..7), bf16-rounded, as a packed pair word for e even.
template <bool F32IN>
__device__ __forceinline__ uint32_t act_pair(const GuRaw<F32IN>& x, int p) {
  float g0, g1, u0, u1;
  if constexpr (F32IN) {
    const float4& gq = p < 2 ? x.g0 : x.g1;
    const float4& uq = p < 2 ? x.u0 : x.u1;
    const bool hi = p & 1;
    g0 = hi ? gq.z : gq.x;
    g1 = hi ? gq.w : gq.y;
    u0 = hi ? uq.z : uq.x;
    u1 = hi ? uq.w : uq.y;
  } else {
    g0 = lo_bf16(x.g.w[p]);
    g1 = hi_bf16(x.g.w[p]);
    u0 = lo_bf16(x.u.w[p]);
    u1 = hi_bf16(x.u.w[p]);
  }
  return pack_bf16_hw(silu_mul(g0, u0), silu_mul(g1, u1));
}

// f(integral_constant<int, 0>) ... f(integral_constant<int, N - 1>), in order.
template <int N, int I = 0, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<N, I + 1>(f);
  }
}

// Vectors (of gate and of up) in flight per lane.
constexpr int kSwU = 2;

// The rest of the grid-stride sweep begun by the kernel; FAST selects the
// FP8 encode form (kOutFp8 only). Returns the lane's max |act| (kOutAmax).
template <int MODE, bool F32IN, bool FAST, class S, class Load>
__device__ __forceinline__ float swiglu_run(const SwArgs& a, const Fp8Enc& f, S& sw, Load load) {
  float m = 0.0f;
  sweep_run(sw, load, [&](int v, const GuRaw<F32IN>& x) {
    const long long off = 8LL * v;
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) w[e] = act_pair<F32IN>(x, e);
    if (MODE == kOutBf16 || (MODE == kOutAmax && a.act != nullptr))
      st8_nt(a.act + off, V8{{w[0], w[1], w[2], w[3]}});
    if (MODE == kOutAmax) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        m = fmaxf(m, fmaxf(lo_bf16(w[e] & 0x7fff7fffu), hi_bf16(w[e] & 0x7fff7fffu)));
    }
    if (MODE == kOutFp8) {
      const uint2 c = fp8x8_encode_bf16<FAST>(w, f);
      st_u32x2_nt(a.codes + off, c.x, c.y);
    }
  });
  return m;
}

template <int MODE, bool F32IN>
__global__ __launch_bounds__(kBlock) void swiglu_kernel(SwArgs a) {
  // The arguments of the first loads fetched in one scalar round trip.
  asm volatile("" ::"s"(a.gu), "s"(a.rows), "s"(a.I), "s"(a.act), "s"(a.inv_nv), "s"(a.codes));
  const int nv = a.I >> 3;
  // The FP8 amax pass loads through the caches (the encode pass re-reads
  // the same gate|up right after it, and part of it is still cached: measured
  // faster in total); single-pass and final passes stream.
  constexpr bool kNt = MODE != kOutAmax;
  const auto load = [&](int v) { return load_gu<F32IN, kNt>(a, v, nv); };
  auto sw = sweep_begin<kSwU>(a.rows * nv, load);
  if (MODE == kOutFp8) {
    // The partials' reduction overlaps the first loads.
    const Fp8Enc f = fp8_enc_of(fp8_scale_for(reduce_partials(a.partials, a.n_partials)));
    if (blockIdx.x == 0 && threadIdx.x == 0) *a.scale_out = f.s;
    if (f.fast) swiglu_run<MODE, F32IN, true>(a, f, sw, load);
    else swiglu_run<MODE, F32IN, false>(a, f, sw, load);
    return;
  }
  const float m = swiglu_run<MODE, F32IN, true>(a, fp8_enc_of(0.0f), sw, load);
  if (MODE == kOutAmax) write_partial(a.partials, m);
}

// FP8 encode of a stored bf16 [rows][I] tensor under the per-tensor scale
// from the pass-1 partials (8 elements per lane per step, four steps in flight).
__global__ __launch_bounds__(kBlock) void encode_bf16_kernel(SwArgs a) {
  const auto load = [&](int v) { return ld8_nt(a.act_in + 8LL * v); };
  auto sw = sweep_begin<4>(a.rows * (a.I >> 3), load);
  const Fp8Enc f = fp8_enc_of(fp8_scale_for(reduce_partials(a.partials, a.n_partials)));
  if (blockIdx.x == 0 && threadIdx.x == 0) *a.scale_out = f.s;
  const auto body = [&](auto fast_tag) {
    return [&, fast_tag](int v, const V8& x) {
      const uint2 c = fp8x8_encode_bf16<decltype(fast_tag)::value>(x.w, f);
      st_u32x2_nt(a.codes + 8LL * v, c.x, c.y);
    };
  };
  if (f.fast) sweep_run(sw, load, body(std::true_type{}));
  else sweep_run(sw, load, body(std::false_type{}));
}

// Single-launch FP8 form: up to kMaxPartials workgroups (at most the
// resident count), each lane holding up to kFusedVpt vectors of act in
// VGPRs; the workgroups agree on max |act| with one grid synchronisation and
// encode what they hold. HBM traffic is the algorithmic 4 B read + 1 B
// written per element (+2 B with the optional bf16 act), against 9 B for
// the two-launch form, and one launch instead of two.
constexpr int kFusedThreads = kBlock;
static_assert(kFusedThreads == kSyncThreads && kBlock == kSyncThreads, "grid_max assumes kSyncThreads-thread workgroups");
constexpr int kFusedVpt = 4;

__global__ __launch_bounds__(kFusedThreads) void swiglu_fp8_fused_kernel(SwArgs a, GridSync gs) {
  // Every argument of the first loads fetched in one scalar round trip.
  asm volatile("" ::"s"(a.gu), "s"(a.rows), "s"(a.I), "s"(a.inv_nv), "s"(a.act), "s"(a.codes),
               "s"(gs.gen), "s"(gs.slots), "s"(gs.result), "s"(gs.blocks));
  const unsigned tag = grid_sync_tag(gs);
  const int nv = a.I >> 3;
  const int total = a.rows * nv;
  const int step = gridDim.x * kFusedThreads;
  const int v0 = blockIdx.x * kFusedThreads + threadIdx.x;
  GuRaw<false> x[kFusedVpt];
#pragma unroll
  for (int k = 0; k < kFusedVpt; ++k) x[k] = load_gu<false, true>(a, min(v0 + k * step, total - 1), nv);
  uint32_t w[kFusedVpt][4];
  // max |act| on the bf16 bit patterns, two per v_pk_max_u16: for
  // non-negative bf16 values the unsigned order of the patterns is the
  // numeric order. A NaN pattern (above 0x7f80 once the sign is cleared)
  // would win that maximum where fmaxf ignores NaN, so a lane that saw one
  // recomputes its maximum with fmaxf from the values it holds.
  u16x2_t mk = {0, 0};
#pragma unroll
  for (int k = 0; k < kFusedVpt; ++k) {
    const int v = v0 + k * step;
#pragma unroll
    for (int e = 0; e < 4; ++e) w[k][e] = act_pair<false>(x[k], e);
    if (v < total) {
      if (a.act != nullptr) st8_nt(a.act + 8LL * v, V8{{w[k][0], w[k][1], w[k][2], w[k][3]}});
#pragma unroll
      for (int e = 0; e < 4; ++e)
        mk = __builtin_elementwise_max(mk, __builtin_bit_cast(u16x2_t, w[k][e] & 0x7fff7fffu));
    }
  }
  const uint32_t mb = mk[0] > mk[1] ? mk[0] : mk[1];
  float m = __uint_as_float(mb << 16);
  if (__builtin_expect(mb > 0x7f80u, 0)) {
    m = 0.0f;
#pragma unroll
    for (int k = 0; k < kFusedVpt; ++k) {
      if (v0 + k * step >= total) break;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        m = fmaxf(m, fmaxf(lo_bf16(w[k][e] & 0x7fff7fffu), hi_bf16(w[k][e] & 0x7fff7fffu)));
    }
  }
  const Fp8Enc f = fp8_enc_of(fp8_scale_for(grid_max(m, gs, tag)));
  if (blockIdx.x == 0 && threadIdx.x == 0) *a.scale_out = f.s;
  const auto encode = [&](auto fast_tag) {
#pragma unroll
    for (int k = 0; k < kFusedVpt; ++k) {
      const int v = v0 + k * step;
      if (v >= total) break;
      const uint2 c = fp8x8_encode_bf16<decltype(fast_tag)::value>(w[k], f);
      st_u32x2_nt(a.codes + 8LL * v, c.x, c.y);
    }
  };
  if (f.fast) encode(std::true_type{});
  else encode(std::false_type{});
}

// Grid of the single-launch form for `vectors` 8-element vectors, or 0 when
// the tensor does not fit the resident grid's registers. One vector per lane
// where the grid allows (up to kMaxPartials workgroups, the slot count):
// measured against 1024-thread workgroups on one per CU, T=512 14.0 vs
// 14.8 us and T=8 5.9 vs 7.4 us.
unsigned fused_grid(long long vectors) {
  if (fp8_launch_mode() == 1) return 0;
  const int resident = resident_blocks(reinterpret_cast<const void*>(swiglu_fp8_fused_kernel),
                                       kFusedThreads);
  const int cap = resident < kMaxPartials ? resident : kMaxPartials;
  const long long per_block = static_cast<long long>(kFusedThreads) * kFusedVpt;
  const long long need = (vectors + per_block - 1) / per_block;
  if (cap <= 0 || need > cap) return 0;
  const long long lanes = (vectors + kFusedThreads - 1) / kFusedThreads;
  return static_cast<unsigned>(lanes < cap ? lanes : cap);
}

// Single-launch FP8 form for tensors beyond the registers' reach: a
// persistent grid (every workgroup resident, at most kMaxPartials of them)
// in which each lane holds its first kHoldR vectors of act in VGPRs and the
// next kHoldL in LDS, and streams the rest once for max |act|. After the
// grid synchronisation it encodes what it holds, interleaved with the
// re-read and encode of only the streamed rest. Every wave sets its issue
// priority from its progress (wave_priority_by_progress), which keeps the
// four workgroups sharing a CU within a quarter of their work of each other
// (the oldest otherwise runs ahead and the youngest ends the launch late).
// HBM traffic per element: 4 B read + 1 B written
// + 4 B re-read for the streamed fraction only (the two-launch form
// re-reads everything: 9 B).
// Held vectors per lane (VGPRs, LDS), held loads and streamed loads in
// flight per lane, waves per SIMD. Measured at T=8192 (µs, one box, four
// interleaved rounds): (18, 9, 4, 2, 4) 131.9-137.3, (22, 9, 2, 1, 4)
// 129.9-132.3; earlier sweeps: (24, 9, 2, 2) 149, (20, 9, 3, 2) 137,
// (28, 13, 3 waves) 132, (36, 16, 2 waves) 143-148.
constexpr int kHoldR = 22;
constexpr int kHoldL = 9;
constexpr int kHold = kHoldR + kHoldL;
constexpr int kHoldBatch = 2;  // held vectors' loads in flight per lane
constexpr int kStreamU = 1;    // streamed vectors' loads in flight per lane
constexpr int kHoldWavesPerEu = 4;
// Held vectors encoded per streamed re-read after the grid maximum (0: all
// held first). With the issue priority by progress in both sweeps, measured
// at T=8192 (one box, two rounds, us): mix 2 123.5-124.5; held first 128.7;
// mix 2 or 3 with the priority in the first sweep only 128.8-129.3; neither
// (the previous form) 128.9-129.5.
constexpr int kMix = 2;

__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(kHoldWavesPerEu))) void swiglu_fp8_hold_kernel(SwArgs a, GridSync gs) {
  asm volatile("" ::"s"(a.gu), "s"(a.rows), "s"(a.I), "s"(a.inv_nv), "s"(a.act), "s"(a.codes),
               "s"(gs.gen), "s"(gs.slots), "s"(gs.result), "s"(gs.blocks));
  __shared__ uint4 s_hold[kHoldL > 0 ? kHoldL : 1][kBlock];
  G4_TRACE_MARK(gs, 0);
  const unsigned tag = grid_sync_tag(gs);
  const int nv = a.I >> 3;
  const int total = a.rows * nv;
  const int step = gridDim.x * kBlock;
  const int v0 = blockIdx.x * kBlock + threadIdx.x;
  float m = 0.0f;
  // act words of one vector; counts them in the maximum (and stores the
  // optional bf16 act) when the vector exists.
  const auto take = [&](const GuRaw<false>& x, int v, uint32_t (&o)[4]) {
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = act_pair<false>(x, e);
    if (v < total) {
      if (a.act != nullptr) st8_nt(a.act + 8LL * v, V8{{o[0], o[1], o[2], o[3]}});
#pragma unroll
      for (int e = 0; e < 4; ++e)
        m = fmaxf(m, fmaxf(lo_bf16(o[e] & 0x7fff7fffu), hi_bf16(o[e] & 0x7fff7fffu)));
    }
  };
  uint32_t w[kHoldR][4];
  // Vectors per lane over both parts (held, then streamed), for the issue
  // priority by progress.
  const int per_lane = (total + step - 1) / step;
#pragma unroll
  for (int k0 = 0; k0 < kHold; k0 += kHoldBatch) {
    wave_priority_by_progress(k0, per_lane);
    GuRaw<false> x[kHoldBatch];
#pragma unroll
    for (int j = 0; j < kHoldBatch; ++j)
      if (k0 + j < kHold) x[j] = load_gu<false, true>(a, min(v0 + (k0 + j) * step, total - 1), nv);
#pragma unroll
    for (int j = 0; j < kHoldBatch; ++j) {
      const int k = k0 + j;
      if (k >= kHold) break;
      uint32_t o[4];
      take(x[j], v0 + k * step, o);
      if (k < kHoldR) {
#pragma unroll
        for (int e = 0; e < 4; ++e) w[k < kHoldR ? k : 0][e] = o[e];
      } else {
        s_hold[k >= kHoldR ? k - kHoldR : 0][threadIdx.x] = make_uint4(o[0], o[1], o[2], o[3]);
      }
    }
  }
  G4_TRACE_MARK(gs, 1);
  // The streamed rest: max only (cached loads: part is still cached when
  // the second sweep comes back to it).
  const int vs = v0 + kHold * step;
  for (int v = vs, i = kHold; v < total; v += kStreamU * step, i += kStreamU) {
    wave_priority_by_progress(i, per_lane);
    GuRaw<false> x[kStreamU];
#pragma unroll
    for (int j = 0; j < kStreamU; ++j) x[j] = load_gu<false, false>(a, min(v + j * step, total - 1), nv);
#pragma unroll
    for (int j = 0; j < kStreamU; ++j) {
      uint32_t o[4];
      take(x[j], v + j * step, o);
    }
  }
  G4_TRACE_MARK(gs, 2);
  __builtin_amdgcn_s_setprio(0);
  const Fp8Enc f = fp8_enc_of(fp8_scale_for(grid_max(m, gs, tag)));
  G4_TRACE_MARK(gs, 3);
  if (blockIdx.x == 0 && threadIdx.x == 0) *a.scale_out = f.s;
  const auto encode = [&](auto fast_tag) {
    constexpr bool kFast = decltype(fast_tag)::value;
    // One 64-bit base and a uniform offset per held vector (64-bit indices
    // per vector kept live across the grid maximum would spill).
    uint8_t* const cbase = a.codes + 8LL * v0;
    const auto streamed = [&](const GuRaw<false>& x, int v) {
      uint32_t o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = act_pair<false>(x, e);
      const uint2 c = fp8x8_encode_bf16<kFast>(o, f);
      st_u32x2_nt(a.codes + 8LL * v, c.x, c.y);
    };
    // The held vectors' encode (stores only) interleaved with the re-read of
    // the streamed rest: after every kMix held vectors (whose registers are
    // then free) the previous streamed vector is encoded and the next one's
    // load issued, so a load is in flight while the held codes are written.
    int vn = vs;
    GuRaw<false> xs;
    const auto held = [&](auto kc) {
      constexpr int k = decltype(kc)::value;
      if (k >= kHold) return;
      if (k % 4 == 0) wave_priority_by_progress(k, per_lane);
      if (v0 >= total - k * step) return;
      uint32_t o[4];
      if constexpr (k < kHoldR) {
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = w[k][e];
      } else {
        const uint4 h = s_hold[k - kHoldR][threadIdx.x];
        o[0] = h.x;
        o[1] = h.y;
        o[2] = h.z;
        o[3] = h.w;
      }
      const uint2 c = fp8x8_encode_bf16<kFast>(o, f);
      st_u32x2_nt(cbase + 8LL * k * step, c.x, c.y);
    };
    constexpr int kGroup = kMix > 0 ? kMix : kHold;
    static_for<(kHold + kGroup - 1) / kGroup>([&](auto gc) {
      constexpr int g = decltype(gc)::value;
      static_for<kGroup>([&](auto kc) { held(std::integral_constant<int, g * kGroup + decltype(kc)::value>{}); });
      if constexpr (kMix > 0) {
        if constexpr (g > 0) {
          if (vn < total) streamed(xs, vn);
          vn += step;
        }
        xs = load_gu<false, true>(a, min(vn, total - 1), nv);
      }
    });
    if constexpr (kMix > 0) {
      if (vn < total) streamed(xs, vn);
      vn += step;
    }
    G4_TRACE_MARK(gs, 4);
    for (int v = vn, i = kHold; v < total; v += step, ++i) {
      wave_priority_by_progress(i, per_lane);
      const GuRaw<false> x = load_gu<false, true>(a, v, nv);
      streamed(x, v);
    }
  };
  if (f.fast) encode(std::true_type{});
  else encode(std::false_type{});
  G4_TRACE_MARK(gs, 5);
}

// Grid of the held single-launch form (every workgroup resident, one
// partial slot each), or 0 when the device cannot hold a useful grid or the
// indices would overflow.
unsigned hold_grid(long long vectors) {
  if (fp8_launch_mode() == 1) return 0;
  const int resident = resident_blocks(reinterpret_cast<const void*>(swiglu_fp8_hold_kernel), kBlock);
  const int grid = resident < kMaxPartials ? resident : kMaxPartials;
  if (grid < kCUs) return 0;
  if (vectors + static_cast<long long>(kHold + kStreamU) * grid * kBlock >= INT_MAX) return 0;
  return static_cast<unsigned>(grid);
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

namespace g4 {

bool launch_encode_bf16(const uint16_t* act, int rows, int I, const float* partials, int n_partials,
                        uint8_t* codes, float* scale_out) {
  SwArgs p = sw_args(act, rows, I);
  p.act_in = act;
  p.codes = codes;
  p.scale_out = scale_out;
  p.partials = const_cast<float*>(partials);
  p.n_partials = n_partials;
  hipLaunchKernelGGL(encode_bf16_kernel, grid_for(static_cast<long long>(rows) * (I / 8), kPersistBlocks),
                     kBlock, 0, stream(), p);
  return launch_status("granite4 FP8 encode") == 0;
}

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
  const long long vectors = static_cast<long long>(rows) * (I / 8);
  const unsigned fgrid = fused_grid(vectors);
  if (fgrid != 0) {
    SwArgs f = sw_args(d_gu, rows, I);
    f.act = d_act;
    f.codes = d_codes;
    f.scale_out = d_scale;
    const GridSync gs{work_slots(d_work), work_gen(d_work), work_result(d_work),
                      static_cast<int>(fgrid), work_err(d_work), fp8_sync_spin_limit()};
    launch_grid_sync(swiglu_fp8_fused_kernel, fgrid, kFusedThreads, stream(), f, gs);
    return launch_status("granite4_swiglu_fp8");
  }
  const unsigned hgrid = hold_grid(vectors);
  if (hgrid != 0) {
    SwArgs h = sw_args(d_gu, rows, I);
    h.act = d_act;
    h.codes = d_codes;
    h.scale_out = d_scale;
    const GridSync gs{work_slots(d_work), work_gen(d_work), work_result(d_work),
                      static_cast<int>(hgrid), work_err(d_work), fp8_sync_spin_limit()};
    launch_grid_sync(swiglu_fp8_hold_kernel, hgrid, kBlock, stream(), h, gs);
    return launch_status("granite4_swiglu_fp8");
  }
  const unsigned grid = grid_for(vectors, kMaxPartials);
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
    // Pass 2 reads only the partials' count from the grid, not its size:
    // it runs at full occupancy.
    hipLaunchKernelGGL((swiglu_kernel<kOutFp8, false>),
                       grid_for(static_cast<long long>(rows) * (I / 8), kPersistBlocks), kBlock, 0,
                       stream(), p2);
  }
  return launch_status("granite4_swiglu_fp8 (encode)");
}

}  // extern "C"
