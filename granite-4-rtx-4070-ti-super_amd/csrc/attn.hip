// attn.hip - split-KV decode attention over the paged KV pool, gfx950.
//
// The reference's attn_split (attention_split.cu:1083-1255; its default
// tensor-core kernel :791-1047 and attn_combine_kernel :1049-1074): causal
// GQA for up to 16 query rows, head dim 128, Hq = 4 Hk, reading the pool
// written by the append kernels (bf16, int8, int4, or K5 K + int4 V, with
// per-row or per-group f32 scales) through a position -> arena-row table.
//
// Work split: positions are cut into 64-position tiles and the tiles into
// splits of tps tiles (tps = ceil(tiles / 256) of the longest sequence, as
// the reference). One 64-lane wave owns one (KV head, split, group of up to
// four query rows of one sequence): the 16 MFMA rows are 4 query rows x the
// KV head's 4 query heads. Per tile:
//
//   S^T = K Q^T   v_mfma_f32_16x16x32_bf16, A = K rows straight from global
//                 memory (codes converted to exact bf16 integers), B = Q^T
//                 held in VGPRs. Lane l ends up owning query column l % 16
//                 and keys 16 mb + 4 (l / 16) + i - a whole query row per
//                 lane, so the online softmax needs no transpose: the row
//                 maximum is an in-register max plus two cross-lane steps.
//   O^T += V^T P^T  A = V^T read from a row-major LDS copy of the tile with
//                 ds_read_b64_tr_b16 (each 16-lane group receives 4 keys x 1
//                 dim per lane), B = P^T packed from the lane's own
//                 probabilities. The MFMA's contraction index runs over the
//                 tile's keys in the order the S^T lanes hold them (4 g + i,
//                 then 16 + 4 g + i), the same for both operands.
//
// Numerics (the reference's tensor-core path): logit = bf16(scale * dot) with
// dot = q . k (bf16 K) or q . codes * k_scale (one scale per row); p =
// exp(logit - m) in f32 against the split's running maximum m, l sums the
// unrounded p, and the value product uses bf16(p * v_scale) (or bf16(p))
// against the V codes (values). Scale groups of 32 / 64 (not a reference
// format) read each element as bf16(code * scale_g) and take the bf16 path
// (kv_deq). The combine
// rescales the splits' (m, l, o) and writes bf16(sum o w / sum l w): by
// default the last split block of each (row group, KV head) does it inside
// the split launch (combine_wave), else a second launch (attn_combine_kernel)
// with the same arithmetic.
// The MFMA accumulates in f32 in its own order; the tests hold the result to
// the oracle's sequential f32 evaluation within stated bf16 tolerances.
#include "g4_common.h"
#include "g4_hw.h"
#include "g4_math.h"
#include "granite4_layerops.h"
#include "rope_unit.h"

#include <atomic>
#include <climits>
#include <cstdlib>
#include <random>
#include <type_traits>
#include <cmath>

namespace g4 {
namespace {

constexpr int kTile = 64;
constexpr int kHd = 128;         // head dim
constexpr int kGq = 4;           // query heads per KV head
constexpr int kRowsPerWave = 4;  // query rows per wave (x 4 heads = 16 MFMA rows)
constexpr int kAttnMaxSplits = 256;
enum : int { kAttnPlain = 0, kAttnRopeAppend = 1, kAttnAppend = 2 };
constexpr int kAttnWaves = 4;  // splits per workgroup, merged before the combine
constexpr int kVPitch = kHd + 16;  // LDS V row pitch (bf16): 288 B, rows 8 banks apart
// Waves per SIMD the split kernel is compiled for: two (so a grid of more
// blocks than CUs keeps two blocks on each), except the bf16 decode-append
// forms, whose appended row's registers on top of the K tile would spill.
constexpr int attn_waves_per_eu(int bits, int mode) { return bits == 16 && mode != 0 ? 1 : 2; }

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));

struct AttnArgs {
  const uint16_t* q;   // [rows][Hq][128]
  const uint8_t* k;    // [Hk][stride][K row bytes]
  const uint8_t* v;    // [Hk][stride][V row bytes]
  const float* ksc;    // [Hk][stride][ngrp] (quantised)
  const float* vsc;
  float scale;
  int Hq, stride, rows, tps, splits, window, kv_base;
  int nblk;  // split blocks (ceil(splits / kAttnWaves)): partials per (row, head)
  const int* d_pos;
  const int* d_pt;
  const int* row_pos;
  const int* const* row_pt;
  float2* part_ml;  // [rows][Hq][nblk]
  float* part_o;    // [rows][Hq][nblk][128]
  uint16_t* out;    // [rows][Hq][128]
  // Combine inside the split launch: the arrival tag of each split block,
  // [row groups][Hk][nblk], and this call's tag (never 0). tags == nullptr:
  // a second launch (attn_combine_kernel) combines.
  unsigned* tags;
  unsigned tag;
  unsigned* err;  // sticky error word (1: a combining block's wait gave up)
  int spin_limit; // polls before the combining block gives up
  // Decode append (one row at *d_pos): q, k, v are the raw bf16 projections
  // (ra.q / ra.k / ra.v); q is rotated in registers, and the wave whose split
  // holds the position rotates and quantises that position's K / V row (the
  // append kernels' arithmetic) into LDS, reads the key from there, and
  // copies the row to the pool when its work is done.
  RopeArgs ra;
};

typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;
// The page tables are device (global) memory; typed so, their loads are
// global_load (vmcnt only) rather than flat (which LDS waits would include).
typedef __attribute__((address_space(1))) const int g4_global_i32;

// Four bf16 of a row-major LDS tile, transposed across each 16-lane group
// (ds_read_b64_tr_b16): lane i of a group receives element i % 4 of the
// 8-byte vectors addressed by lanes i / 4, 4 + i / 4, 8 + i / 4, 12 + i / 4.
__device__ __forceinline__ u32x2_t lds_read_tr(const uint16_t* p) {
  return __builtin_bit_cast(u32x2_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(p)));
}

__device__ __forceinline__ bf16x8_t as_bf16x8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  const u32x4_t u = {a, b, c, d};
  return __builtin_bit_cast(bf16x8_t, u);
}

constexpr float kLog2E = 1.44269504088896341f;

// Exact bf16 pair of two small integers (|x| <= 127).
__device__ __forceinline__ uint32_t int_pair_bf16(int a, int b) {
  return pack_bf16_hw(static_cast<float>(a), static_cast<float>(b));
}
// The int4 codes at bits [b, b + 4) and [b + 4, b + 8) of x, as their
// values code - 8, in bf16: the code xor 8 read as a signed 4-bit field is
// code - 8, so each value is one sign-extending field extract (xs = x ^
// 0x88888888, once per word) instead of an extract and a subtraction.
__device__ __forceinline__ int sfield4(uint32_t xs, int b) {
  return static_cast<int>(xs << (28 - b)) >> 28;
}
__device__ __forceinline__ uint32_t int4_pair_bf16(uint32_t xs, int b) {
  return int_pair_bf16(sfield4(xs, b), sfield4(xs, b + 4));
}

// Row bytes of the K / V caches per format.
__host__ __device__ constexpr int k_row_bytes(int bits) {
  return bits == 16 ? 2 * kHd : bits == 8 ? kHd : bits == 4 ? kHd / 2 : kHd / 2 + kHd / 8;
}
__host__ __device__ constexpr int v_row_bytes(int bits) {
  return bits == 16 ? 2 * kHd : bits == 8 ? kHd : kHd / 2;
}

// Raw bytes of eight K elements (dims c .. c + 7, c a multiple of 8) of one
// cached row: bf16 16 B, int8 8 B, int4 4 B, K5 4 nibble bytes + the high-bit
// plane byte. Loading and converting are separate so that a tile's K and V
// loads are all in flight before any of them is used.
template <int BITS>
__device__ __forceinline__ u32x4_t load_k_raw(const uint8_t* row, int c) {
  u32x4_t r = {0u, 0u, 0u, 0u};
  if constexpr (BITS == 16) {
    r = *reinterpret_cast<const u32x4_t*>(row + 2 * c);
  } else if constexpr (BITS == 8) {
    const u32x2_t u = *reinterpret_cast<const u32x2_t*>(row + c);
    r.x = u.x;
    r.y = u.y;
  } else {
    r.x = *reinterpret_cast<const uint32_t*>(row + c / 2);
    if constexpr (BITS == 5) r.y = row[kHd / 2 + c / 8];
  }
  return r;
}

// The eight K elements as bf16: the value (bf16 cache) or the integer code.
template <int BITS>
__device__ __forceinline__ bf16x8_t k_raw_bf16(const u32x4_t& r) {
  if constexpr (BITS == 16) {
    return __builtin_bit_cast(bf16x8_t, r);
  } else if constexpr (BITS == 8) {
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t x = e < 2 ? r.x : r.y;
      const int sh = 16 * (e & 1);
      w[e] = int_pair_bf16(static_cast<int8_t>(x >> sh), static_cast<int8_t>(x >> (sh + 8)));
    }
    return as_bf16x8(w[0], w[1], w[2], w[3]);
  } else if constexpr (BITS == 4) {
    const uint32_t xs = r.x ^ 0x88888888u;
    return as_bf16x8(int4_pair_bf16(xs, 0), int4_pair_bf16(xs, 8), int4_pair_bf16(xs, 16),
                     int4_pair_bf16(xs, 24));
  } else {
    // K5: the eight 5-bit codes assembled bytewise, four at a time: the low
    // nibbles (dims c + 2 e) and the high nibbles (c + 2 e + 1) masked out of
    // x, and the high-bit plane's bits 2 e (+ 1) moved to bit 4 of byte e by
    // one 24-bit multiply (bit 2 e of t times 2^4 + 2^10 + 2^16 + 2^22 lands
    // on 8 e + 4; the other products miss bits 4, 12, 20 and 28 and carry
    // into none of them). Each byte then converts to f32 in one instruction
    // (v_cvt_f32_ubyte*) and value = code - 16 exactly.
    static_assert(BITS == 5, "k_raw_bf16: bf16, int8, int4 or K5");
    constexpr uint32_t kSpread = (1u << 4) | (1u << 10) | (1u << 16) | (1u << 22);
    const uint32_t lo = (r.x & 0x0F0F0F0Fu) | (__umul24(r.y & 0x55u, kSpread) & 0x10101010u);
    const uint32_t hi = ((r.x >> 4) & 0x0F0F0F0Fu) | (__umul24((r.y >> 1) & 0x55u, kSpread) & 0x10101010u);
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      w[e] = pack_bf16_hw(static_cast<float>((lo >> (8 * e)) & 0xFFu) - 16.0f,
                          static_cast<float>((hi >> (8 * e)) & 0xFFu) - 16.0f);
    return as_bf16x8(w[0], w[1], w[2], w[3]);
  }
}

// Scale groups smaller than a row (32 or 64: this build's extension; the
// reference keeps one scale per row): the attention reads each element
// dequantised, bf16(code * scale_g), and then runs the bf16 path (logits
// bf16(scale * q . k), unscaled bf16 probabilities). One scale per row keeps
// the reference's form: codes in the products, the row's scales on the dot
// and on p.
template <int BITS, int GROUP>
constexpr bool kv_deq() { return BITS != 16 && GROUP < kHd; }

// The eight K elements of a quantised row as f32 codes.
template <int BITS>
__device__ __forceinline__ void k_raw_f32(const u32x4_t& r, float (&f)[8]) {
  if constexpr (BITS == 8) {
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = static_cast<float>(static_cast<int8_t>((e < 4 ? r.x : r.y) >> (8 * (e & 3))));
  } else if constexpr (BITS == 4) {
    const uint32_t xs = r.x ^ 0x88888888u;
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = static_cast<float>(sfield4(xs, 4 * e));
  } else {
    static_assert(BITS == 5, "k_raw_f32: int8, int4 or K5");
    constexpr uint32_t kSpread = (1u << 4) | (1u << 10) | (1u << 16) | (1u << 22);
    const uint32_t lo = (r.x & 0x0F0F0F0Fu) | (__umul24(r.y & 0x55u, kSpread) & 0x10101010u);
    const uint32_t hi = ((r.x >> 4) & 0x0F0F0F0Fu) | (__umul24((r.y >> 1) & 0x55u, kSpread) & 0x10101010u);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      f[2 * e] = static_cast<float>((lo >> (8 * e)) & 0xFFu) - 16.0f;
      f[2 * e + 1] = static_cast<float>((hi >> (8 * e)) & 0xFFu) - 16.0f;
    }
  }
}
// Unsigned codes held one per byte of lo (dims 2 e) and hi (dims 2 e + 1),
// dequantised as bf16((code - bias) * s): fma(code, s, -bias * s) is the same
// f32 (code * s - bias * s is exactly (code - bias) * s, and both round it
// once; bias * s is exact), one instruction instead of a subtraction and a
// multiply.
__device__ __forceinline__ bf16x8_t bytes_deq(uint32_t lo, uint32_t hi, float s, float nbs) {
  uint32_t w[4];
#pragma unroll
  for (int e = 0; e < 4; ++e)
    w[e] = pack_bf16_hw(fmaf(static_cast<float>((lo >> (8 * e)) & 0xFFu), s, nbs),
                        fmaf(static_cast<float>((hi >> (8 * e)) & 0xFFu), s, nbs));
  return as_bf16x8(w[0], w[1], w[2], w[3]);
}

// ... dequantised with the elements' group scale: bf16(code * s).
template <int BITS>
__device__ __forceinline__ bf16x8_t k_raw_deq(const u32x4_t& r, float s) {
  if constexpr (BITS == 5) {
    constexpr uint32_t kSpread = (1u << 4) | (1u << 10) | (1u << 16) | (1u << 22);
    const uint32_t lo = (r.x & 0x0F0F0F0Fu) | (__umul24(r.y & 0x55u, kSpread) & 0x10101010u);
    const uint32_t hi = ((r.x >> 4) & 0x0F0F0F0Fu) | (__umul24((r.y >> 1) & 0x55u, kSpread) & 0x10101010u);
    return bytes_deq(lo, hi, s, -16.0f * s);
  } else if constexpr (BITS == 4) {
    return bytes_deq(r.x & 0x0F0F0F0Fu, (r.x >> 4) & 0x0F0F0F0Fu, s, -8.0f * s);
  } else {
    float f[8];
    k_raw_f32<BITS>(r, f);
    return as_bf16x8(pack_bf16_hw(f[0] * s, f[1] * s), pack_bf16_hw(f[2] * s, f[3] * s),
                     pack_bf16_hw(f[4] * s, f[5] * s), pack_bf16_hw(f[6] * s, f[7] * s));
  }
}
// One 16-byte V chunk (int8: 16 values, int4: 32), dequantised with scale s,
// as bf16 pairs w[0 .. 8 or 16).
template <int BITS>
__device__ __forceinline__ void v_chunk_deq(const u32x4_t& u, float s, uint32_t (&w)[BITS == 8 ? 8 : 16]) {
  if constexpr (BITS == 8) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t x = u[e >> 1];
      const int sh = 16 * (e & 1);
      w[e] = pack_bf16_hw(static_cast<float>(static_cast<int8_t>(x >> sh)) * s,
                          static_cast<float>(static_cast<int8_t>(x >> (sh + 8))) * s);
    }
  } else {
    // bf16((code - 8) * s) per nibble, the low nibble of byte b first
    const float nbs = -8.0f * s;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t lo = u[q] & 0x0F0F0F0Fu, hi = (u[q] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
      for (int b = 0; b < 4; ++b)
        w[4 * q + b] = pack_bf16_hw(fmaf(static_cast<float>((lo >> (8 * b)) & 0xFFu), s, nbs),
                                    fmaf(static_cast<float>((hi >> (8 * b)) & 0xFFu), s, nbs));
    }
  }
}

// V staging: each step moves one 16-byte chunk per lane of the tile's rows
// (bf16: 4 keys x 16 chunks per step, 16 steps; int8: 8 keys x 8 chunks, 8
// steps; int4: 16 keys x 4 chunks, 4 steps) from the pool into a row-major
// LDS tile, as bf16 values / integer codes; keys without an arena row read 0.
template <int BITS>
struct VStage {
  static constexpr int kSteps = BITS == 16 ? 16 : BITS == 8 ? 8 : 4;
  static constexpr int kChunks = 64 / (kTile / kSteps);  // chunks per row
  static constexpr int kRowB = BITS == 16 ? 256 : BITS == 8 ? 128 : 64;
};

template <int BITS>
__device__ __forceinline__ void v_load(const uint8_t* vbase, int prow,
                                       u32x4_t (&raw)[VStage<BITS>::kSteps]) {
  using VS = VStage<BITS>;
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < VS::kSteps; ++i) {
    const int key = i * (64 / VS::kChunks) + lane / VS::kChunks, c = lane % VS::kChunks;
    const int pr = __shfl(prow, key);
    // Unconditional (row 0 for keys without a row); v_store zeroes those.
    raw[i] = *reinterpret_cast<const u32x4_t*>(vbase + static_cast<size_t>(pr >= 0 ? pr : 0) * VS::kRowB + 16 * c);
  }
}

// bf16 V tiles go from global memory straight to LDS (global_load_lds, 16
// bytes per lane): no registers hold them, so the bf16 kernel fits two waves
// per SIMD. The tile is 64 rows of 256 bytes without padding; the 16-byte
// chunk c of row r sits at chunk c ^ 2 (r & 7), so that the transposed reads
// of 16 consecutive rows (32 bytes each) spread over all 64 banks (two
// passes, as with the padded layout). Load i writes rows 4 i .. 4 i + 3.
typedef __attribute__((address_space(3))) void* lds_ptr_t;
__device__ __forceinline__ int v_swz(int row) { return 2 * (row & 7); }
__device__ __forceinline__ void v_dma_bf16(const uint8_t* vbase, int prow, uint16_t* vl) {
  const int lane = threadIdx.x & 63;
  uint8_t* dst = reinterpret_cast<uint8_t*>(vl);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int row = 4 * i + (lane >> 4), c = (lane & 15) ^ v_swz(row);
    const int pr = __shfl(prow, row);
    // Unconditional (row 0 for keys without a row); v_fix_bf16 zeroes those.
    __builtin_amdgcn_global_load_lds(vbase + static_cast<size_t>(pr >= 0 ? pr : 0) * 256 + 16 * c,
                                     (lds_ptr_t)(dst + 1024 * i), 16, 0, 0);
  }
}
// After the loads have landed: rows without an arena row become 0.
__device__ __forceinline__ void v_fix_bf16(uint16_t* vl, unsigned long long valid) {
  if (valid == ~0ull) return;
  const int lane = threadIdx.x & 63;
  uint8_t* dst = reinterpret_cast<uint8_t*>(vl);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int row = 4 * i + (lane >> 4);
    if (!((valid >> row) & 1ull))
      *reinterpret_cast<u32x4_t*>(dst + 1024 * i + 16 * lane) = u32x4_t{0u, 0u, 0u, 0u};
  }
}

// v_store for scale groups smaller than a row: each chunk dequantised with
// its key's group scale, scale_of(key, group) (keys without a row: 0).
template <int BITS, int GROUP, typename F>
__device__ __forceinline__ void v_store_deq(const u32x4_t (&raw)[VStage<BITS>::kSteps], uint16_t* vl,
                                            unsigned long long valid, F scale_of) {
  using VS = VStage<BITS>;
  static_assert(BITS == 8 || BITS == 4 || BITS == 5, "quantised V");
  constexpr int kDims = kHd / VS::kChunks;  // dims per chunk (16 or 32), within one group
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < VS::kSteps; ++i) {
    const int key = i * (64 / VS::kChunks) + lane / VS::kChunks, c = lane % VS::kChunks;
    const float sc = ((valid >> key) & 1ull) ? scale_of(key, (kDims * c) / GROUP) : 0.0f;
    uint32_t w[BITS == 8 ? 8 : 16];
    v_chunk_deq<BITS>(raw[i], sc, w);
    uint16_t* dst = vl + key * kVPitch + kDims * c;
#pragma unroll
    for (int e = 0; e < kDims / 8; ++e)
      *reinterpret_cast<u32x4_t*>(dst + 8 * e) = u32x4_t{w[4 * e], w[4 * e + 1], w[4 * e + 2], w[4 * e + 3]};
    __builtin_amdgcn_sched_barrier(0);  // one step's values live at a time
  }
}

// valid: bit k set when key k of the tile has an arena row (others store 0).
template <int BITS>
__device__ __forceinline__ void v_store(const u32x4_t (&raw)[VStage<BITS>::kSteps], uint16_t* vl,
                                        unsigned long long valid) {
  using VS = VStage<BITS>;
  const int lane = threadIdx.x & 63;
  const uint32_t z = BITS == 16 || BITS == 8 ? 0u : 0x88888888u;  // int4 code 8 = value 0
#pragma unroll
  for (int i = 0; i < VS::kSteps; ++i) {
    const int key = i * (64 / VS::kChunks) + lane / VS::kChunks, c = lane % VS::kChunks;
    const u32x4_t u = ((valid >> key) & 1ull) ? raw[i] : u32x4_t{z, z, z, z};
    if constexpr (BITS == 16) {
      *reinterpret_cast<u32x4_t*>(vl + key * kVPitch + 8 * c) = u;
    } else if constexpr (BITS == 8) {
      uint32_t w[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t x = u[e >> 1];
        const int sh = 16 * (e & 1);
        w[e] = int_pair_bf16(static_cast<int8_t>(x >> sh), static_cast<int8_t>(x >> (sh + 8)));
      }
      uint16_t* dst = vl + key * kVPitch + 16 * c;
      *reinterpret_cast<u32x4_t*>(dst) = u32x4_t{w[0], w[1], w[2], w[3]};
      *reinterpret_cast<u32x4_t*>(dst + 8) = u32x4_t{w[4], w[5], w[6], w[7]};
    } else {
      uint32_t w[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const uint32_t x = u[e >> 2];
        const int b = 8 * (e & 3);
        w[e] = int4_pair_bf16(x ^ 0x88888888u, b);
      }
      uint16_t* dst = vl + key * kVPitch + 32 * c;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        *reinterpret_cast<u32x4_t*>(dst + 8 * e) = u32x4_t{w[4 * e], w[4 * e + 1], w[4 * e + 2], w[4 * e + 3]};
    }
  }
}

// Completes this wave's LDS writes before other lanes of the wave read them
// (each wave owns its LDS tile, so no workgroup barrier is needed).
__device__ __forceinline__ void wave_lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Partials and arrival tags are written and read at device scope (sc1 on
// gfx950): the workgroup that combines may run on another XCD, whose L2
// holds none of the writer's lines, and a tag must not be seen before the
// partial it announces.
__device__ __forceinline__ void st_dev_u64(void* p, unsigned long long v) {
  __hip_atomic_store(static_cast<unsigned long long*>(p), v, __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long ld_dev_u64(const void* p) {
  return __hip_atomic_load(static_cast<unsigned long long*>(const_cast<void*>(p)), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long f2_bits(float x, float y) {
  return static_cast<unsigned long long>(__float_as_uint(x)) |
         (static_cast<unsigned long long>(__float_as_uint(y)) << 32);
}
__device__ __forceinline__ void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Causal length of row `row` (unclamped): its position + 1.
__device__ __forceinline__ int combine_len(const AttnArgs& a, int row) {
  return a.row_pos != nullptr ? a.row_pos[row] + 1
                              : (a.d_pos != nullptr ? *a.d_pos : a.kv_base) + row + 1;
}

// The split blocks [s0, used) whose partials make up a row of causal length
// len: the blocks up to len (clamped to the arena), from the block holding
// the window's first key.
__device__ __forceinline__ void combine_range(const AttnArgs& a, int len, int& s0, int& used) {
  const int span = kAttnWaves * a.tps * kTile;  // positions per split block
  used = min((min(max(len, 0), a.stride) + span - 1) / span, a.nblk);
  s0 = a.window > 0 ? max(0, len - a.window) / span : 0;
}

// One wave combines the split-block partials of one (row, head)
// (attn_combine_kernel, attention_split.cu:1049-1074): M = max m_b,
// w_b = exp(m_b - M) (0 for a block without keys of the row), L = sum l_b w_b
// and out = bf16(sum o_b w_b / L), both sums in block order. Lane j holds
// block s0 + j's (m, l) (at most 64 blocks: kAttnMaxSplits / kAttnWaves);
// each lane owns dims 2 lane and 2 lane + 1, whose partials are loaded 16
// blocks at a time. (32 at a time, one round trip up to 32 blocks, measured
// 0.1-0.3 us faster at 17 blocks and 0.2-0.5 us slower at 1-16 and 32.)
//
// len: the row's causal length (combine_len), known before the call: loaded
// here, after the partials' loads, its wait would also wait for all of them
// (memory loads complete in order), one more round trip.
__device__ void combine_wave(const AttnArgs& a, int row, int h, int len) {
  static_assert(kAttnMaxSplits / kAttnWaves <= 64, "one (m, l) per lane");
  const int lane = threadIdx.x & 63;
  constexpr int kChunk = 16;
  const size_t rbase = (static_cast<size_t>(row) * a.Hq + h) * a.nblk;
  const float* prow = a.part_o + rbase * kHd + 2 * lane;
  // The first chunk and the (m, l) loads go out before the row's block range
  // is known, from block 0; a window that starts the row's blocks later
  // loads them again from its first block.
  unsigned long long ov[kChunk];
#pragma unroll
  for (int j = 0; j < kChunk; ++j) ov[j] = ld_dev_u64(prow + static_cast<size_t>(min(j, a.nblk - 1)) * kHd);
  unsigned long long mlb = ld_dev_u64(a.part_ml + rbase + min(lane, a.nblk - 1));
  int s0, used;
  combine_range(a, len, s0, used);
  if (s0 > 0) {
    const int sc = min(s0, a.nblk - 1), lc = max(min(used, a.nblk) - 1, sc);
#pragma unroll
    for (int j = 0; j < kChunk; ++j) ov[j] = ld_dev_u64(prow + static_cast<size_t>(min(sc + j, lc)) * kHd);
    mlb = ld_dev_u64(a.part_ml + rbase + min(sc + lane, lc));
  }
  const int nb = used - s0;  // blocks s0 + j, j < nb (the loads above start at block s0)
  const float mj = lane < nb ? __uint_as_float(static_cast<unsigned>(mlb)) : -INFINITY;
  const float lj = lane < nb ? __uint_as_float(static_cast<unsigned>(mlb >> 32)) : 0.0f;
  float M = mj;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o));
  const float wj = mj == -INFINITY ? 0.0f : expf(mj - M);
  float L = 0.0f, acc0 = 0.0f, acc1 = 0.0f;
  for (int c = 0; c < nb; c += kChunk) {
    if (c > 0) {
#pragma unroll
      for (int j = 0; j < kChunk; ++j)
        ov[j] = ld_dev_u64(prow + static_cast<size_t>(s0 + min(c + j, nb - 1)) * kHd);
    }
#pragma unroll
    for (int j = 0; j < kChunk; ++j) {
      if (c + j < nb) {
        const float wb = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wj), c + j));
        const float lb = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lj), c + j));
        L += lb * wb;
        acc0 += __uint_as_float(static_cast<unsigned>(ov[j])) * wb;
        acc1 += __uint_as_float(static_cast<unsigned>(ov[j] >> 32)) * wb;
      }
    }
  }
  *reinterpret_cast<uint32_t*>(a.out + (static_cast<size_t>(row) * a.Hq + h) * kHd + 2 * lane) =
      f32_to_bf16(acc0 / L) | (f32_to_bf16(acc1 / L) << 16);
}

// MODE: kAttnPlain; kAttnRopeAppend (granite4_attn_decode_append: raw q, k
// rotated here, the new K / V row appended); kAttnAppend
// (granite4_attn_decode_append_rotated: q and k already rotated, the new row
// appended). A template parameter so that the plain kernels carry none of
// the append's registers.
// parameter so that the plain kernels carry none of its registers.
template <int BITS, int GROUP, int MODE>
__global__ __launch_bounds__(kAttnWaves * 64) __attribute__((amdgpu_waves_per_eu(attn_waves_per_eu(BITS, MODE))))
void attn_split_kernel(AttnArgs a) {
  constexpr bool kQuant = BITS != 16;
  constexpr int kNgrp = kQuant ? kHd / GROUP : 1;
  constexpr bool kDeq = kv_deq<BITS, GROUP>();  // elements dequantised before the products
  constexpr bool kQB = kQuant && !kDeq;         // the products see codes and row scales
  constexpr int kNgrpB = kQB ? kNgrp : 1;       // P packs per key
  constexpr int kKb = k_row_bytes(BITS), kVb = v_row_bytes(BITS);
  // Per wave: its V tile (reused for the end-of-block merge); each row's K and
  // V scales sit in the row's padding (dims 128..143: 8 floats), so the
  // block's LDS stays under half a CU's and two blocks fit on one.
  __shared__ __align__(16) uint16_t vl_all[kAttnWaves][kTile * kVPitch];
  static_assert(2 * kNgrp * sizeof(float) <= (kVPitch - kHd) * sizeof(uint16_t), "scales in the pad");

  // The kernel arguments of the prologue fetched together (one scalar-cache
  // miss instead of a chain of them before the position is even requested).
  asm volatile("" ::"s"(a.d_pos), "s"(a.d_pt), "s"(a.row_pos), "s"(a.row_pt), "s"(a.rows),
               "s"(a.stride), "s"(a.tps), "s"(a.splits), "s"(a.window), "s"(a.kv_base),
               "s"(a.q), "s"(a.k), "s"(a.v), "s"(a.Hq));
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint16_t* vl = vl_all[wave];
  // Scale slots of key `key`, group gi: floats 64 + gi (K) and 68 + gi (V) of its row.
  float* const vlf = reinterpret_cast<float*>(vl);
  auto ksc_at = [&](int key, int gi) -> float& { return vlf[key * (kVPitch / 2) + kHd / 2 + gi]; };
  auto vsc_at = [&](int key, int gi) -> float& { return vlf[key * (kVPitch / 2) + kHd / 2 + 4 + gi]; };
  const int g = lane >> 4;   // lane group: keys 4 g + i of each 16-key block
  const int n = lane & 15;   // query column: row n / 4, head n % 4
  const int hkv = blockIdx.x, split = blockIdx.y * kAttnWaves + wave;
  const int per = a.row_pos != nullptr ? 1 : kRowsPerWave;
  const int r0 = blockIdx.z * per;
  const int nr = min(per, a.rows - r0);
  // The position, the row's position and the row's page table, loaded at
  // once and unconditionally (absent ones read the q buffer and are unused),
  // so that no wait for one sits in a branch ahead of the others.
  const void* qv = a.q;
  const int pos_raw = *(a.d_pos != nullptr ? a.d_pos : static_cast<const int*>(qv));
  const int rpos_raw = *(a.row_pos != nullptr ? a.row_pos + r0 : static_cast<const int*>(qv));
  const int* const rpt_raw =
      *(a.row_pt != nullptr ? a.row_pt + r0 : static_cast<const int* const*>(qv));
  const int base = a.row_pos != nullptr ? 0 : (a.d_pos != nullptr ? pos_raw : a.kv_base);
  // Causal length, clamped to the arena (a position read from device memory
  // never sends the page-table reads past the arena's positions).
  // Multi-sequence rows (row_pos) take one row per wave, so only rr = 0 is
  // ever asked for there: one scalar load.
  const int row_pos0 = a.row_pos != nullptr ? rpos_raw : 0;
  auto row_len = [&](int rr) {
    const int len = a.row_pos != nullptr ? row_pos0 + 1 : base + r0 + rr + 1;
    return min(max(len, 0), a.stride);
  };
  auto row_lo = [&](int rr) { return a.window > 0 ? max(0, row_len(rr) - a.window) : 0; };
  int kv_max = 0, lo_min = INT_MAX;
  for (int rr = 0; rr < nr; ++rr) {
    kv_max = max(kv_max, row_len(rr));
    lo_min = min(lo_min, row_lo(rr));
  }
  const int span = a.tps * kTile;
  const int bspan = kAttnWaves * span;
  const int blk_begin = blockIdx.y * bspan;
  // The group's blocks with work, [b_lo, b_hi): the others return at once.
  // With the combine fused, block 0 of a group with none still combines
  // (every row then gets the combine's output for no keys).
  const int b_lo = lo_min / bspan;
  const int b_hi = min((kv_max + bspan - 1) / bspan, a.nblk);
  const bool in_range = static_cast<int>(blockIdx.y) >= b_lo && static_cast<int>(blockIdx.y) < b_hi;
  if (!in_range && !(a.tags != nullptr && b_lo >= b_hi && blockIdx.y == 0)) return;
  const int t_begin = split * span;
  const int t_end_max = min(kv_max, t_begin + span);
  const bool active = split < a.splits && t_begin < kv_max && t_end_max > lo_min;
  const int t_first = max(t_begin, (lo_min / kTile) * kTile);
  const int* pt = a.row_pt != nullptr ? rpt_raw : a.d_pt;
  const g4_global_i32* ptg = (const g4_global_i32*)pt;  // global loads, not flat

  const uint8_t* kbase = a.k + static_cast<size_t>(hkv) * a.stride * kKb;
  const uint8_t* vbase = a.v + static_cast<size_t>(hkv) * a.stride * kVb;
  const float* kscb = kQuant ? a.ksc + static_cast<size_t>(hkv) * a.stride * kNgrp : nullptr;
  const float* vscb = kQuant ? a.vsc + static_cast<size_t>(hkv) * a.stride * kNgrp : nullptr;

  // Page-table entry of position p, loaded unconditionally from a clamped
  // index (a guarded load would be waited for inside its branch), and the
  // arena row it gives: -1 past the split's end or outside [0, stride)
  // (skipped like the append kernels skip them).
  const int p_last = max(t_end_max - 1, 0);
  auto pt_entry = [&](int p) { return pt != nullptr ? ptg[min(p, p_last)] : p; };
  auto arena_row_of = [&](int p, int r) { return (p < t_end_max && r >= 0 && r < a.stride) ? r : -1; };
  // Every load that depends only on the position is issued before the first
  // wait: the first tile's page-table entries, this lane's q (and, fused,
  // its cos / sin).
  int pt_next = active ? pt_entry(t_first + lane) : -1;

  // This lane's query column.
  const int rr = n >> 2, hq = hkv * kGq + (n & 3);
  const bool live = rr < nr;
  const int my_len = live ? row_len(rr) : 0;
  const int my_lo = live ? row_lo(rr) : 0;
  bf16x8_t qb[4];
  u32x4_t raw[4];
  float cs[2][8], sn[2][8];
  constexpr bool FUSE = MODE == kAttnRopeAppend;  // q rotated here
  const bool q_ok = FUSE ? (live && active && base >= 0 && base < a.ra.max_pos)
                                  : (live && active);
  {
    const uint16_t* qp = FUSE
                             ? a.ra.q + static_cast<size_t>(hq) * kHd
                             : a.q + (static_cast<size_t>(r0 + (live ? rr : 0)) * a.Hq + hq) * kHd;
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) raw[s4] = *reinterpret_cast<const u32x4_t*>(qp + 32 * s4 + 8 * g);
    if constexpr (FUSE) {
      const long long rp = q_ok ? base : 0;
#pragma unroll
      for (int s4 = 0; s4 < 2; ++s4) {
        const float* cp = a.ra.cos_t + rp * 64 + 32 * s4 + 8 * g;
        const float* sp = a.ra.sin_t + rp * 64 + 32 * s4 + 8 * g;
        *reinterpret_cast<float4*>(cs[s4]) = *reinterpret_cast<const float4*>(cp);
        *reinterpret_cast<float4*>(cs[s4] + 4) = *reinterpret_cast<const float4*>(cp + 4);
        *reinterpret_cast<float4*>(sn[s4]) = *reinterpret_cast<const float4*>(sp);
        *reinterpret_cast<float4*>(sn[s4] + 4) = *reinterpret_cast<const float4*>(sp + 4);
      }
    }
  }

  // Decode append: the one wave whose split holds the new position writes
  // its K / V row to the pool and keeps the same bytes in LDS, inside the
  // tile that holds the position once that tile's loads are in flight (its
  // own loads overlap them). The tile then takes the key from LDS: its pool
  // loads were issued before the store. A position outside the RoPE table
  // leaves K unwritten (as the append kernels do), so only V is taken.
  __shared__ __align__(16) uint8_t mir_k[kAttnWaves][2 * kHd];
  __shared__ __align__(16) uint8_t mir_v[kAttnWaves][2 * kHd];
  __shared__ float mir_s[kAttnWaves][2][kNgrp];
  const bool own_new = MODE != kAttnPlain && active && base >= t_begin && base < t_end_max;

  // q for the MFMAs: fused, rotated at the position, done in the first tile
  // once its loads are in flight (the cos / sin wait then overlaps them).
  auto make_q = [&] {
    if constexpr (FUSE) {
      // Raw q rotated at the position: the lane's dims 32 s + 8 g + j pair with
      // 32 (s + 2) + 8 g + j, so the rotation is lane-local; the same products
      // and roundings as the append kernels' rotate8 (out = a c + b' s with b'
      // the negated or plain partner), then bf16 RNE.
      uint32_t rot[4][4];
#pragma unroll
      for (int s4 = 0; s4 < 2; ++s4) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const uint32_t xa = raw[s4][w], xb = raw[s4 + 2][w];
          const float a0 = lo_bf16(xa), a1 = hi_bf16(xa), b0 = lo_bf16(xb), b1 = hi_bf16(xb);
          rot[s4][w] = pack_bf16_hw(a0 * cs[s4][2 * w] + (-b0) * sn[s4][2 * w],
                                    a1 * cs[s4][2 * w + 1] + (-b1) * sn[s4][2 * w + 1]);
          rot[s4 + 2][w] = pack_bf16_hw(b0 * cs[s4][2 * w] + a0 * sn[s4][2 * w],
                                        b1 * cs[s4][2 * w + 1] + a1 * sn[s4][2 * w + 1]);
        }
      }
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4)
        qb[s4] = q_ok ? as_bf16x8(rot[s4][0], rot[s4][1], rot[s4][2], rot[s4][3])
                      : as_bf16x8(0u, 0u, 0u, 0u);
    } else {
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4)
        qb[s4] = __builtin_bit_cast(bf16x8_t, q_ok ? raw[s4] : u32x4_t{0u, 0u, 0u, 0u});
    }
  };
  f32x4_t o[8];
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) o[nb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  float m = -INFINITY, l = 0.0f;
  int new_row = -1;  // arena row of the appended key once its LDS copy is made
  for (int t0 = active ? t_first : t_end_max; t0 < t_end_max; t0 += kTile) {
    // Arena row of key t0 + lane; the next tile's entry is fetched a tile ahead.
    const int prow = arena_row_of(t0 + lane, pt_next);
    if (t0 + kTile < t_end_max) pt_next = pt_entry(t0 + kTile + lane);
    // Every K and V load of the tile first (one memory round trip), then V
    // and the scales to LDS.
    // The appended row's inputs, issued before the tile's loads so that the
    // wait for them does not include the tile: lanes 0-15 the key head (and
    // its cos / sin), 16-31 the value head, 8 dims per lane, no branch.
    const bool new_tile = own_new && base >= t0 && base < t0 + kTile;  // wave-uniform
    V8 nx;
    float ncs[8], nsn[8];
    if (new_tile) {
      const int l16 = lane & 15;
      const uint16_t* src = (lane < 16 ? a.ra.k : a.ra.v) + hkv * kHd + 8 * l16;
      nx = ld8(src);
      if constexpr (FUSE) {
        const long long rp = base < a.ra.max_pos ? base : 0;
        const float* cp = a.ra.cos_t + rp * 64 + 8 * (l16 & 7);
        const float* sp = a.ra.sin_t + rp * 64 + 8 * (l16 & 7);
        *reinterpret_cast<float4*>(ncs) = *reinterpret_cast<const float4*>(cp);
        *reinterpret_cast<float4*>(ncs + 4) = *reinterpret_cast<const float4*>(cp + 4);
        *reinterpret_cast<float4*>(nsn) = *reinterpret_cast<const float4*>(sp);
        *reinterpret_cast<float4*>(nsn + 4) = *reinterpret_cast<const float4*>(sp + 4);
      }
    }
    // V straight to LDS: the plain bf16 kernel (two waves per SIMD with it).
    // The decode-append forms stay at one wave per SIMD either way, and there
    // the copy through registers measured faster: a 40-layer decode step with
    // the append in the attention 2285-2288 us against 2307-2310 us.
    constexpr bool kVDma = BITS == 16 && MODE == kAttnPlain;
    u32x4_t vraw[VStage<BITS>::kSteps];
    if constexpr (kVDma) v_dma_bf16(vbase, prow, vl);
    else v_load<BITS>(vbase, prow, vraw);
    u32x4_t kraw[4][4];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
      const int kr = __shfl(prow, 16 * mb + n);  // key 16 mb + n: the A row of this lane
      const uint8_t* krow = kbase + static_cast<size_t>(kr >= 0 ? kr : 0) * kKb;
#pragma unroll
      for (int s = 0; s < 4; ++s) kraw[mb][s] = load_k_raw<BITS>(krow, 32 * s + 8 * g);
    }
    if (t0 == t_first) make_q();
    float ksr[kNgrp], vsr[kNgrp];
    if constexpr (kQuant) {
#pragma unroll
      for (int gi = 0; gi < kNgrp; ++gi) {
        const size_t si = static_cast<size_t>(prow >= 0 ? prow : 0) * kNgrp + gi;
        ksr[gi] = kscb[si];
        vsr[gi] = vscb[si];
      }
    }
    if (new_tile) {
      // The appended key: K rotated as the append kernels' rope_unit does it
      // (rotate8, bf16, then the code of the rotated value or of its bf16
      // rounding), V as is, both quantised by store_quant into this wave's
      // LDS copy of the row. Lanes 32-63 compute the same and write nothing.
      const int j = base - t0;
      const int pj = __shfl(prow, j);
      const int l16 = lane & 15;
      const bool is_k = lane < 16;
      // kAttnAppend: k is the rotated bf16 row already (its code is that of
      // the bf16 value, the decode append's rounding).
      float rot[8];
      V8 rb = nx;
      if constexpr (FUSE) {
        rotate8(nx, ncs, nsn, l16 < 8, rot);
        rb = to_bf16x8(rot);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) rot[e] = v8_get(nx, e);
      }
      if (lane < 32) {
        if constexpr (BITS == 16) {
          st8(reinterpret_cast<uint16_t*>(is_k ? mir_k[wave] : mir_v[wave]) + 8 * l16, is_k ? rb : nx);
        } else {
          float val[8];
#pragma unroll
          for (int e = 0; e < 8; ++e)
            val[e] = is_k ? (a.ra.k_round ? v8_get(rb, e) : rot[e]) : v8_get(nx, e);
          store_quant<BITS, GROUP>(a.ra, val, is_k, 0, l16,
                                   RowSink{mir_k[wave], mir_v[wave], mir_s[wave][0], mir_s[wave][1]});
        }
      }
      wave_lds_sync();
      const bool k_new = base < a.ra.max_pos;
      new_row = pj;
      if (pj >= 0) {
        if (k_new) {
#pragma unroll
          for (int mb = 0; mb < 4; ++mb) {
            if (mb == (j >> 4) && n == (j & 15)) {
#pragma unroll
              for (int s = 0; s < 4; ++s) kraw[mb][s] = load_k_raw<BITS>(mir_k[wave], 32 * s + 8 * g);
            }
          }
        }
        if constexpr (!kVDma) {  // the append forms stage V through registers
          using VS = VStage<BITS>;
#pragma unroll
          for (int i = 0; i < VS::kSteps; ++i) {
            const int key = i * (64 / VS::kChunks) + lane / VS::kChunks, c = lane % VS::kChunks;
            if (key == j) vraw[i] = *reinterpret_cast<const u32x4_t*>(mir_v[wave] + 16 * c);
          }
        }
        if constexpr (kQuant) {
          if (lane == j) {
#pragma unroll
            for (int gi = 0; gi < kNgrp; ++gi) {
              if (k_new) ksr[gi] = mir_s[wave][0][gi];
              vsr[gi] = mir_s[wave][1][gi];
            }
          }
        }
      }
    }
    const unsigned long long kvalid = __ballot(prow >= 0);
    const auto store_scales = [&] {
      if constexpr (kQuant) {
#pragma unroll
        for (int gi = 0; gi < kNgrp; ++gi) {
          ksc_at(lane, gi) = prow >= 0 ? ksr[gi] : 0.0f;
          vsc_at(lane, gi) = prow >= 0 ? vsr[gi] : 0.0f;
        }
      }
    };
    if constexpr (kVDma) {
      // Every load of the tile has landed (the K loads, issued after the V
      // tile's, are needed next anyway); then the tile's fix-ups.
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      v_fix_bf16(vl, kvalid);
    } else if constexpr (kDeq) {
      store_scales();
      wave_lds_sync();  // the scales, read per key below
      v_store_deq<BITS, GROUP>(vraw, vl, kvalid, vsc_at);
    } else {
      v_store<BITS>(vraw, vl, kvalid);
    }
    if constexpr (!kDeq) store_scales();
    wave_lds_sync();  // V tile and scales in LDS
    // S^T = K Q^T per 16-key block mb: lane l holds keys 16 mb + 4 g + i.
    float sv[4][4];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
      bf16x8_t ka[4];
      if constexpr (kDeq) {
        // this lane's A row, key 16 mb + n, dims 32 s + 8 g ..: group 32 s / GROUP
#pragma unroll
        for (int s = 0; s < 4; ++s) ka[s] = k_raw_deq<BITS>(kraw[mb][s], ksc_at(16 * mb + n, (32 * s) / GROUP));
      } else {
#pragma unroll
        for (int s = 0; s < 4; ++s) ka[s] = k_raw_bf16<BITS>(kraw[mb][s]);
      }
      f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int s = 0; s < 4; ++s) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[s], qb[s], acc, 0, 0, 0);
      if constexpr (kQB) {  // one scale per row
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = acc[i] * ksc_at(16 * mb + 4 * g + i, 0);
      }
      // logit = bf16(scale * dot), two per hardware conversion (equal to the
      // integer rounding for every non-NaN value)
      const uint32_t lg01 = pack_bf16_hw(a.scale * acc[0], a.scale * acc[1]);
      const uint32_t lg23 = pack_bf16_hw(a.scale * acc[2], a.scale * acc[3]);
      const float lg[4] = {lo_bf16(lg01), hi_bf16(lg01), lo_bf16(lg23), hi_bf16(lg23)};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int p = t0 + 16 * mb + 4 * g + i;
        const bool ok = live && p < my_len && p >= my_lo && ((kvalid >> (16 * mb + 4 * g + i)) & 1ull);
        sv[mb][i] = ok ? lg[i] : -INFINITY;
      }
    }
    // Online softmax of this lane's query row over the tile.
    float mx = m;
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int i = 0; i < 4; ++i) mx = fmaxf(mx, sv[mb][i]);
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float alpha = mx == -INFINITY ? 1.0f : __expf(m - mx);
    m = mx;
    l *= alpha;
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) o[nb] *= alpha;
    float e[4][4];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        e[mb][i] = m == -INFINITY ? 0.0f : __expf(sv[mb][i] - m);
        l += e[mb][i];
      }
    // O^T += V^T P^T, two 32-key steps: contraction slot j -> key 32 s + 4 g + j
    // (j < 4) or 32 s + 16 + 4 g + j - 4.
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      bf16x8_t pb[kNgrpB];
#pragma unroll
      for (int gi = 0; gi < kNgrpB; ++gi) {
        float pv[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int mb = 2 * s + (j >> 2), i = j & 3;
          const float sc = kQB ? vsc_at(16 * mb + 4 * g + i, gi) : 1.0f;
          pv[j] = e[mb][i] * sc;
        }
        pb[gi] = as_bf16x8(pack_bf16_hw(pv[0], pv[1]), pack_bf16_hw(pv[2], pv[3]),
                           pack_bf16_hw(pv[4], pv[5]), pack_bf16_hw(pv[6], pv[7]));
      }
      const int kk = n >> 2, dd = 4 * (n & 3);
      const int vrow = 32 * s + 4 * g + kk;  // and vrow + 16 (same swizzle)
      const uint16_t* r1 = vl + vrow * (kVDma ? kHd : kVPitch) + dd;
      const uint16_t* r2 = r1 + 16 * (kVDma ? kHd : kVPitch);
      const int vt = vrow & 7;
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) {
        // bf16 (swizzled): dims 16 nb + dd.. sit in chunk pair nb ^ (row & 7).
        const int co = kVDma ? 16 * (nb ^ vt) : 16 * nb;
        const u32x2_t lo = lds_read_tr(r1 + co);
        const u32x2_t hi = lds_read_tr(r2 + co);
        const bf16x8_t va = as_bf16x8(lo.x, lo.y, hi.x, hi.y);
        const int gi = kQB ? (16 * nb) / GROUP : 0;
        o[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pb[gi], o[nb], 0, 0, 0);
      }
    }
    wave_lds_sync();  // this tile's LDS reads are done before the next tile's writes
  }
  // l: sum over the four lanes of this query column.
  l += __shfl_xor(l, 16);
  l += __shfl_xor(l, 32);

  // Merge the block's kAttnWaves splits (the combine's formula over these
  // splits): per query column, M = max m_w, w_w = exp(m_w - M), then one
  // partial (M, sum l_w w_w, sum o_w w_w) per (row, head, block).
  __syncthreads();  // every wave's last tile reads are done: vl_all is free
  float* mo = reinterpret_cast<float*>(&vl_all[0][0]);  // [wave][16 cols][128 dims]
  float* mml = mo + kAttnWaves * 16 * kHd;              // [wave][16 cols][2]
  static_assert(sizeof(vl_all) >= sizeof(float) * kAttnWaves * 16 * (kHd + 2), "merge area");
#pragma unroll
  for (int nb = 0; nb < 8; ++nb)
    *reinterpret_cast<f32x4_t*>(mo + (wave * 16 + n) * kHd + 16 * nb + 4 * g) = o[nb];
  if (g == 0) {
    const bool has = active && live && t_begin < my_len && t_end_max > my_lo;
    mml[(wave * 16 + n) * 2] = has ? m : -INFINITY;
    mml[(wave * 16 + n) * 2 + 1] = has ? l : 0.0f;
  }
  __syncthreads();
  {
    const int col = threadIdx.x >> 4, dc = threadIdx.x & 15;  // 16 columns x 8 dims each
    const int crr = col >> 2, chq = hkv * kGq + (col & 3);
    if (new_row >= 0) {
      // The appended row from LDS to the pool, last: nothing in this wave
      // waits for these stores (k: lanes 0-15, v: 16-31, scales: 32-39).
      const size_t slot = static_cast<size_t>(hkv) * a.stride + new_row;
      const bool k_new = base < a.ra.max_pos;
      if (lane < 16) {
        if (k_new && 16 * lane < kKb)
          *reinterpret_cast<u32x4_t*>(static_cast<uint8_t*>(a.ra.cache_k) + slot * kKb + 16 * lane) =
              *reinterpret_cast<const u32x4_t*>(mir_k[wave] + 16 * lane);
      } else if (lane < 32) {
        const int c = lane - 16;
        if (16 * c < kVb)
          *reinterpret_cast<u32x4_t*>(static_cast<uint8_t*>(a.ra.cache_v) + slot * kVb + 16 * c) =
              *reinterpret_cast<const u32x4_t*>(mir_v[wave] + 16 * c);
      } else if (kQuant && lane < 32 + 2 * kNgrp) {
        const int gi = (lane - 32) % kNgrp;
        const bool is_k = lane - 32 < kNgrp;
        if (is_k ? k_new : true)
          (is_k ? a.ra.k_scale : a.ra.v_scale)[slot * kNgrp + gi] = mir_s[wave][is_k ? 0 : 1][gi];
      }
    }
    // A block with no key of the row (its positions all unmapped) publishes
    // (-inf, 0, 0), which the combine weighs with 0, instead of leaving the
    // previous call's partial in its slot.
    if (crr < nr) {
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < kAttnWaves; ++w) M = fmaxf(M, mml[(w * 16 + col) * 2]);
      float L = 0.0f, acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int w = 0; w < kAttnWaves; ++w) {
        const float mw = mml[(w * 16 + col) * 2];
        const float wt = mw == -INFINITY ? 0.0f : expf(mw - M);
        L += mml[(w * 16 + col) * 2 + 1] * wt;
        const float* ow = mo + (w * 16 + col) * kHd + 8 * dc;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] += ow[e] * wt;
      }
      const size_t slot = (static_cast<size_t>(r0 + crr) * a.Hq + chq) * a.nblk + blockIdx.y;
      if (dc == 0) st_dev_u64(a.part_ml + slot, f2_bits(M, L));
      float* po = a.part_o + slot * kHd + 8 * dc;
#pragma unroll
      for (int e = 0; e < 8; e += 2) st_dev_u64(po + e, f2_bits(acc[e], acc[e + 1]));
    }
  }
  if (a.tags == nullptr) return;

  // Combine fused: the group's last block with work (b_hi - 1; block 0 of a
  // group with none) combines. The others publish their tag once their
  // partials are stored and exit; the combining block polls the group's tags
  // (one per lane, bounded), clears them (so a graph replay, which reuses
  // the tag, starts from zeros) and combines. Its wait cannot starve the
  // blocks it waits for: they have lower workgroup ids, and each XCD
  // dispatches its workgroups in id order, so the lowest unfinished
  // workgroup of the launch can always be dispatched and depends only on
  // finished ones. A wait that gives up after the spin limit (which that
  // excludes) writes NaN outputs rather than hang.
  const bool combiner = b_lo < b_hi ? static_cast<int>(blockIdx.y) == b_hi - 1 : blockIdx.y == 0;
  unsigned* gt = a.tags + (static_cast<size_t>(blockIdx.z) * gridDim.x + hkv) * a.nblk;
  wait_stores();
  __syncthreads();
  if (!combiner) {
    if (threadIdx.x == 0)
      __hip_atomic_store(gt + blockIdx.y, a.tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  __shared__ int s_ok;
  if (wave == 0) {
    const int b = b_lo + lane;
    const bool mine = b < b_hi - 1;  // every block with work but this one
    bool seen = !mine;
    int spin = 0;
    // A spin limit of 0 (the test hook) gives up before polling, so the
    // outcome does not depend on timing.
    const bool forced = a.spin_limit <= 0;
    while (!forced) {
      if (!seen) seen = __hip_atomic_load(gt + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == a.tag;
      if (__all(seen) || ++spin >= a.spin_limit) break;
      __builtin_amdgcn_s_sleep(1);
    }
    // Only slots seen carrying the tag are cleared: an unseen block may
    // still store its tag after a give-up, so its slot is left alone, and
    // the give-up is recorded in the sticky error word for the host, which
    // then zero-fills the scratch before the next call.
    if (mine && seen) __hip_atomic_store(gt + b, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool ok = !forced && __all(seen);
    if (lane == 0) {
      s_ok = ok;
      if (!ok) __hip_atomic_store(a.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __syncthreads();
  if (!s_ok) {
    for (int rr = 0; rr < nr; ++rr)
      *reinterpret_cast<uint32_t*>(a.out + (static_cast<size_t>(r0 + rr) * a.Hq + hkv * kGq + wave) * kHd +
                                   2 * lane) = 0x7fc07fc0u;
    return;
  }
  for (int rr = 0; rr < nr; ++rr)
    combine_wave(a, r0 + rr, hkv * kGq + wave, a.row_pos != nullptr ? row_pos0 + 1 : base + r0 + rr + 1);
}

// The combine as its own launch (the split launch without tags): one
// workgroup per (row, 4 heads), one wave per head.
constexpr int kCombineThreads = kGq * 64;

__global__ __launch_bounds__(kCombineThreads) void attn_combine_kernel(AttnArgs a) {
  // The arguments fetched in one scalar round trip.
  asm volatile("" ::"s"(a.d_pos), "s"(a.row_pos), "s"(a.part_ml), "s"(a.part_o), "s"(a.out),
               "s"(a.nblk), "s"(a.tps), "s"(a.stride), "s"(a.window), "s"(a.kv_base), "s"(a.Hq));
  const int len = combine_len(a, blockIdx.y);  // loaded before the partials
  combine_wave(a, blockIdx.y, blockIdx.x * kGq + (threadIdx.x >> 6), len);
}

// ---------------------------------------------------------------------------
// Causal prefill attention over the pool (prefill_gemm.cu:626-1188,
// prefill_attention :1392-1474): query rows at positions base + r, each
// attending to [lo, base + r] in one pass of 64-position tiles.
//
// One workgroup = one KV head x 16 consecutive positions: its 4 waves each
// own 4 positions x the 4 query heads (16 MFMA columns, the decode wave's
// layout), and share every K / V tile, which the 256 lanes stage into LDS
// once (codes converted to exact bf16 integers, scales alongside). Per tile
// each wave runs S^T = K Q^T with A read from the K tile, the causal / window
// mask, the online softmax, and O^T += V^T P^T as the decode kernel does; the
// output is bf16(o * (1 / l)) (prefill_gemm.cu:930-940).
// ---------------------------------------------------------------------------
constexpr int kKPitch = kHd + 8;  // K tile pitch (bf16): 272 B, 16 rows on distinct banks
// Waves per prefill workgroup (template parameter W): 8, or 4 where 8-wave
// workgroups would not give every CU one. Staging a tile's K / V into LDS is
// split over all of them, so more waves sharing a tile cost less staging per
// score; fewer waves per workgroup give short prompts more workgroups.
// Measured: T=8192 at 57344 K5V4 8 waves 23.6 ms, 4 waves 48.5 ms; T=512
// int8 (128 8-wave workgroups) 23.3 us, 4 waves 21.5 us.

struct PrefillArgs {
  const uint16_t* q;  // [rows][Hq][128]
  const uint8_t* k;
  const uint8_t* v;
  const float* ksc;
  const float* vsc;
  float scale;
  int Hq, stride, rows, base, window;
  const int* d_pt;
  uint16_t* out;      // [rows][Hq][128]
};

// Staging of keys [j0, j0 + 64) for all 4 waves, pipelined: a tile's raw
// bytes (K / V chunks, scales, arena rows) are loaded into registers one tile
// ahead (prefill_load, issued before the current tile's compute), then
// converted into the LDS tile (prefill_store: K codes as exact bf16
// integers, V as the decode staging does, scales alongside, zeros for keys
// without a row). The page-table entries of a tile are loaded a tile before
// its bytes, so no load waits for another inside the loop. Loads are
// unconditional (row 0 for keys without a row, masked when stored).
// Measured against staging each tile after the previous one's compute:
// T=512 int8 33.7 -> 29.6 us, T=8192 at 57344 K5V4 38.3 -> 35.1 ms.
template <int BITS, int GROUP, int W>
struct PrefillRaw {
  static constexpr int kPrefThreads = W * 64;
  static constexpr bool kQuant = BITS != 16;
  static constexpr int kNgrp = kQuant ? kHd / GROUP : 1;
  static constexpr bool kDeq = kv_deq<BITS, GROUP>();  // staged dequantised
  static constexpr int kKElems = BITS == 16 ? 8 : BITS == 8 ? 16 : 32;  // per K chunk
  static constexpr int kKRowChunks = kHd / kKElems;
  static constexpr int kKIt = (kTile * kKRowChunks + kPrefThreads - 1) / (kPrefThreads);
  static constexpr int kVRowChunks = VStage<BITS>::kChunks;
  static constexpr int kVIt = (kTile * kVRowChunks + kPrefThreads - 1) / (kPrefThreads);
  // V chunks start on the thread after the last K chunk's, so a tile whose K
  // chunks fill only part of the workgroup puts its V on the idle threads.
  static constexpr int kVShift = (kTile * kKRowChunks) % kPrefThreads;
  u32x4_t k[kKIt][kKElems / 8];
  u32x4_t v[kVIt];
  float ksc[kKIt][kNgrp], vsc[kKIt][kNgrp];
  float vsd[kDeq ? kVIt : 1];  // kDeq: each V chunk's group scale
  int kr[kKIt], vr[kVIt];  // arena rows (-1: no row)
};

// Page-table entries of tile j0's keys for this thread's K and V chunks.
template <int BITS, int GROUP, int W>
__device__ __forceinline__ void prefill_pt(const PrefillArgs& a, int j0, int kv_end,
                                           int (&ptk)[PrefillRaw<BITS, GROUP, W>::kKIt],
                                           int (&ptv)[PrefillRaw<BITS, GROUP, W>::kVIt], int t) {
  using R = PrefillRaw<BITS, GROUP, W>;
  constexpr int kPrefThreads = R::kPrefThreads;
  const int tv = (t + R::kVShift) % kPrefThreads;
  const int last = max(kv_end - 1, 0);
#pragma unroll
  for (int it = 0; it < R::kKIt; ++it) {
    const int key = min((t + it * kPrefThreads) / R::kKRowChunks, kTile - 1);
    const int p = j0 + key;
    ptk[it] = a.d_pt != nullptr ? a.d_pt[min(p, last)] : p;
  }
#pragma unroll
  for (int it = 0; it < R::kVIt; ++it) {
    const int key = min((tv + it * kPrefThreads) / R::kVRowChunks, kTile - 1);
    const int p = j0 + key;
    ptv[it] = a.d_pt != nullptr ? a.d_pt[min(p, last)] : p;
  }
}

template <int BITS, int GROUP, int W>
__device__ __forceinline__ void prefill_load(const PrefillArgs& a, const uint8_t* kbase,
                                             const uint8_t* vbase, const float* kscb,
                                             const float* vscb, int j0, int kv_end,
                                             const int (&ptk)[PrefillRaw<BITS, GROUP, W>::kKIt],
                                             const int (&ptv)[PrefillRaw<BITS, GROUP, W>::kVIt],
                                             PrefillRaw<BITS, GROUP, W>& raw, int t) {
  using R = PrefillRaw<BITS, GROUP, W>;
  constexpr int kPrefThreads = R::kPrefThreads;
  constexpr int kKb = k_row_bytes(BITS);
  const int tv = (t + R::kVShift) % kPrefThreads;
  auto valid = [&](int key, int r) {
    return (j0 + key < kv_end && r >= 0 && r < a.stride) ? r : -1;
  };
#pragma unroll
  for (int it = 0; it < R::kKIt; ++it) {
    const int idx = t + it * kPrefThreads;
    raw.kr[it] = -1;
    if (idx >= kTile * R::kKRowChunks) continue;  // no K chunk (whole waves)
    const int key = idx / R::kKRowChunks;
    const int c = (idx % R::kKRowChunks) * R::kKElems;
    const int pr = valid(key, ptk[it]);
    raw.kr[it] = pr;
    const uint8_t* row = kbase + static_cast<size_t>(pr >= 0 ? pr : 0) * kKb;
#pragma unroll
    for (int h = 0; h < R::kKElems / 8; ++h) raw.k[it][h] = load_k_raw<BITS>(row, c + 8 * h);
    if constexpr (R::kQuant) {
      const size_t si = static_cast<size_t>(pr >= 0 ? pr : 0) * R::kNgrp;
#pragma unroll
      for (int gi = 0; gi < R::kNgrp; ++gi) {
        raw.ksc[it][gi] = kscb[si + gi];
        raw.vsc[it][gi] = vscb[si + gi];
      }
    }
  }
#pragma unroll
  for (int it = 0; it < R::kVIt; ++it) {
    const int idx = tv + it * kPrefThreads;
    raw.vr[it] = -1;
    if (idx >= kTile * R::kVRowChunks) continue;  // no V chunk (whole waves)
    const int key = idx / R::kVRowChunks;
    const int c = idx % R::kVRowChunks;
    const int pr = valid(key, ptv[it]);
    raw.vr[it] = pr;
    raw.v[it] = *reinterpret_cast<const u32x4_t*>(
        vbase + static_cast<size_t>(pr >= 0 ? pr : 0) * VStage<BITS>::kRowB + 16 * c);
    if constexpr (R::kDeq)
      raw.vsd[it] = vscb[static_cast<size_t>(pr >= 0 ? pr : 0) * R::kNgrp +
                         (c * (kHd / R::kVRowChunks)) / GROUP];
  }
}

template <int BITS, int GROUP, int W>
__device__ __forceinline__ void prefill_store(const PrefillRaw<BITS, GROUP, W>& raw, uint16_t* ks,
                                              uint16_t* vs, float* ksc_l, float* vsc_l,
                                              unsigned* s_valid, float kmul, int t) {
  using R = PrefillRaw<BITS, GROUP, W>;
  constexpr int kPrefThreads = R::kPrefThreads;
  const int tv = (t + R::kVShift) % kPrefThreads;
#pragma unroll
  for (int it = 0; it < R::kKIt; ++it) {
    const int idx = t + it * kPrefThreads;
    if (idx >= kTile * R::kKRowChunks) break;
    const int key = idx / R::kKRowChunks, c = (idx % R::kKRowChunks) * R::kKElems;
    const int pr = raw.kr[it];
    uint16_t* dst = ks + key * kKPitch + c;
#pragma unroll
    for (int h = 0; h < R::kKElems / 8; ++h) {
      bf16x8_t kv = __builtin_bit_cast(bf16x8_t, u32x4_t{0u, 0u, 0u, 0u});
      if constexpr (R::kDeq) {
        // the chunk's group scale, selected without indexing registers at run time
        const int gsel = (c + 8 * h) / GROUP;
        float sk = raw.ksc[it][0];
#pragma unroll
        for (int gi = 1; gi < R::kNgrp; ++gi) sk = gi == gsel ? raw.ksc[it][gi] : sk;
        if (pr >= 0) kv = k_raw_deq<BITS>(raw.k[it][h], sk);
      } else {
        if (pr >= 0) kv = k_raw_bf16<BITS>(raw.k[it][h]);
      }
      *reinterpret_cast<bf16x8_t*>(dst + 8 * h) = kv;
    }
    if (c == 0) {
      if constexpr (R::kQuant && !R::kDeq) {
#pragma unroll
        for (int gi = 0; gi < R::kNgrp; ++gi) {
          ksc_l[key * R::kNgrp + gi] = pr >= 0 ? raw.ksc[it][gi] * kmul : 0.0f;
          vsc_l[key * R::kNgrp + gi] = pr >= 0 ? raw.vsc[it][gi] : 0.0f;
        }
      }
      s_valid[key] = pr >= 0 ? 1u : 0u;
    }
  }
#pragma unroll
  for (int it = 0; it < R::kVIt; ++it) {
    const int idx = tv + it * kPrefThreads;
    if (idx >= kTile * R::kVRowChunks) break;
    const int key = idx / R::kVRowChunks, c = idx % R::kVRowChunks;
    const uint32_t z = BITS == 16 || BITS == 8 ? 0u : 0x88888888u;
    const u32x4_t u = raw.vr[it] >= 0 ? raw.v[it] : u32x4_t{z, z, z, z};
    if constexpr (R::kDeq) {
      constexpr int kDims = kHd / R::kVRowChunks;
      uint32_t w[BITS == 8 ? 8 : 16];
      v_chunk_deq<BITS>(u, raw.vr[it] >= 0 ? raw.vsd[it] : 0.0f, w);
      uint16_t* dst = vs + key * kVPitch + kDims * c;
#pragma unroll
      for (int e = 0; e < kDims / 8; ++e)
        *reinterpret_cast<u32x4_t*>(dst + 8 * e) = u32x4_t{w[4 * e], w[4 * e + 1], w[4 * e + 2], w[4 * e + 3]};
    } else if constexpr (BITS == 16) {
      *reinterpret_cast<u32x4_t*>(vs + key * kVPitch + 8 * c) = u;
    } else if constexpr (BITS == 8) {
      uint32_t w[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t x = u[e >> 1];
        const int sh = 16 * (e & 1);
        w[e] = int_pair_bf16(static_cast<int8_t>(x >> sh), static_cast<int8_t>(x >> (sh + 8)));
      }
      uint16_t* dst = vs + key * kVPitch + 16 * c;
      *reinterpret_cast<u32x4_t*>(dst) = u32x4_t{w[0], w[1], w[2], w[3]};
      *reinterpret_cast<u32x4_t*>(dst + 8) = u32x4_t{w[4], w[5], w[6], w[7]};
    } else {
      uint32_t w[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const uint32_t x = u[e >> 2];
        const int b = 8 * (e & 3);
        w[e] = int4_pair_bf16(x ^ 0x88888888u, b);
      }
      uint16_t* dst = vs + key * kVPitch + 32 * c;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        *reinterpret_cast<u32x4_t*>(dst + 8 * e) = u32x4_t{w[4 * e], w[4 * e + 1], w[4 * e + 2], w[4 * e + 3]};
    }
  }
}

// CB: column blocks per wave (4 CB positions x 4 heads each); the K and V^T
// fragments read from LDS serve all CB blocks, and a staged tile serves
// 16 CB positions.
// KSP = 2 (W = 8): the keys split inside the workgroup. Two 4-wave groups own
// the same 16 positions (waves w and w + 4 the same 4); group k stages and
// runs tiles j_first + (2 i + k) * 64 through its own two tile buffers, and
// at the end group 1's (m, l, o) merge into group 0's through LDS
// (M = max m, each side's o and l scaled by exp(m - M)). Two waves per SIMD
// where a short prompt gives each CU one 16-position workgroup.
template <int BITS, int GROUP, int CB, int W, int KSP = 1>
__global__ __launch_bounds__(W * 64) void attn_prefill_kernel(PrefillArgs a) {
  static_assert(KSP == 1 || (KSP == 2 && W == 8), "key split: two 4-wave groups");
  constexpr int kPrefWaves = W / KSP;  // waves owning positions (and staging a tile)
  constexpr bool kQuant = BITS != 16;
  constexpr int kNgrp = kQuant ? kHd / GROUP : 1;
  constexpr bool kQB = kQuant && !kv_deq<BITS, GROUP>();  // codes and row scales in the products
  constexpr int kNgrpB = kQB ? kNgrp : 1;
  constexpr int kKb = k_row_bytes(BITS), kVb = v_row_bytes(BITS);
  constexpr int kPos = kPrefWaves * 4 * CB;  // positions per workgroup
  // Two tile buffers per key group: tile t + 1 is staged into one while tile
  // t is read from the other, with one barrier per tile.
  __shared__ __align__(16) uint16_t ks2[KSP][2][kTile * kKPitch];
  __shared__ __align__(16) uint16_t vs2[KSP][2][kTile * kVPitch];
  __shared__ float ksc2[KSP][2][kTile * kNgrp], vsc2[KSP][2][kTile * kNgrp];
  __shared__ unsigned valid2[KSP][2][kTile];

  const int lane = threadIdx.x & 63;
  const int gk = KSP == 2 ? static_cast<int>(threadIdx.x >> 8) : 0;  // key group
  const int wave = static_cast<int>(threadIdx.x >> 6) & (kPrefWaves - 1);
  const int tst = threadIdx.x & (kPrefWaves * 64 - 1);  // staging thread within the group
  const int g = lane >> 4, n = lane & 15;
  // Longest rows first: the dispatch order (x fastest) walks every KV head of
  // the last position block, then of the one before it, so the longest causal
  // rows start first and the shortest end the launch. Measured (int8 from
  // position 0, against position blocks in order): T=4096 451 -> 270 us,
  // T=8192 1349 -> 966 us; K5V4 T=8192 at 57344 14.79 -> 14.01 ms; T <= 2048
  // unchanged (one round of workgroups).
  const int lin = blockIdx.x + blockIdx.y * gridDim.x;
  const int hkv = lin % gridDim.y;
  const int p0 = (gridDim.x - 1 - lin / gridDim.y) * kPos;
  const int hq = hkv * kGq + (n & 3);
  int r[CB], my_pos[CB], my_lo[CB];
  bool live[CB];
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) {
    r[cb] = p0 + 4 * (CB * wave + cb) + (n >> 2);  // this lane's query row in block cb
    live[cb] = r[cb] < a.rows;
    my_pos[cb] = a.base + r[cb];
    my_lo[cb] = a.window > 0 ? max(0, my_pos[cb] + 1 - a.window) : 0;
  }
  const int last = min(p0 + kPos, a.rows) - 1;
  const int kv_end = min(a.base + last + 1, a.stride);
  const int j_first = a.window > 0 ? (max(0, a.base + p0 + 1 - a.window) / kTile) * kTile : 0;

  bf16x8_t qb[CB][4];
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) {
    const uint16_t* qp = a.q + (static_cast<size_t>(live[cb] ? r[cb] : 0) * a.Hq + hq) * kHd;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      u32x4_t u = {0u, 0u, 0u, 0u};
      if (live[cb]) u = *reinterpret_cast<const u32x4_t*>(qp + 32 * s + 8 * g);
      qb[cb][s] = __builtin_bit_cast(bf16x8_t, u);
    }
  }
  const uint8_t* kbase = a.k + static_cast<size_t>(hkv) * a.stride * kKb;
  const uint8_t* vbase = a.v + static_cast<size_t>(hkv) * a.stride * kVb;
  const float* kscb = kQuant ? a.ksc + static_cast<size_t>(hkv) * a.stride * kNgrp : nullptr;
  const float* vscb = kQuant ? a.vsc + static_cast<size_t>(hkv) * a.stride * kNgrp : nullptr;

  f32x4_t o[CB][8];
  float m[CB], l[CB];
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) {
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) o[cb][nb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    m[cb] = -INFINITY;
    l[cb] = 0.0f;
  }

  // The wave's columns span positions [wave_pos_min, wave_pos_min + 4 CB);
  // the last one's window starts at wave_lo_max.
  const int wave_row0 = p0 + 4 * CB * wave;
  const bool wave_live = wave_row0 + 4 * CB - 1 < a.rows;
  const int wave_pos_min = a.base + wave_row0;
  const int wave_lo_max = a.window > 0 ? max(0, wave_pos_min + 4 * CB - a.window) : 0;

  constexpr int PW = kPrefWaves;
  using Raw = PrefillRaw<BITS, GROUP, PW>;
  Raw raw;
  int ptk[Raw::kKIt], ptv[Raw::kVIt];
  constexpr int kStep = KSP * kTile;    // between a group's tiles
  const int jg = j_first + gk * kTile;  // this group's first tile
  if (jg < kv_end) {
    prefill_pt<BITS, GROUP, PW>(a, jg, kv_end, ptk, ptv, tst);
    prefill_load<BITS, GROUP, PW>(a, kbase, vbase, kscb, vscb, jg, kv_end, ptk, ptv, raw, tst);
    prefill_pt<BITS, GROUP, PW>(a, jg + kStep, kv_end, ptk, ptv, tst);
    prefill_store<BITS, GROUP, PW>(raw, ks2[gk][0], vs2[gk][0], ksc2[gk][0], vsc2[gk][0],
                                   valid2[gk][0], a.scale, tst);
    if (jg + kStep < kv_end) {
      prefill_load<BITS, GROUP, PW>(a, kbase, vbase, kscb, vscb, jg + kStep, kv_end, ptk, ptv, raw, tst);
      prefill_pt<BITS, GROUP, PW>(a, jg + 2 * kStep, kv_end, ptk, ptv, tst);
    }
  }
  __syncthreads();
  // Both groups run the same number of steps (one barrier each); group 1
  // idles through the last when the tile count is odd.
  const int steps = kv_end > j_first ? (kv_end - j_first + kStep - 1) / kStep : 0;
  int buf = 0;
  for (int it = 0; it < steps; ++it, buf ^= 1) {
    const int j0 = jg + it * kStep;
    if (KSP == 2 && j0 >= kv_end) {
      __syncthreads();
      continue;
    }
    const uint16_t* ks = ks2[gk][buf];
    const uint16_t* vs = vs2[gk][buf];
    const float* ksc_l = ksc2[gk][buf];
    const float* vsc_l = vsc2[gk][buf];
    const unsigned* s_valid = valid2[gk][buf];
    // A tile that every column of this wave sees whole (all keys at or below
    // the wave's first position, at or above its last window start, each with
    // an arena row) takes the form without the mask.
    const bool full = wave_live && j0 + kTile - 1 <= wave_pos_min && j0 >= wave_lo_max &&
                      __all(s_valid[lane] != 0u);
    auto tile = [&](auto mask_tag) {
      constexpr bool kMask = decltype(mask_tag)::value;
      float e[CB][4][4];
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        bf16x8_t ka[4];
#pragma unroll
        for (int s = 0; s < 4; ++s)
          ka[s] = *reinterpret_cast<const bf16x8_t*>(ks + (16 * mb + n) * kKPitch + 32 * s + 8 * g);
        float ksv[4][kNgrpB];
        bool kv_ok[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = 16 * mb + 4 * g + i;
          kv_ok[i] = kMask ? s_valid[key] != 0u : true;
#pragma unroll
          for (int gi = 0; gi < kNgrpB; ++gi) ksv[i][gi] = kQB ? ksc_l[key * kNgrp + gi] : 1.0f;
        }
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
          // dot * scale: the staged K scales carry the logit scale.
          f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
          // (one scale per row: the staged scales carry the logit scale)
#pragma unroll
          for (int s = 0; s < 4; ++s) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[s], qb[cb][s], acc, 0, 0, 0);
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[i] = acc[i] * (kQB ? ksv[i][0] : a.scale);
          const uint32_t lg01 = pack_bf16_hw(acc[0], acc[1]);
          const uint32_t lg23 = pack_bf16_hw(acc[2], acc[3]);
          const float lg[4] = {lo_bf16(lg01), hi_bf16(lg01), lo_bf16(lg23), hi_bf16(lg23)};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if constexpr (kMask) {
              const int j = j0 + 16 * mb + 4 * g + i;
              const bool ok = live[cb] && j <= my_pos[cb] && j >= my_lo[cb] && kv_ok[i];
              e[cb][mb][i] = ok ? lg[i] : -INFINITY;
            } else {
              e[cb][mb][i] = lg[i];
            }
          }
        }
      }
      // Online softmax per column block (e holds the logits until here).
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        float mx = m[cb];
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
#pragma unroll
          for (int i = 0; i < 4; ++i) mx = fmaxf(mx, e[cb][mb][i]);
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        // Where no column's maximum moved, the rescale factor is exactly 1:
        // skip the multiply of o and l (a wave-uniform branch).
        if (__any(mx != m[cb])) {
          const float alpha = mx == -INFINITY ? 1.0f : __expf(m[cb] - mx);
          m[cb] = mx;
          l[cb] *= alpha;
#pragma unroll
          for (int nb = 0; nb < 8; ++nb) o[cb][nb] *= alpha;
        }
        // exp(e - mx) as exp2(e log2(e) - mx log2(e)): one FMA feeds the
        // hardware exponential instead of a subtraction and a multiply (the
        // argument's error is the rounding of mx log2(e), of the same order as
        // that of (e - mx) log2(e)); T=8192 K5V4 13.63 -> 13.18 ms.
        const float nml = -mx * kLog2E;
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float p = __builtin_amdgcn_exp2f(fmaf(e[cb][mb][i], kLog2E, nml));
            if constexpr (kMask) e[cb][mb][i] = mx == -INFINITY ? 0.0f : p;
            else e[cb][mb][i] = p;
            l[cb] += e[cb][mb][i];
          }
      }
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        float vsv[8][kNgrpB];
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
          const int key = 16 * (2 * s + (jj >> 2)) + 4 * g + (jj & 3);
#pragma unroll
          for (int gi = 0; gi < kNgrpB; ++gi) vsv[jj][gi] = kQB ? vsc_l[key * kNgrp + gi] : 1.0f;
        }
        bf16x8_t pb[CB][kNgrpB];
#pragma unroll
        for (int cb = 0; cb < CB; ++cb)
#pragma unroll
          for (int gi = 0; gi < kNgrpB; ++gi) {
            float pv[8];
#pragma unroll
            for (int jj = 0; jj < 8; ++jj)
              pv[jj] = kQB ? e[cb][2 * s + (jj >> 2)][jj & 3] * vsv[jj][gi] : e[cb][2 * s + (jj >> 2)][jj & 3];
            pb[cb][gi] = as_bf16x8(pack_bf16_hw(pv[0], pv[1]), pack_bf16_hw(pv[2], pv[3]),
                                   pack_bf16_hw(pv[4], pv[5]), pack_bf16_hw(pv[6], pv[7]));
          }
        const int kk = n >> 2, dd = 4 * (n & 3);
        const uint16_t* r1 = vs + (32 * s + 4 * g + kk) * kVPitch + dd;
        const uint16_t* r2 = r1 + 16 * kVPitch;
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) {
          const u32x2_t lo2 = lds_read_tr(r1 + 16 * nb);
          const u32x2_t hi2 = lds_read_tr(r2 + 16 * nb);
          const bf16x8_t va = as_bf16x8(lo2.x, lo2.y, hi2.x, hi2.y);
          const int gi = kQB ? (16 * nb) / GROUP : 0;
#pragma unroll
          for (int cb = 0; cb < CB; ++cb)
            o[cb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pb[cb][gi], o[cb][nb], 0, 0, 0);
        }
      }
    };
    if (full) tile(std::false_type{});
    else tile(std::true_type{});
    if (j0 + kStep < kv_end) {
      // Stage the group's next tile (its bytes were loaded a tile ago) into
      // its other buffer, whose last readers passed the previous barrier;
      // then load the bytes of the tile after it and the page-table entries
      // of the third.
      prefill_store<BITS, GROUP, PW>(raw, ks2[gk][buf ^ 1], vs2[gk][buf ^ 1], ksc2[gk][buf ^ 1],
                                     vsc2[gk][buf ^ 1], valid2[gk][buf ^ 1], a.scale, tst);
      if (j0 + 2 * kStep < kv_end) {
        prefill_load<BITS, GROUP, PW>(a, kbase, vbase, kscb, vscb, j0 + 2 * kStep, kv_end, ptk,
                                      ptv, raw, tst);
        prefill_pt<BITS, GROUP, PW>(a, j0 + 3 * kStep, kv_end, ptk, ptv, tst);
      }
    }
    __syncthreads();
  }
  if constexpr (KSP == 2) {
    // Group 1's state to group 0 through the tile buffers (free: the loop
    // ended with a barrier): o lane-contiguous per (wave, cb, nb), then m, l.
    f32x4_t* xo = reinterpret_cast<f32x4_t*>(&ks2[0][0][0]) + (wave * CB * 8) * 64 + lane;
    float* xm = reinterpret_cast<float*>(&vs2[0][0][0]) + (wave * CB * 2) * 64 + lane;
    static_assert(sizeof(ks2) >= sizeof(f32x4_t) * 4 * CB * 8 * 64, "merge area (o)");
    static_assert(sizeof(vs2) >= sizeof(float) * 4 * CB * 2 * 64, "merge area (m, l)");
    if (gk == 1) {
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) xo[(cb * 8 + nb) * 64] = o[cb][nb];
        xm[(cb * 2) * 64] = m[cb];
        xm[(cb * 2 + 1) * 64] = l[cb];
      }
    }
    __syncthreads();
    if (gk == 1) return;
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
      const float m1 = xm[(cb * 2) * 64], l1 = xm[(cb * 2 + 1) * 64];
      const float mm = fmaxf(m[cb], m1);
      const float a0 = m[cb] == -INFINITY ? 0.0f : __expf(m[cb] - mm);
      const float a1 = m1 == -INFINITY ? 0.0f : __expf(m1 - mm);
      l[cb] = l[cb] * a0 + l1 * a1;
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) o[cb][nb] = o[cb][nb] * a0 + xo[(cb * 8 + nb) * 64] * a1;
    }
  }
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) {
    float lt = l[cb];
    lt += __shfl_xor(lt, 16);
    lt += __shfl_xor(lt, 32);
    if (!live[cb]) continue;
    const float inv = 1.0f / lt;
    uint16_t* dst = a.out + (static_cast<size_t>(r[cb]) * a.Hq + hq) * kHd + 4 * g;
#pragma unroll
    for (int nb = 0; nb < 8; ++nb)
      *reinterpret_cast<u32x2_t*>(dst + 16 * nb) =
          u32x2_t{pack_bf16_hw(o[cb][nb][0] * inv, o[cb][nb][1] * inv),
                  pack_bf16_hw(o[cb][nb][2] * inv, o[cb][nb][3] * inv)};
  }
}

}  // namespace
}  // namespace g4

namespace g4 {
namespace {

// Tiles per split and split count for sequences up to max_len positions
// (attention_split.cu:61-76, 1154-1157): at most 256 splits.
int attn_tps(int max_len) {
  const int tiles = (max_len + kTile - 1) / kTile;
  return (tiles + kAttnMaxSplits - 1) / kAttnMaxSplits;
}
int attn_splits(int max_len) {
  const int tiles = (max_len + kTile - 1) / kTile;
  const int tps = attn_tps(max_len);
  return (tiles + tps - 1) / tps;
}

// Combine mode (granite4_set_attn_combine_mode): 0 inside the split launch,
// 1 as a second launch.
std::atomic<int> g_attn_combine{0};

// Arrival tags: a process-wide counter from a random start, never 0. The
// slots need only differ from the call's tag before the call: the combining
// block re-zeroes every slot of its group.
std::atomic<unsigned> g_attn_tag{static_cast<unsigned>(std::random_device{}())};
unsigned next_attn_tag() {
  unsigned t;
  do t = g_attn_tag.fetch_add(1, std::memory_order_relaxed) + 1u;
  while (t == 0u);
  return t;
}

// Scratch layout: a 256-byte head holding the sticky error word, then the
// partials (m, l) [rows][Hq][nblk], the partial outputs [rows][Hq][nblk][128]
// and the arrival tags.
constexpr size_t kAttnScratchHead = 256;

void set_scratch(AttnArgs& a, void* scratch, int rows) {
  a.err = static_cast<unsigned*>(scratch);
  a.spin_limit = fp8_sync_spin_limit();
  a.part_ml = reinterpret_cast<float2*>(static_cast<char*>(scratch) + kAttnScratchHead);
  a.part_o = reinterpret_cast<float*>(a.part_ml + static_cast<size_t>(rows) * a.Hq * a.nblk);
}

// Points a at its tag slots (after the partials) and draws the call's tag,
// or leaves tags null for the two-launch form. Returns whether the combine
// is fused.
bool set_combine(AttnArgs& a, int rows) {
  if (g_attn_combine.load(std::memory_order_relaxed) != 0) {
    a.tags = nullptr;
    return false;
  }
  a.tags = reinterpret_cast<unsigned*>(a.part_o + static_cast<size_t>(rows) * a.Hq * a.nblk * kHd);
  a.tag = next_attn_tag();
  return true;
}

template <int BITS, int FUSE>
void launch_attn_bits(const AttnArgs& a, int group, dim3 grid, hipStream_t st) {
  if constexpr (BITS == 16) {
    (void)group;
    hipLaunchKernelGGL((attn_split_kernel<16, kHd, FUSE>), grid, kAttnWaves * 64, 0, st, a);
  } else {
    if (group == kHd) hipLaunchKernelGGL((attn_split_kernel<BITS, kHd, FUSE>), grid, kAttnWaves * 64, 0, st, a);
    else if (group == 64) hipLaunchKernelGGL((attn_split_kernel<BITS, 64, FUSE>), grid, kAttnWaves * 64, 0, st, a);
    else hipLaunchKernelGGL((attn_split_kernel<BITS, 32, FUSE>), grid, kAttnWaves * 64, 0, st, a);
  }
}

// Column blocks per wave: CB = 2 (each wave 8 positions x the 4 query heads,
// 64 positions per 8-wave workgroup) where those workgroups still give every
// CU one, else CB = 1. Two column blocks halve the staging (code -> bf16
// conversion, the VALU-heaviest part) per MFMA; with fewer workgroups the
// occupancy they cost matters more. Measured (8 KV heads, one box, us): int8
// from position 0, CB = 1 / 2: T=1024 46.3 / 50.5 (CB = 2 there runs the
// key-split form), 2048 161.9 / 122.8, 4096 462.5 / 444.1, 8192 1475 / 1274;
// K5V4 group 32 at 57344..: T=2048 4288 / 3482, 4096 8583 / 7102, 8192 18357
// / 14779. (Before the group-32 tiles were staged dequantised: CB = 1 / 2 / 4
// at T=512 int8 33.7 / 45.1 / 69.0 us, at T=8192 K5V4 38.2 / 49.2 / 42.2 ms.)

template <int BITS, int W, int KSP = 1, int CB = 1>
void launch_prefill_w(const PrefillArgs& a, int group, dim3 grid, hipStream_t st) {
  if constexpr (BITS == 16) {
    (void)group;
    hipLaunchKernelGGL((attn_prefill_kernel<16, kHd, CB, W, KSP>), grid, W * 64, 0, st, a);
  } else {
    if (group == kHd) hipLaunchKernelGGL((attn_prefill_kernel<BITS, kHd, CB, W, KSP>), grid, W * 64, 0, st, a);
    else if (group == 64) hipLaunchKernelGGL((attn_prefill_kernel<BITS, 64, CB, W, KSP>), grid, W * 64, 0, st, a);
    else hipLaunchKernelGGL((attn_prefill_kernel<BITS, 32, CB, W, KSP>), grid, W * 64, 0, st, a);
  }
}

// 8-wave workgroups of 64 positions (CB = 2) or 32 (CB = 1) where they give
// every CU one, else 16-position workgroups for twice the workgroups: 8 waves
// splitting the keys between two 4-wave groups.
template <int BITS>
void launch_prefill_bits(const PrefillArgs& a, int group, int Hk, hipStream_t st) {
  const long long blocks64 = static_cast<long long>((a.rows + 63) / 64) * Hk;
  const long long blocks32 = static_cast<long long>((a.rows + 31) / 32) * Hk;
  if (blocks64 >= kCUs) {
    launch_prefill_w<BITS, 8, 1, 2>(a, group, dim3((a.rows + 63) / 64, Hk), st);
  } else if (blocks32 >= kCUs) {
    launch_prefill_w<BITS, 8, 1, 1>(a, group, dim3((a.rows + 31) / 32, Hk), st);
  } else {
    launch_prefill_w<BITS, 8, 2, 1>(a, group, dim3((a.rows + 15) / 16, Hk), st);
  }
}

}  // namespace
}  // namespace g4

using namespace g4;

extern "C" {

int granite4_prefill_attn(const uint16_t* q_rot, int rows, int Hq, int Hk, int d, float scale,
                          const void* cache_k, const void* cache_v, const float* k_scale,
                          const float* v_scale, int bits, int group, int stride, int base_pos,
                          const int* d_pt, int window, uint16_t* out) {
  const bool quant = bits != 16;
  if (q_rot == nullptr || out == nullptr || cache_k == nullptr || cache_v == nullptr ||
      !std::isfinite(scale) || d != kHd || Hk <= 0 || Hq != kGq * Hk || rows <= 0 ||
      base_pos < 0 || stride < base_pos + rows || window < 0 ||
      (bits != 16 && bits != 8 && bits != 4 && bits != 5) ||
      (quant && (k_scale == nullptr || v_scale == nullptr ||
                 (group != 32 && group != 64 && group != kHd)))) {
    std::fprintf(stderr, "granite4: granite4_prefill_attn: invalid arguments\n");
    return -1;
  }
  PrefillArgs a{};
  a.q = q_rot;
  a.k = static_cast<const uint8_t*>(cache_k);
  a.v = static_cast<const uint8_t*>(cache_v);
  a.ksc = k_scale;
  a.vsc = v_scale;
  a.scale = scale;
  a.Hq = Hq;
  a.stride = stride;
  a.rows = rows;
  a.base = base_pos;
  a.window = window;
  a.d_pt = d_pt;
  a.out = out;
  const hipStream_t st = stream();
  switch (bits) {
    case 16: launch_prefill_bits<16>(a, group, Hk, st); break;
    case 8: launch_prefill_bits<8>(a, group, Hk, st); break;
    case 4: launch_prefill_bits<4>(a, group, Hk, st); break;
    default: launch_prefill_bits<5>(a, group, Hk, st); break;
  }
  return launch_status("granite4_prefill_attn");
}

int granite4_prefill_attention(const uint16_t* q_rot, const uint16_t* cache_k,
                               const uint16_t* cache_v, float scale, int Hq, int Hk, int d,
                               int base_pos, int rows, int stride, uint16_t* out,
                               const int8_t* cache_k8, const int8_t* cache_v8,
                               const float* k_scale, const float* v_scale, int int8,
                               const uint8_t* cache_k4, const uint8_t* cache_v4, int int4,
                               const int* d_pt, int k5, int window) {
  if ((int8 && int4) || (k5 && !int4)) {
    std::fprintf(stderr, "granite4: granite4_prefill_attention: invalid arguments\n");
    return -1;
  }
  const int bits = int8 ? 8 : (int4 ? (k5 ? 5 : 4) : 16);
  const void* ck = int8 ? static_cast<const void*>(cache_k8)
                        : (int4 ? static_cast<const void*>(cache_k4) : cache_k);
  const void* cv = int8 ? static_cast<const void*>(cache_v8)
                        : (int4 ? static_cast<const void*>(cache_v4) : cache_v);
  return granite4_prefill_attn(q_rot, rows, Hq, Hk, d, scale, ck, cv, k_scale, v_scale, bits, kHd,
                               stride, base_pos, d_pt, window, out);
}

size_t granite4_attn_split_scratch_bytes(int Hq, int rows, int stride) {
  if (Hq <= 0 || rows <= 0 || stride <= 0) return 0;
  // Enough for every split layout a call over this arena may take (max_len
  // <= stride): the split count is not monotone in the length (256 tiles
  // give 256 splits, 257 give 129), so the bound is min(tiles, 256).
  const int tiles = (stride + kTile - 1) / kTile;
  const size_t nblk = ((tiles < kAttnMaxSplits ? tiles : kAttnMaxSplits) + kAttnWaves - 1) / kAttnWaves;
  const size_t slots = static_cast<size_t>(rows) * Hq * nblk;
  // Partial (m, l) and output per slot, then the arrival tags (one per
  // (row group, KV head, block): at most one per slot).
  return kAttnScratchHead + slots * (sizeof(float2) + kHd * sizeof(float) + sizeof(unsigned));
}

int granite4_attn_sync_status(void* scratch, int clear) {
  if (scratch == nullptr) return -1;
  unsigned v = 0;
  const hipStream_t st = stream();
  bool ok = hipMemcpyAsync(&v, scratch, sizeof v, hipMemcpyDeviceToHost, st) == hipSuccess &&
            hipStreamSynchronize(st) == hipSuccess;
  if (ok && clear && v != 0) {
    static const unsigned zero = 0;
    ok = hipMemcpyAsync(scratch, &zero, sizeof zero, hipMemcpyHostToDevice, st) == hipSuccess &&
         hipStreamSynchronize(st) == hipSuccess;
  }
  if (!ok) {
    std::fprintf(stderr, "granite4: granite4_attn_sync_status: %s\n",
                 hipGetErrorString(hipGetLastError()));
    return -1;
  }
  return v != 0 ? 1 : 0;
}

int granite4_set_attn_combine_mode(int mode) {
  if (mode != 0 && mode != 1) return -1;
  return g_attn_combine.exchange(mode);
}

int granite4_attn_paged(const uint16_t* q, int rows, int Hq, int Hk, int d, float scale,
                        const void* cache_k, const void* cache_v, const float* k_scale,
                        const float* v_scale, int bits, int group, int stride, int kv_base,
                        const int* d_pos, const int* d_pt, const int* row_pos,
                        const int* const* row_pt, int max_len, int window, void* scratch,
                        uint16_t* out) {
  const int ml = max_len > 0 ? max_len : stride;
  const bool quant = bits != 16;
  if (q == nullptr || scratch == nullptr || out == nullptr || cache_k == nullptr ||
      cache_v == nullptr || !std::isfinite(scale) || d != kHd || Hk <= 0 || Hq != kGq * Hk ||
      rows <= 0 || rows > kMaxVerifyRows || stride <= 0 || ml > stride || window < 0 ||
      (d_pos == nullptr && row_pos == nullptr && kv_base + rows > ml) || kv_base < 0 ||
      ((row_pos == nullptr) != (row_pt == nullptr)) ||
      (bits != 16 && bits != 8 && bits != 4 && bits != 5) ||
      (quant && (k_scale == nullptr || v_scale == nullptr ||
                 (group != 32 && group != 64 && group != kHd)))) {
    std::fprintf(stderr, "granite4: granite4_attn_paged: invalid arguments\n");
    return -1;
  }
  AttnArgs a{};
  a.q = q;
  a.k = static_cast<const uint8_t*>(cache_k);
  a.v = static_cast<const uint8_t*>(cache_v);
  a.ksc = k_scale;
  a.vsc = v_scale;
  a.scale = scale;
  a.Hq = Hq;
  a.stride = stride;
  a.rows = rows;
  a.tps = attn_tps(ml);
  a.splits = attn_splits(ml);
  a.window = window;
  a.kv_base = kv_base;
  a.d_pos = d_pos;
  a.d_pt = d_pt;
  a.row_pos = row_pos;
  a.row_pt = row_pt;
  a.nblk = (a.splits + kAttnWaves - 1) / kAttnWaves;
  set_scratch(a, scratch, rows);
  a.out = out;
  // Multi-sequence rows (row_pos) take one wave each; rows of one sequence
  // share a wave in groups of four (their keys are read once per group).
  const int nz = row_pos != nullptr ? rows : (rows + kRowsPerWave - 1) / kRowsPerWave;
  const bool fused = set_combine(a, rows);
  const dim3 grid(Hk, a.nblk, nz);
  const hipStream_t st = stream();
  switch (bits) {
    case 16: launch_attn_bits<16, kAttnPlain>(a, group, grid, st); break;
    case 8: launch_attn_bits<8, kAttnPlain>(a, group, grid, st); break;
    case 4: launch_attn_bits<4, kAttnPlain>(a, group, grid, st); break;
    default: launch_attn_bits<5, kAttnPlain>(a, group, grid, st); break;
  }
  if (launch_status("granite4_attn_paged (split)") != 0) return -1;
  if (fused) return 0;
  hipLaunchKernelGGL(attn_combine_kernel, dim3(Hq / kGq, rows), kCombineThreads, 0, st, a);
  return launch_status("granite4_attn_paged (combine)");
}

}  // extern "C"

namespace {

template <int M>
int attn_decode_append(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                const float* cos_tbl, const float* sin_tbl, int max_pos,
                                const int* d_pos, const int* d_pt, int Hq, int Hk, float scale,
                                void* cache_k, void* cache_v, float* k_scale, float* v_scale,
                                int bits, int group, int stride, void* scratch, uint16_t* out,
                                const char* what) {
  RopeArgs ra;
  // q_rot is never written here (only the K / V units run): q stands in for it.
  if (scratch == nullptr || out == nullptr || !std::isfinite(scale) || Hq != kGq * Hk ||
      !rope_args_at_pos(ra, q, k, v, cos_tbl, sin_tbl, max_pos, d_pos, d_pt, Hq, Hk, kHd, bits,
                        bits == 16 ? kHd : group, const_cast<uint16_t*>(q), cache_k, cache_v,
                        k_scale, v_scale, stride)) {
    std::fprintf(stderr, "granite4: %s: invalid arguments\n", what);
    return -1;
  }
  const int grp = bits == 16 ? kHd : group;
  AttnArgs a{};
  a.q = q;  // kAttnAppend reads the rotated q here
  a.k = static_cast<const uint8_t*>(cache_k);
  a.v = static_cast<const uint8_t*>(cache_v);
  a.ksc = k_scale;
  a.vsc = v_scale;
  a.scale = scale;
  a.Hq = Hq;
  a.stride = stride;
  a.rows = 1;
  a.tps = attn_tps(stride);
  a.splits = attn_splits(stride);
  a.d_pos = d_pos;
  a.d_pt = d_pt;
  a.nblk = (a.splits + kAttnWaves - 1) / kAttnWaves;
  set_scratch(a, scratch, 1);
  a.out = out;
  a.ra = ra;
  const bool fused = set_combine(a, 1);
  const dim3 grid(Hk, a.nblk, 1);
  const hipStream_t st = stream();
  switch (bits) {
    case 16: launch_attn_bits<16, M>(a, grp, grid, st); break;
    case 8: launch_attn_bits<8, M>(a, grp, grid, st); break;
    case 4: launch_attn_bits<4, M>(a, grp, grid, st); break;
    default: launch_attn_bits<5, M>(a, grp, grid, st); break;
  }
  if (launch_status(what) != 0) return -1;
  if (fused) return 0;
  hipLaunchKernelGGL(attn_combine_kernel, dim3(Hq / kGq, 1), kCombineThreads, 0, st, a);
  return launch_status(what);
}

}  // namespace

extern "C" {

int granite4_attn_decode_append(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                const float* cos_tbl, const float* sin_tbl, int max_pos,
                                const int* d_pos, const int* d_pt, int Hq, int Hk, float scale,
                                void* cache_k, void* cache_v, float* k_scale, float* v_scale,
                                int bits, int group, int stride, void* scratch, uint16_t* out) {
  return attn_decode_append<kAttnRopeAppend>(q, k, v, cos_tbl, sin_tbl, max_pos, d_pos, d_pt, Hq,
                                             Hk, scale, cache_k, cache_v, k_scale, v_scale, bits,
                                             group, stride, scratch, out,
                                             "granite4_attn_decode_append");
}

int granite4_attn_decode_append_rotated(const uint16_t* q_rot, const uint16_t* k_rot,
                                        const uint16_t* v, int max_pos, const int* d_pos,
                                        const int* d_pt, int Hq, int Hk, float scale,
                                        void* cache_k, void* cache_v, float* k_scale,
                                        float* v_scale, int bits, int group, int stride,
                                        void* scratch, uint16_t* out) {
  // No table is read in this form: q_rot stands in for the cos / sin
  // pointers in the shared argument checks.
  const float* none = reinterpret_cast<const float*>(q_rot);
  return attn_decode_append<kAttnAppend>(q_rot, k_rot, v, none, none, max_pos, d_pos, d_pt, Hq,
                                         Hk, scale, cache_k, cache_v, k_scale, v_scale, bits,
                                         group, stride, scratch, out,
                                         "granite4_attn_decode_append_rotated");
}


int granite4_attn_split(const uint16_t* q, const uint16_t* cache_k, const uint16_t* cache_v,
                        float scale, int Hq, int Hk, int d, int kv_base, const int* d_pos,
                        int rows, int stride, void* scratch, uint16_t* out,
                        const int8_t* cache_k8, const int8_t* cache_v8,
                        const float* cache_k_scale, const float* cache_v_scale, int int8,
                        const uint8_t* cache_k4, const uint8_t* cache_v4, int int4,
                        const int* d_pt, int max_len, const int* row_pos,
                        const int* const* row_pt, const int* row_grp, int ngroups,
                        const int* row_tbase, const int* row_tail, int kv_hint, int k5,
                        int window) {
  (void)kv_hint;  // a launch-size hint only; every split still exits at once past the rows
  if ((row_grp != nullptr && (row_pos == nullptr || ngroups <= 0 || ngroups > rows)) ||
      (int8 && int4) || (k5 && !int4)) {
    std::fprintf(stderr, "granite4: granite4_attn_split: invalid arguments\n");
    return -1;
  }
  if (row_tbase != nullptr || row_tail != nullptr) {
    std::fprintf(stderr, "granite4: granite4_attn_split: draft-tree rows are not supported\n");
    return -1;
  }
  // row_grp groups rows of one sequence so they share K/V tiles; results are
  // identical without it (attention_gpu.h), so rows run one per wave here.
  const int bits = int8 ? 8 : (int4 ? (k5 ? 5 : 4) : 16);
  const void* ck = int8 ? static_cast<const void*>(cache_k8)
                        : (int4 ? static_cast<const void*>(cache_k4) : cache_k);
  const void* cv = int8 ? static_cast<const void*>(cache_v8)
                        : (int4 ? static_cast<const void*>(cache_v4) : cache_v);
  return granite4_attn_paged(q, rows, Hq, Hk, d, scale, ck, cv, cache_k_scale, cache_v_scale,
                             bits, kHd, stride, kv_base, d_pos, d_pt, row_pos, row_pt, max_len,
                             window, scratch, out);
}

}  // extern "C"
