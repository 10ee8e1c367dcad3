// rope_unit.h - the per-head work of RoPE fused with the quantised KV write
// (one 16-lane DPP row per head row, lane l holding dims [8l, 8l + 8)):
// shared by the append kernels (rope.hip) and the decode q|k|v GEMV that
// appends from its own output (gemv.hip), so both write identical bytes.
#ifndef G4_ROPE_UNIT_H
#define G4_ROPE_UNIT_H

#include "g4_common.h"
#include "g4_hw.h"
#include "g4_math.h"
#include "g4_wave.h"
#include "granite4_layerops.h"

namespace g4 {

struct RopeArgs {
  const uint16_t* q;
  long long q_stride;
  const uint16_t* k;
  long long k_stride;
  const uint16_t* v;
  long long v_stride;
  const float* cos_t;
  const float* sin_t;
  int max_pos;
  int rows, Hq, Hk, d;
  int base_pos;
  const int* pos_rows;    // per-row KV position
  const int* pos_ptr;     // decode: *pos_ptr
  const int* pt;          // position -> arena row
  const int* arena_rows;  // per-row arena row
  const GpuMultiRows* mr;
  int rope_by_row;  // 1: RoPE table row r for row r (verify tables), KV at base_pos + r
  uint16_t* q_rot;
  long long q_rot_stride;
  uint16_t* k_rot;  // optional bf16 rotated K [rows][Hk d]
  void* cache_k;
  void* cache_v;
  float* k_scale;
  float* v_scale;
  int stride;
  int rotate_k;
  int k_round;
  int units_per_row;  // Hq + (kv ? 2 Hk : Hk)
  int has_kv;         // 0: rotate only (K heads go to k_rot)
};

// RoPE table row of row r.
__device__ __forceinline__ int rope_pos(const RopeArgs& a, int r) {
  if (a.mr != nullptr) return a.mr->pos[r];
  if (a.rope_by_row) return r;
  return a.pos_rows != nullptr ? a.pos_rows[r] : (a.pos_ptr != nullptr ? *a.pos_ptr : a.base_pos + r);
}

// Arena row that row r's K / V go to (only K / V units ask, so query heads
// never wait on the page-table load).
__device__ __forceinline__ int arena_row(const RopeArgs& a, int r) {
  if (a.mr != nullptr) {
    const int pos = a.mr->pos[r];
    const int slot = a.mr->tree ? a.mr->slot[r] : pos;
    const int* pt = a.mr->pt[r];
    return pt != nullptr ? pt[slot] : slot;
  }
  if (a.arena_rows != nullptr) return a.arena_rows[r];
  const int pos =
      a.pos_rows != nullptr ? a.pos_rows[r] : (a.pos_ptr != nullptr ? *a.pos_ptr : a.base_pos + r);
  return a.pt != nullptr ? a.pt[pos] : pos;
}

// Rotates the lane's 8 dims; cs / sn are the lane's cos / sin (dims mod 64).
__device__ __forceinline__ void rotate8(const V8& x, const float* cs, const float* sn,
                                        bool first_half, float* out) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t pw = dpp_u32<kDppRor8>(x.w[e]);
    const float a0 = lo_bf16(x.w[e]), a1 = hi_bf16(x.w[e]);
    float b0 = lo_bf16(pw), b1 = hi_bf16(pw);
    if (first_half) {
      b0 = -b0;
      b1 = -b1;
    }
    out[2 * e] = a0 * cs[2 * e] + b0 * sn[2 * e];
    out[2 * e + 1] = a1 * cs[2 * e + 1] + b1 * sn[2 * e + 1];
  }
}

__device__ __forceinline__ V8 to_bf16x8(const float* f) {
  V8 v;
#pragma unroll
  for (int e = 0; e < 4; ++e) v.w[e] = pack_bf16_hw(f[2 * e], f[2 * e + 1]);
  return v;
}

// Where store_quant puts a row: the pool (PoolSink), or a caller's copy of
// the row in the pool's byte layout (RowSink: k / v one row each, ks / vs
// its group scales; the decode attention keeps the row it appends in LDS).
struct PoolSink {
  static constexpr bool kPool = true;
  __device__ __forceinline__ void bytes8(bool, int, uint2) const {}
  __device__ __forceinline__ void bytes4(bool, int, uint32_t) const {}
  __device__ __forceinline__ void bytes1(bool, int, uint8_t) const {}
  __device__ __forceinline__ void scale(bool, int, float) const {}
};
struct RowSink {
  static constexpr bool kPool = false;
  uint8_t* k;
  uint8_t* v;
  float* ks;
  float* vs;
  __device__ __forceinline__ void bytes8(bool is_k, int off, uint2 x) const {
    *reinterpret_cast<uint2*>((is_k ? k : v) + off) = x;
  }
  __device__ __forceinline__ void bytes4(bool is_k, int off, uint32_t x) const {
    *reinterpret_cast<uint32_t*>((is_k ? k : v) + off) = x;
  }
  __device__ __forceinline__ void bytes1(bool is_k, int off, uint8_t x) const { (is_k ? k : v)[off] = x; }
  __device__ __forceinline__ void scale(bool is_k, int gi, float x) const { (is_k ? ks : vs)[gi] = x; }
};

template <int BITS, int GROUP, class Sink = PoolSink>
__device__ __forceinline__ void store_quant(const RopeArgs& a, const float* val, bool is_k,
                                            long long slot, int lane16, const Sink& sink = Sink{}) {
  constexpr int GL = GROUP / 8;
  float am = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) am = fmaxf(am, fabsf(val[e]));
  am = group_max<GL>(am);
  const int qmax = BITS == 8 ? 127 : ((BITS == 5 && is_k) ? 15 : 7);
  const float s = am / static_cast<float>(qmax);
  float* scales = is_k ? a.k_scale : a.v_scale;
  if (lane16 % GL == 0) {
    if constexpr (Sink::kPool) scales[slot * (128 / GROUP) + lane16 / GL] = s;
    else sink.scale(is_k, lane16 / GL, s);
  }
  const float inv = 1.0f / s;
  int c[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) c[e] = kv_code_inv(val[e], s, inv, qmax);
  uint8_t* cache = static_cast<uint8_t*>(is_k ? a.cache_k : a.cache_v);
  if (BITS == 8) {
    uint32_t w0 = 0, w1 = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      w0 |= (static_cast<uint32_t>(c[e]) & 0xffu) << (8 * e);
      w1 |= (static_cast<uint32_t>(c[e + 4]) & 0xffu) << (8 * e);
    }
    if constexpr (Sink::kPool) *reinterpret_cast<uint2*>(cache + slot * 128 + 8 * lane16) = make_uint2(w0, w1);
    else sink.bytes8(is_k, 8 * lane16, make_uint2(w0, w1));
    return;
  }
  uint32_t nib = 0, plane = 0;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint32_t code = static_cast<uint32_t>(c[e] + qmax + 1);
    nib |= (code & 0xfu) << (4 * e);
    plane |= ((code >> 4) & 1u) << e;
  }
  if constexpr (!Sink::kPool) {
    sink.bytes4(is_k, 4 * lane16, nib);
    if (BITS == 5 && is_k) sink.bytes1(true, 64 + lane16, static_cast<uint8_t>(plane));
  } else if (BITS == 5 && is_k) {
    *reinterpret_cast<uint32_t*>(cache + slot * 80 + 4 * lane16) = nib;
    cache[slot * 80 + 64 + lane16] = static_cast<uint8_t>(plane);
  } else {
    *reinterpret_cast<uint32_t*>(cache + slot * 64 + 4 * lane16) = nib;
  }
}

// Whether unit u (Hq query heads, then Hk key heads, then Hk value heads) is
// rotated here: a query head, or a key head when the call rotates K.
__device__ __forceinline__ bool unit_rotated(const RopeArgs& a, int u) {
  return u < a.Hq + a.Hk && (u < a.Hq || a.rotate_k);
}

// The bf16 head row unit u of row r reads.
__device__ __forceinline__ const uint16_t* unit_src(const RopeArgs& a, int r, int u) {
  if (u < a.Hq) return a.q + r * a.q_stride + u * 128LL;
  if (u < a.Hq + a.Hk) return a.k + r * a.k_stride + (u - a.Hq) * 128LL;
  return a.v + r * a.v_stride + (u - a.Hq - a.Hk) * 128LL;
}

// The lane's cos / sin (dims mod 64) of table row rp, clamped into [0,
// max_pos) so that the loads can be issued before rp is checked.
__device__ __forceinline__ void unit_trig(const RopeArgs& a, int rp, int lane16, float* cs,
                                          float* sn) {
  const long long rc = static_cast<long long>(min(max(rp, 0), a.max_pos - 1));
  const float* cp = a.cos_t + rc * 64 + 8 * (lane16 & 7);
  const float* sp = a.sin_t + rc * 64 + 8 * (lane16 & 7);
  *reinterpret_cast<float4*>(cs) = *reinterpret_cast<const float4*>(cp);
  *reinterpret_cast<float4*>(cs + 4) = *reinterpret_cast<const float4*>(cp + 4);
  *reinterpret_cast<float4*>(sn) = *reinterpret_cast<const float4*>(sp);
  *reinterpret_cast<float4*>(sn + 4) = *reinterpret_cast<const float4*>(sp + 4);
}

// The arithmetic and stores of one unit for the calling 16-lane row, given
// its loaded head row x (the lane's 8 dims), the lane's cos / sin of table
// row rp (rotated units) and its arena row (K / V units; arena_row's value).
// A rotated unit outside the table, or a K / V row outside [0, stride),
// writes nothing.
template <int BITS, int GROUP>
__device__ __forceinline__ void unit_finish(const RopeArgs& a, int r, int u, int lane16,
                                            const V8& x, const float* cs, const float* sn,
                                            int rp, int row) {
  const bool first_half = lane16 < 8;
  if (unit_rotated(a, u)) {
    if (rp < 0 || rp >= a.max_pos) return;
    const bool is_q = u < a.Hq;
    const int h = is_q ? u : u - a.Hq;
    float rot[8];
    rotate8(x, cs, sn, first_half, rot);
    const V8 rb = to_bf16x8(rot);
    if (is_q) {
      st8_nt(a.q_rot + r * a.q_rot_stride + h * 128LL + 8 * lane16, rb);
      return;
    }
    if (a.k_rot != nullptr) st8(a.k_rot + (static_cast<long long>(r) * a.Hk + h) * 128 + 8 * lane16, rb);
    if (!a.has_kv) return;
    if (row < 0 || row >= a.stride) return;
    const long long slot = static_cast<long long>(h) * a.stride + row;
    if (BITS == 16) {
      st8(static_cast<uint16_t*>(a.cache_k) + slot * 128 + 8 * lane16, rb);
      return;
    }
    float val[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) val[e] = a.k_round ? v8_get(rb, e) : rot[e];
    store_quant<BITS, GROUP>(a, val, true, slot, lane16);
    return;
  }
  // Unrotated K (already rotated by the caller) or V.
  if (!a.has_kv) return;
  if (row < 0 || row >= a.stride) return;
  const bool is_k = u < a.Hq + a.Hk;
  const int h = is_k ? u - a.Hq : u - a.Hq - a.Hk;
  const long long slot = static_cast<long long>(h) * a.stride + row;
  if (BITS == 16) {
    st8(static_cast<uint16_t*>(is_k ? a.cache_k : a.cache_v) + slot * 128 + 8 * lane16, x);
    return;
  }
  float val[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) val[e] = v8_get(x, e);
  store_quant<BITS, GROUP>(a, val, is_k, slot, lane16);
}

// One unit (row r, head unit u) for the calling 16-lane row. load(head)
// returns the lane's 8 dims of the bf16 head row at global address `head`
// (or wherever the caller keeps them). Only rotated units read the table
// and only K / V units (with a pool) ask for the arena row, so query heads
// never wait on the page-table load.
template <int BITS, int GROUP, class Load>
__device__ __forceinline__ void rope_unit(const RopeArgs& a, int r, int u, int lane16, Load load) {
  const bool rot = unit_rotated(a, u);
  // The head row first: its address needs no position, so its load overlaps
  // the position's (and the page table's) instead of waiting behind them.
  const V8 x = load(unit_src(a, r, u));
  int rp = 0;
  if (rot) {
    rp = rope_pos(a, r);
    if (rp < 0 || rp >= a.max_pos) return;
  }
  float cs[8], sn[8];
  if (rot) unit_trig(a, rp, lane16, cs, sn);
  const int row = (u >= a.Hq && a.has_kv) ? arena_row(a, r) : -1;
  unit_finish<BITS, GROUP>(a, r, u, lane16, x, cs, sn, rp, row);
}

// Fills a for the decode append at *d_pos (granite4_rope_append_at_pos's
// arguments); false when they are invalid.
bool rope_args_at_pos(RopeArgs& a, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                      const float* cos_tbl, const float* sin_tbl, int max_pos, const int* d_pos,
                      const int* d_pt, int Hq, int Hk, int d, int bits, int group, uint16_t* q_rot,
                      void* cache_k, void* cache_v, float* k_scale, float* v_scale, int stride);

}  // namespace g4

#endif  // G4_ROPE_UNIT_H
