// rope.hip - RoPE on Q/K fused with the quantised write into the paged KV
// arena, and the embedding gather, for gfx950.
//
// RoPE (Llama half split, kernel_math.h:208-219): for i < 64,
//   out[i]      = a * c - b * s        a = x[i], b = x[i + 64]
//   out[i + 64] = b * c + a * s        c, s = cos / sin table row of the position
// in f32 with two roundings per product term (built with -ffp-contract=off),
// then bf16 RNE: bit-identical to the reference's kernels.
//
// One head row (d = 128) is one 16-lane DPP row: lane l holds dims
// [8l, 8l + 8) as one 16-byte vector, and the rotation partner of lane l is
// lane l ^ 8, fetched with one row_ror:8 DPP move per packed pair. A 256-thread
// workgroup handles 16 head rows; the units of a token are its Hq query heads,
// then Hk key heads, then Hk value heads.
//
// KV quantisation per group of `GROUP` dims (GROUP / 8 lanes): amax by DPP
// max, s = amax / qmax (IEEE division), code = clamp(round_half_away(x / s))
// (device_math.cuh:105-210). Stores per lane: int8 8 B, int4 4 B, K5 4 nibble
// bytes + 1 plane byte (bit j of plane byte l is bit 4 of dim 8l + j), scales
// by the group's first lane.
#include "g4_common.h"
#include "g4_hw.h"
#include "g4_math.h"
#include "g4_wave.h"
#include "granite4_layerops.h"
#include "rope_unit.h"

#include <atomic>
#include <cstdlib>
#include <map>
#include <mutex>

namespace g4 {


// Table-size registry for tables this library allocated, so the reference's
// entry points (which carry no table length) still get a position bound.
// Lookups run on every launch of those entry points: they scan a fixed array
// of atomic (table, length) slots without a lock. Registration and removal
// (once per table) take the mutex; a table registered beyond the slots goes
// to an overflow map that lookups consult only while it is non-empty.
namespace {
constexpr int kTabSlots = 64;
std::atomic<const float*> g_tab_key[kTabSlots];
std::atomic<int> g_tab_len[kTabSlots];
std::atomic<int> g_tab_used{0};      // slots [0, used) may hold tables
std::atomic<int> g_tab_overflow{0};  // entries in g_tab_more
std::mutex g_tab_mu;
std::map<const float*, int> g_tab_more;
}  // namespace

int table_bound(const float* t) {
  const int used = g_tab_used.load(std::memory_order_acquire);
  for (int i = 0; i < used; ++i)
    if (g_tab_key[i].load(std::memory_order_acquire) == t)
      return g_tab_len[i].load(std::memory_order_relaxed);
  if (g_tab_overflow.load(std::memory_order_acquire) == 0) return INT_MAX;
  std::lock_guard<std::mutex> lk(g_tab_mu);
  const auto it = g_tab_more.find(t);
  return it == g_tab_more.end() ? INT_MAX : it->second;
}
void table_register(const float* t, int max_pos) {
  std::lock_guard<std::mutex> lk(g_tab_mu);
  int free_slot = -1;
  const int used = g_tab_used.load(std::memory_order_relaxed);
  for (int i = 0; i < used; ++i) {
    const float* k = g_tab_key[i].load(std::memory_order_relaxed);
    if (k == t) {
      g_tab_len[i].store(max_pos, std::memory_order_relaxed);
      return;
    }
    if (k == nullptr && free_slot < 0) free_slot = i;
  }
  if (free_slot < 0 && used < kTabSlots) free_slot = used;
  if (free_slot < 0) {
    g_tab_more[t] = max_pos;
    g_tab_overflow.store(static_cast<int>(g_tab_more.size()), std::memory_order_release);
    return;
  }
  // The length before the key: a lookup that sees the key sees its length.
  g_tab_len[free_slot].store(max_pos, std::memory_order_relaxed);
  g_tab_key[free_slot].store(t, std::memory_order_release);
  if (free_slot == used) g_tab_used.store(used + 1, std::memory_order_release);
}
void table_forget(const float* t) {
  std::lock_guard<std::mutex> lk(g_tab_mu);
  const int used = g_tab_used.load(std::memory_order_relaxed);
  for (int i = 0; i < used; ++i)
    if (g_tab_key[i].load(std::memory_order_relaxed) == t)
      g_tab_key[i].store(nullptr, std::memory_order_release);
  if (g_tab_more.erase(t) != 0)
    g_tab_overflow.store(static_cast<int>(g_tab_more.size()), std::memory_order_release);
}

namespace {

template <int BITS, int GROUP>
__global__ __launch_bounds__(kBlock) void rope_append_kernel(RopeArgs a) {
  // The kernel arguments the first loads need, fetched in one scalar round
  // trip (otherwise each is a dependent scalar-cache miss where first used).
  asm volatile("" ::"s"(a.q), "s"(a.k), "s"(a.v), "s"(a.q_stride), "s"(a.k_stride),
               "s"(a.v_stride), "s"(a.pos_ptr), "s"(a.pos_rows), "s"(a.pt), "s"(a.arena_rows),
               "s"(a.mr), "s"(a.rows), "s"(a.units_per_row), "s"(a.Hq), "s"(a.Hk));
  const int lane16 = threadIdx.x & 15;
  // rows * units_per_row < 2^31 (checked on the host), so 32-bit indexing.
  const unsigned unit = blockIdx.x * (kBlock / 16) + (threadIdx.x >> 4);
  if (unit >= static_cast<unsigned>(a.rows) * static_cast<unsigned>(a.units_per_row)) return;  // whole DPP rows
  const int r = static_cast<int>(unit / static_cast<unsigned>(a.units_per_row));
  const int u = static_cast<int>(unit - static_cast<unsigned>(r) * static_cast<unsigned>(a.units_per_row));
  rope_unit<BITS, GROUP>(a, r, u, lane16, [&](const uint16_t* head) { return ld8_nt(head + 8 * lane16); });
}

// One workgroup per token row (units_per_row <= 16 UPL): lane group g owns
// units g, g + 16, ... of the row. The row's position and arena row are
// loaded once, then every head row of the group (UPL 16-byte loads per lane
// in flight together), then the row's cos / sin; the arithmetic is
// unit_finish's, so the bytes written equal rope_append_kernel's. One unit
// per lane group kept one 16-byte load per lane in flight and a dependent
// page-table / table round trip per unit; measured at T=8192 (K5V4 group
// 32): 40.3 us there, 32.9 us here.
template <int BITS, int GROUP, int UPL>
__global__ __launch_bounds__(kBlock) void rope_append_row_kernel(RopeArgs a) {
  asm volatile("" ::"s"(a.q), "s"(a.k), "s"(a.v), "s"(a.q_stride), "s"(a.k_stride),
               "s"(a.v_stride), "s"(a.pos_ptr), "s"(a.pos_rows), "s"(a.pt), "s"(a.arena_rows),
               "s"(a.mr), "s"(a.units_per_row), "s"(a.Hq), "s"(a.Hk), "s"(a.cos_t), "s"(a.sin_t));
  const int lane16 = threadIdx.x & 15, grp = threadIdx.x >> 4;
  const int r = blockIdx.x;
  const int nu = a.units_per_row;
  const int rp = rope_pos(a, r);
  const int row = a.has_kv ? arena_row(a, r) : -1;
  V8 x[UPL];
#pragma unroll
  for (int j = 0; j < UPL; ++j) {
    const int u = min(grp + 16 * j, nu - 1);
    x[j] = ld8_nt(unit_src(a, r, u) + 8 * lane16);
  }
  float cs[8], sn[8];
  unit_trig(a, rp, lane16, cs, sn);
#pragma unroll
  for (int j = 0; j < UPL; ++j) {
    const int u = grp + 16 * j;
    if (u < nu) unit_finish<BITS, GROUP>(a, r, u, lane16, x[j], cs, sn, rp, row);
  }
}

// Any head dim (even, <= 1024; quantised forms one scale per row): one
// workgroup per unit, values staged in LDS.
template <int BITS>
__global__ __launch_bounds__(kBlock) void rope_append_generic_kernel(RopeArgs a) {
  const long long unit = blockIdx.x;
  const int r = static_cast<int>(unit / a.units_per_row);
  const int u = static_cast<int>(unit - static_cast<long long>(r) * a.units_per_row);
  const int d = a.d, half = d / 2;
  __shared__ float s_val[1024];
  __shared__ float s_scale;
  const bool rotated = u < a.Hq + a.Hk && (u < a.Hq || a.rotate_k);
  const bool is_q = u < a.Hq;
  const bool is_k = !is_q && u < a.Hq + a.Hk;
  const int h = is_q ? u : (is_k ? u - a.Hq : u - a.Hq - a.Hk);
  const int rp = rotated ? rope_pos(a, r) : 0;
  if (rotated && (rp < 0 || rp >= a.max_pos)) return;
  const int row = (a.has_kv && !is_q) ? arena_row(a, r) : -1;
  const bool kv_ok = row >= 0 && row < a.stride;
  const uint16_t* src = is_q ? a.q + r * a.q_stride : (is_k ? a.k + r * a.k_stride : a.v + r * a.v_stride);
  src += static_cast<long long>(h) * d;
  const long long slot = static_cast<long long>(h) * a.stride + row;
  for (int i = threadIdx.x; i < d; i += kBlock) {
    uint32_t bits;
    float val;
    if (rotated) {
      const int j = i < half ? i : i - half;
      const float c = a.cos_t[static_cast<long long>(rp) * half + j];
      const float s = a.sin_t[static_cast<long long>(rp) * half + j];
      const float x0 = bf16_to_f32(src[i]);
      const float x1 = bf16_to_f32(src[i < half ? i + half : i - half]);
      const float rv = i < half ? x0 * c - x1 * s : x0 * c + x1 * s;
      bits = f32_to_bf16(rv);
      val = a.k_round ? bf16_to_f32(bits) : rv;
    } else {
      bits = src[i];
      val = bf16_to_f32(bits);
    }
    if (is_q) {
      a.q_rot[r * a.q_rot_stride + static_cast<long long>(h) * d + i] = static_cast<uint16_t>(bits);
      continue;
    }
    if (is_k && rotated && a.k_rot != nullptr)
      a.k_rot[(static_cast<long long>(r) * a.Hk + h) * d + i] = static_cast<uint16_t>(bits);
    if (BITS == 16 && kv_ok)
      static_cast<uint16_t*>(is_k ? a.cache_k : a.cache_v)[slot * d + i] = static_cast<uint16_t>(bits);
    s_val[i] = val;
  }
  if (BITS == 16 || is_q || !kv_ok) return;  // uniform per workgroup
  __syncthreads();
  const int qmax = BITS == 8 ? 127 : 7;
  if (threadIdx.x == 0) {
    float am = 0.0f;
    for (int i = 0; i < d; ++i) am = fmaxf(am, fabsf(s_val[i]));
    s_scale = am / static_cast<float>(qmax);
    (is_k ? a.k_scale : a.v_scale)[slot] = s_scale;
  }
  __syncthreads();
  const float s = s_scale;
  uint8_t* cache = static_cast<uint8_t*>(is_k ? a.cache_k : a.cache_v);
  if (BITS == 8) {
    for (int i = threadIdx.x; i < d; i += kBlock)
      cache[slot * d + i] = static_cast<uint8_t>(kv_code(s_val[i], s, 127));
  } else {
    for (int w = threadIdx.x; w < half; w += kBlock)
      cache[slot * half + w] = static_cast<uint8_t>((kv_code(s_val[2 * w], s, 7) + 8) |
                                                    ((kv_code(s_val[2 * w + 1], s, 7) + 8) << 4));
  }
}

template <int BITS, int GROUP>
void launch_row_kernel(const RopeArgs& a, int upl) {
  const hipStream_t st = stream();
  const dim3 grid(static_cast<unsigned>(a.rows));
  switch (upl) {
    case 1: hipLaunchKernelGGL((rope_append_row_kernel<BITS, GROUP, 1>), grid, kBlock, 0, st, a); break;
    case 2: hipLaunchKernelGGL((rope_append_row_kernel<BITS, GROUP, 2>), grid, kBlock, 0, st, a); break;
    case 3: hipLaunchKernelGGL((rope_append_row_kernel<BITS, GROUP, 3>), grid, kBlock, 0, st, a); break;
    default: hipLaunchKernelGGL((rope_append_row_kernel<BITS, GROUP, 4>), grid, kBlock, 0, st, a); break;
  }
}

template <int BITS>
void launch_row_bits(const RopeArgs& a, int group, int upl) {
  if (BITS == 16 || group == 128) launch_row_kernel<BITS, 128>(a, upl);
  else if (group == 64) launch_row_kernel<BITS, 64>(a, upl);
  else launch_row_kernel<BITS, 32>(a, upl);
}

template <int BITS>
void launch_fast_bits(const RopeArgs& a, int group, unsigned grid) {
  const hipStream_t st = stream();
  if (group == 32) hipLaunchKernelGGL((rope_append_kernel<BITS, 32>), grid, kBlock, 0, st, a);
  else if (group == 64) hipLaunchKernelGGL((rope_append_kernel<BITS, 64>), grid, kBlock, 0, st, a);
  else hipLaunchKernelGGL((rope_append_kernel<BITS, 128>), grid, kBlock, 0, st, a);
}

}  // namespace

// Per-token workgroups (rope_append_row_kernel) or one unit per lane group
// (rope_append_kernel); both write the same bytes.

// Measured (int8, A/B on one box, per-unit kernel / row kernel, us): 512 rows
// 5.06 / 5.38, 640 5.62 / 5.98, 768 7.09 / 6.18, 1024 8.20 / 7.25, 4096
// 23.4 / 18.6.
constexpr int kRopeRowKernelMinRows = 704;

// Validated launch of the fused kernel (d == 128) or the generic one.
int launch_rope_append(RopeArgs a, int bits, int group, const char* what) {
  a.units_per_row = a.Hq + (a.has_kv ? 2 * a.Hk : (a.rotate_k ? a.Hk : 0));
  const long long units = static_cast<long long>(a.rows) * a.units_per_row;
  if (units <= 0) return 0;
  if (a.d == 128 && (bits == 16 || group == 32 || group == 64 || group == 128)) {
    if (units > INT_MAX) {
      std::fprintf(stderr, "granite4: %s: %lld (row, head) units exceed 2^31 - 1\n", what, units);
      return -1;
    }
    const long long blocks = (units + (kBlock / 16) - 1) / (kBlock / 16);
    const unsigned grid = static_cast<unsigned>(blocks);
    const int upl = (a.units_per_row + 15) / 16;
    // Per-token workgroups for long inputs; fewer rows (decode, T = 8, up to
    // about 700 rows) keep one unit per lane group, which spreads them over
    // more workgroups (T=8: 24 instead of 8, 2.7 vs 3.3 us).
    if (upl <= 4 && a.rows >= kRopeRowKernelMinRows) {
      switch (bits) {
        case 16: launch_row_bits<16>(a, 128, upl); break;
        case 8: launch_row_bits<8>(a, group, upl); break;
        case 4: launch_row_bits<4>(a, group, upl); break;
        case 5: launch_row_bits<5>(a, group, upl); break;
        default: return -1;
      }
      return launch_status(what);
    }
    switch (bits) {
      case 16: launch_fast_bits<16>(a, 128, grid); break;
      case 8: launch_fast_bits<8>(a, group, grid); break;
      case 4: launch_fast_bits<4>(a, group, grid); break;
      case 5: launch_fast_bits<5>(a, group, grid); break;
      default: return -1;
    }
  } else {
    if (bits == 5 || a.d > 1024 || (bits != 16 && group != a.d) || units > INT_MAX) {
      std::fprintf(stderr, "granite4: %s: unsupported shape (d %d, bits %d, group %d)\n", what,
                   a.d, bits, group);
      return -1;
    }
    const unsigned grid = static_cast<unsigned>(units);
    const hipStream_t st = stream();
    if (bits == 16) hipLaunchKernelGGL((rope_append_generic_kernel<16>), grid, kBlock, 0, st, a);
    else if (bits == 8) hipLaunchKernelGGL((rope_append_generic_kernel<8>), grid, kBlock, 0, st, a);
    else if (bits == 4) hipLaunchKernelGGL((rope_append_generic_kernel<4>), grid, kBlock, 0, st, a);
    else return -1;
  }
  return launch_status(what);
}

RopeArgs rope_args_zero() {
  RopeArgs a{};
  a.max_pos = INT_MAX;
  return a;
}

// ---------------------------------------------------------------------------
// Embedding gather.
// ---------------------------------------------------------------------------
namespace {

template <bool VEC>
__global__ __launch_bounds__(kBlock) void embed_kernel(const int32_t* tokens, int start,
                                                       const int* d_pos, const uint16_t* emb,
                                                       int vocab, int H, float mult,
                                                       uint16_t* out) {
  asm volatile("" ::"s"(tokens), "s"(start), "s"(d_pos), "s"(emb), "s"(vocab), "s"(H), "s"(mult),
               "s"(out));
  const int r = blockIdx.y;
  const int tok = d_pos != nullptr ? tokens[*d_pos] : tokens[start + r];
  const bool valid = vocab < 0 || (tok >= 0 && tok < vocab);
  const long long src = static_cast<long long>(tok) * H;
  const long long dst = static_cast<long long>(r) * H;
  if (VEC) {
    const int j = 8 * (blockIdx.x * kBlock + threadIdx.x);
    if (j >= H) return;
    V8 v{{0u, 0u, 0u, 0u}};
    if (valid) {
      v = ld8_nt(emb + src + j);
#pragma unroll
      for (int e = 0; e < 4; ++e) v.w[e] = pack_bf16_hw(mult * lo_bf16(v.w[e]), mult * hi_bf16(v.w[e]));
    }
    st8_nt(out + dst + j, v);
  } else {
    const int j = blockIdx.x * kBlock + threadIdx.x;
    if (j >= H) return;
    out[dst + j] = valid ? static_cast<uint16_t>(f32_to_bf16(mult * bf16_to_f32(emb[src + j]))) : 0;
  }
}

// Whole rows, RPW tokens per workgroup, for H = NV * 8 * kBlock (NV = 2:
// H = 4096, the width the host dispatch checks): the token ids
// first, then every vector of the workgroup's rows in flight (NV per row per
// thread), then the stores; the arithmetic is embed_kernel's.
template <int NV, int RPW>
__global__ __launch_bounds__(kBlock) void embed_rows_kernel(const int32_t* tokens, int start,
                                                            int rows, const uint16_t* emb,
                                                            int vocab, float mult, uint16_t* out) {
  asm volatile("" ::"s"(tokens), "s"(start), "s"(rows), "s"(emb), "s"(vocab), "s"(mult), "s"(out));
  constexpr int H = NV * 8 * kBlock;
  const int r0 = blockIdx.x * RPW;
  int tok[RPW];
#pragma unroll
  for (int i = 0; i < RPW; ++i) tok[i] = tokens[start + min(r0 + i, rows - 1)];
  V8 v[RPW][NV];
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const bool valid = vocab < 0 || (tok[i] >= 0 && tok[i] < vocab);
    const long long src = static_cast<long long>(valid ? tok[i] : 0) * H;
#pragma unroll
    for (int k = 0; k < NV; ++k) v[i][k] = ld8_nt(emb + src + 8 * (threadIdx.x + k * kBlock));
  }
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    if (r0 + i >= rows) break;
    const bool valid = vocab < 0 || (tok[i] >= 0 && tok[i] < vocab);
    const long long dst = static_cast<long long>(r0 + i) * H;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      V8 w{{0u, 0u, 0u, 0u}};
      if (valid) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          w.w[e] = pack_bf16_hw(mult * lo_bf16(v[i][k].w[e]), mult * hi_bf16(v[i][k].w[e]));
      }
      st8_nt(out + dst + 8 * (threadIdx.x + k * kBlock), w);
    }
  }
}

int launch_embed(const int32_t* tokens, int start, const int* d_pos, int rows,
                 const uint16_t* emb, int vocab, int H, float mult, uint16_t* out,
                 const char* what) {
  if (tokens == nullptr || emb == nullptr || out == nullptr || rows <= 0 || rows > 65535 ||
      H <= 0 || !std::isfinite(mult) || start < 0) {
    std::fprintf(stderr, "granite4: %s: invalid arguments\n", what);
    return -1;
  }
  const hipStream_t st = stream();
  // H = 4096: whole rows per workgroup, two below 4096 rows (measured at
  // T=512: 3.09 vs 3.31 us for the vector-per-lane grid), one from 4096 rows
  // (T=8192, A/B over two rounds on one box: one row 23.72, two 24.48, four
  // 24.18-24.26, the vector-per-lane grid 24.12-24.13 us).
  if (d_pos == nullptr && H == 4096) {
    if (rows < 4096)
      hipLaunchKernelGGL((embed_rows_kernel<2, 2>), dim3((rows + 1) / 2), kBlock, 0, st, tokens,
                         start, rows, emb, vocab, mult, out);
    else
      hipLaunchKernelGGL((embed_rows_kernel<2, 1>), dim3(rows), kBlock, 0, st, tokens, start,
                         rows, emb, vocab, mult, out);
    return launch_status(what);
  }
  if (H % 8 == 0) {
    const dim3 grid((H / 8 + kBlock - 1) / kBlock, rows);
    hipLaunchKernelGGL((embed_kernel<true>), grid, kBlock, 0, st, tokens, start, d_pos, emb,
                       vocab, H, mult, out);
  } else {
    const dim3 grid((H + kBlock - 1) / kBlock, rows);
    hipLaunchKernelGGL((embed_kernel<false>), grid, kBlock, 0, st, tokens, start, d_pos, emb,
                       vocab, H, mult, out);
  }
  return launch_status(what);
}

}  // namespace
bool rope_args_at_pos(RopeArgs& a, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                      const float* cos_tbl, const float* sin_tbl, int max_pos, const int* d_pos,
                      const int* d_pt, int Hq, int Hk, int d, int bits, int group, uint16_t* q_rot,
                      void* cache_k, void* cache_v, float* k_scale, float* v_scale, int stride) {
  if (d_pos == nullptr || q == nullptr || Hq <= 0 || d != 128 || k == nullptr || v == nullptr ||
      cos_tbl == nullptr || sin_tbl == nullptr || max_pos <= 0 || q_rot == nullptr ||
      cache_k == nullptr || cache_v == nullptr || Hk <= 0 || stride <= 0 ||
      (bits != 16 && bits != 8 && bits != 4 && bits != 5) ||
      (bits != 16 && (group != 32 && group != 64 && group != 128)) ||
      (bits != 16 && (k_scale == nullptr || v_scale == nullptr)))
    return false;
  a = rope_args_zero();
  a.q = q;
  a.q_stride = static_cast<long long>(Hq) * d;
  a.k = k;
  a.k_stride = static_cast<long long>(Hk) * d;
  a.v = v;
  a.v_stride = a.k_stride;
  a.cos_t = cos_tbl;
  a.sin_t = sin_tbl;
  a.max_pos = max_pos;
  a.rows = 1;
  a.Hq = Hq;
  a.Hk = Hk;
  a.d = d;
  a.pos_ptr = d_pos;
  a.pt = d_pt;
  a.q_rot = q_rot;
  a.q_rot_stride = a.q_stride;
  a.cache_k = cache_k;
  a.cache_v = cache_v;
  a.k_scale = k_scale;
  a.v_scale = v_scale;
  a.stride = stride;
  a.rotate_k = 1;
  a.k_round = 1;
  a.has_kv = 1;
  a.units_per_row = Hq + 2 * Hk;
  return true;
}

}  // namespace g4

using namespace g4;

extern "C" {

int granite4_prefill_embed_rows(const int32_t* d_tokens, int start, int rows,
                                const uint16_t* emb, float mult, uint16_t* out, int H) {
  return launch_embed(d_tokens, start, nullptr, rows, emb, -1, H, mult, out,
                      "granite4_prefill_embed_rows");
}

int granite4_embed_rows(const int32_t* d_tokens, int rows, const uint16_t* emb, int vocab,
                        int H, float mult, uint16_t* out) {
  if (vocab <= 0) return -1;
  return launch_embed(d_tokens, 0, nullptr, rows, emb, vocab, H, mult, out,
                      "granite4_embed_rows");
}

int granite4_embed_at_pos(const int32_t* d_tokens, const int* d_pos, const uint16_t* emb,
                          int vocab, int H, float mult, uint16_t* out) {
  if (d_pos == nullptr || vocab <= 0) return -1;
  return launch_embed(d_tokens, 0, d_pos, 1, emb, vocab, H, mult, out, "granite4_embed_at_pos");
}

// --- RoPE only ---------------------------------------------------------------

int granite4_kernel_rope(const uint16_t* d_x, const float* d_cos, const float* d_sin, int rows,
                         int head_dim, uint16_t* d_out) {
  if (d_x == nullptr || d_cos == nullptr || d_sin == nullptr || d_out == nullptr || rows <= 0 ||
      head_dim <= 0 || (head_dim & 1) || head_dim > kMaxHeadDim ||
      !fits_int(static_cast<long long>(rows) * head_dim))
    return -1;
  RopeArgs a = rope_args_zero();
  a.q = d_x;
  a.q_stride = head_dim;
  a.q_rot = d_out;
  a.q_rot_stride = head_dim;
  a.cos_t = d_cos;
  a.sin_t = d_sin;
  a.max_pos = table_bound(d_cos);
  a.rows = rows;
  a.Hq = 1;
  a.d = head_dim;
  return launch_rope_append(a, 16, head_dim, "granite4_kernel_rope");
}

int granite4_kernel_rope_at_pos(const uint16_t* d_x, const float* d_cos_row,
                                const float* d_sin_row, int heads, int d, uint16_t* d_out) {
  if (d_x == nullptr || d_cos_row == nullptr || d_sin_row == nullptr || d_out == nullptr ||
      heads <= 0 || d <= 0 || (d & 1) || d > kMaxHeadDim ||
      !fits_int(static_cast<long long>(heads) * d))
    return -1;
  RopeArgs a = rope_args_zero();
  a.q = d_x;
  a.q_stride = static_cast<long long>(heads) * d;
  a.q_rot = d_out;
  a.q_rot_stride = a.q_stride;
  a.cos_t = d_cos_row;
  a.sin_t = d_sin_row;
  a.max_pos = 1;
  a.rows = 1;
  a.Hq = heads;
  a.d = d;
  return launch_rope_append(a, 16, d, "granite4_kernel_rope_at_pos");
}

int granite4_kernel_rope_at_pos_batched(const uint16_t* d_x, const float* d_cos,
                                        const float* d_sin, int rows, int heads, int d,
                                        uint16_t* d_out) {
  if (d_x == nullptr || d_cos == nullptr || d_sin == nullptr || d_out == nullptr || rows <= 0 ||
      rows > kMaxVerifyRows || heads <= 0 || d <= 0 || (d & 1) || d > kMaxHeadDim ||
      !fits_int(static_cast<long long>(rows) * heads * d))
    return -1;
  RopeArgs a = rope_args_zero();
  a.q = d_x;
  a.q_stride = static_cast<long long>(heads) * d;
  a.q_rot = d_out;
  a.q_rot_stride = a.q_stride;
  a.cos_t = d_cos;
  a.sin_t = d_sin;
  a.max_pos = rows;
  a.rows = rows;
  a.Hq = heads;
  a.d = d;
  a.rope_by_row = 1;
  return launch_rope_append(a, 16, d, "granite4_kernel_rope_at_pos_batched");
}

// --- standalone batched KV appends (kernels_phase2.cu:1087-1181) ---------------

static int kv_append_batched(const uint16_t* k, const uint16_t* v, void* ck, void* cv, float* ks,
                             float* vs, int base_pos, int rows, int stride, int Hk, int d,
                             const int* d_pt, int bits, const char* what) {
  const bool quant = bits != 16;
  if (k == nullptr || v == nullptr || ck == nullptr || cv == nullptr ||
      (quant && (ks == nullptr || vs == nullptr)) || base_pos < 0 || rows <= 0 ||
      rows > kMaxVerifyRows || Hk <= 0 || d <= 0 || d > 1024 || base_pos > INT_MAX - rows ||
      stride < base_pos + rows || stride > INT_MAX / Hk ||
      (bits == 4 && (d & 1)) || (bits == 5 && d != 128))
    return -1;
  RopeArgs a = rope_args_zero();
  a.k = k;
  a.k_stride = static_cast<long long>(Hk) * d;
  a.v = v;
  a.v_stride = a.k_stride;
  a.rows = rows;
  a.Hk = Hk;
  a.d = d;
  a.base_pos = base_pos;
  a.pt = d_pt;
  a.cache_k = ck;
  a.cache_v = cv;
  a.k_scale = ks;
  a.v_scale = vs;
  a.stride = stride;
  a.has_kv = 1;
  return launch_rope_append(a, bits, d, what);
}

int granite4_kernel_kv_append_batched(const uint16_t* d_src_k, const uint16_t* d_src_v,
                                      uint16_t* d_cache_k, uint16_t* d_cache_v, int base_pos,
                                      int rows, int stride, int Hk, int d, const int* d_pt) {
  return kv_append_batched(d_src_k, d_src_v, d_cache_k, d_cache_v, nullptr, nullptr, base_pos,
                           rows, stride, Hk, d, d_pt, 16, "granite4_kernel_kv_append_batched");
}

int granite4_kernel_kv_append_int8_batched(const uint16_t* d_src_k, const uint16_t* d_src_v,
                                           int8_t* d_cache_k, int8_t* d_cache_v,
                                           float* d_cache_k_scale, float* d_cache_v_scale,
                                           int base_pos, int rows, int stride, int Hk, int d,
                                           const int* d_pt) {
  return kv_append_batched(d_src_k, d_src_v, d_cache_k, d_cache_v, d_cache_k_scale,
                           d_cache_v_scale, base_pos, rows, stride, Hk, d, d_pt, 8,
                           "granite4_kernel_kv_append_int8_batched");
}

int granite4_kernel_kv_append_int4_batched(const uint16_t* d_src_k, const uint16_t* d_src_v,
                                           uint8_t* d_cache_k, uint8_t* d_cache_v,
                                           float* d_cache_k_scale, float* d_cache_v_scale,
                                           int base_pos, int rows, int stride, int Hk, int d,
                                           const int* d_pt) {
  return kv_append_batched(d_src_k, d_src_v, d_cache_k, d_cache_v, d_cache_k_scale,
                           d_cache_v_scale, base_pos, rows, stride, Hk, d, d_pt, 4,
                           "granite4_kernel_kv_append_int4_batched");
}

int granite4_kernel_kv_append_k5v4_batched(const uint16_t* d_src_k, const uint16_t* d_src_v,
                                           uint8_t* d_cache_k, uint8_t* d_cache_v,
                                           float* d_cache_k_scale, float* d_cache_v_scale,
                                           int base_pos, int rows, int stride, int Hk, int d,
                                           const int* d_pt) {
  return kv_append_batched(d_src_k, d_src_v, d_cache_k, d_cache_v, d_cache_k_scale,
                           d_cache_v_scale, base_pos, rows, stride, Hk, d, d_pt, 5,
                           "granite4_kernel_kv_append_k5v4_batched");
}

int granite4_kernel_verify_qkv_stage(const uint16_t* d_q, const uint16_t* d_k,
                                     const uint16_t* d_v, const float* d_cos,
                                     const float* d_sin, int base_pos, int rows, int Hq, int Hk,
                                     int d, int cache_stride, uint16_t* d_q_rot,
                                     uint16_t* d_k_rot, uint16_t* d_cache_k,
                                     uint16_t* d_cache_v, const int* d_pt) {
  if (d_q == nullptr || d_k == nullptr || d_v == nullptr || d_cos == nullptr ||
      d_sin == nullptr || d_q_rot == nullptr || d_k_rot == nullptr || d_cache_k == nullptr ||
      d_cache_v == nullptr || base_pos < 0 || rows <= 0 || rows > kMaxVerifyRows || Hq <= 0 ||
      Hk <= 0 || Hq < Hk || Hq % Hk != 0 || d <= 0 || (d & 1) || d > kMaxHeadDim ||
      base_pos > INT_MAX - rows + 1 || cache_stride <= base_pos + rows - 1)
    return -1;
  RopeArgs a = rope_args_zero();
  a.q = d_q;
  a.q_stride = static_cast<long long>(Hq) * d;
  a.k = d_k;
  a.k_stride = static_cast<long long>(Hk) * d;
  a.v = d_v;
  a.v_stride = a.k_stride;
  a.cos_t = d_cos;
  a.sin_t = d_sin;
  a.max_pos = rows;
  a.rope_by_row = 1;
  a.rows = rows;
  a.Hq = Hq;
  a.Hk = Hk;
  a.d = d;
  a.base_pos = base_pos;
  a.pt = d_pt;
  a.q_rot = d_q_rot;
  a.q_rot_stride = a.q_stride;
  a.k_rot = d_k_rot;
  a.cache_k = d_cache_k;
  a.cache_v = d_cache_v;
  a.stride = cache_stride;
  a.rotate_k = 1;
  a.k_round = 1;
  a.has_kv = 1;
  return launch_rope_append(a, 16, d, "granite4_kernel_verify_qkv_stage");
}

// --- prefill split + append (prefill_gemm.cu:1311-1391) -------------------------

static int prefill_split(const uint16_t* qkv, const float* c, const float* s, int base_pos,
                         int rows, int Hq, int Hk, int d, int stride, uint16_t* q_rot, void* ck,
                         void* cv, float* ks, float* vs, const int* d_pt, int bits,
                         const char* what) {
  if (qkv == nullptr || c == nullptr || s == nullptr || q_rot == nullptr || ck == nullptr ||
      cv == nullptr || rows <= 0 || rows > 65535 || Hq <= 0 || Hk <= 0 || d <= 0 || (d & 1) ||
      base_pos < 0 || base_pos > INT_MAX - rows || stride < base_pos + rows ||
      (bits != 16 && (d != 128 || ks == nullptr || vs == nullptr))) {
    std::fprintf(stderr, "granite4: %s: invalid arguments\n", what);
    return -1;
  }
  const long long row = static_cast<long long>(Hq + 2 * Hk) * d;
  RopeArgs a = rope_args_zero();
  a.q = qkv;
  a.q_stride = row;
  a.k = qkv + static_cast<long long>(Hq) * d;
  a.k_stride = row;
  a.v = qkv + static_cast<long long>(Hq + Hk) * d;
  a.v_stride = row;
  a.cos_t = c;
  a.sin_t = s;
  a.max_pos = table_bound(c);
  a.rows = rows;
  a.Hq = Hq;
  a.Hk = Hk;
  a.d = d;
  a.base_pos = base_pos;
  a.pt = d_pt;
  a.q_rot = q_rot;
  a.q_rot_stride = static_cast<long long>(Hq) * d;
  a.cache_k = ck;
  a.cache_v = cv;
  a.k_scale = ks;
  a.v_scale = vs;
  a.stride = stride;
  a.rotate_k = 1;
  a.k_round = 0;
  a.has_kv = 1;
  return launch_rope_append(a, bits, d, what);
}

int granite4_prefill_rope_split_append(const uint16_t* qkv, const float* cos_tbl,
                                       const float* sin_tbl, int base_pos, int rows, int Hq,
                                       int Hk, int d, int stride, uint16_t* q_rot,
                                       uint16_t* cache_k, uint16_t* cache_v, const int* d_pt) {
  return prefill_split(qkv, cos_tbl, sin_tbl, base_pos, rows, Hq, Hk, d, stride, q_rot, cache_k,
                       cache_v, nullptr, nullptr, d_pt, 16, "granite4_prefill_rope_split_append");
}

int granite4_prefill_rope_split_append_int8(const uint16_t* qkv, const float* cos_tbl,
                                            const float* sin_tbl, int base_pos, int rows,
                                            int Hq, int Hk, int d, int stride, uint16_t* q_rot,
                                            int8_t* cache_k, int8_t* cache_v,
                                            float* cache_k_scale, float* cache_v_scale,
                                            const int* d_pt) {
  return prefill_split(qkv, cos_tbl, sin_tbl, base_pos, rows, Hq, Hk, d, stride, q_rot, cache_k,
                       cache_v, cache_k_scale, cache_v_scale, d_pt, 8,
                       "granite4_prefill_rope_split_append_int8");
}

int granite4_prefill_rope_split_append_int4(const uint16_t* qkv, const float* cos_tbl,
                                            const float* sin_tbl, int base_pos, int rows,
                                            int Hq, int Hk, int d, int stride, uint16_t* q_rot,
                                            uint8_t* cache_k, uint8_t* cache_v,
                                            float* cache_k_scale, float* cache_v_scale,
                                            const int* d_pt) {
  return prefill_split(qkv, cos_tbl, sin_tbl, base_pos, rows, Hq, Hk, d, stride, q_rot, cache_k,
                       cache_v, cache_k_scale, cache_v_scale, d_pt, 4,
                       "granite4_prefill_rope_split_append_int4");
}

int granite4_prefill_rope_split_append_k5v4(const uint16_t* qkv, const float* cos_tbl,
                                            const float* sin_tbl, int base_pos, int rows,
                                            int Hq, int Hk, int d, int stride, uint16_t* q_rot,
                                            uint8_t* cache_k, uint8_t* cache_v,
                                            float* cache_k_scale, float* cache_v_scale,
                                            const int* d_pt) {
  return prefill_split(qkv, cos_tbl, sin_tbl, base_pos, rows, Hq, Hk, d, stride, q_rot, cache_k,
                       cache_v, cache_k_scale, cache_v_scale, d_pt, 5,
                       "granite4_prefill_rope_split_append_k5v4");
}

// --- multi-session (forward_gpu.cu:3891-3937) -----------------------------------

}  // extern "C"

namespace g4 {
namespace {
// embed_multi_v8_kernel (forward_gpu.cu:370-378): row r is the token of
// session row r at its position (tok[r][slot], slot = tree ? slot[r] :
// pos[r]), times the embedding multiplier; a token outside [0, vocab)
// gives a zero row, as granite4_embed_rows.
__global__ __launch_bounds__(kBlock) void multi_embed_kernel(const GpuMultiRows* mr,
                                                             const uint16_t* emb, int vocab,
                                                             int H, float mult, uint16_t* out) {
  const int r = blockIdx.y;
  const int j = 8 * (blockIdx.x * kBlock + threadIdx.x);
  if (j >= H) return;
  const int slot = mr->tree ? mr->slot[r] : mr->pos[r];
  const int32_t* tp = mr->tok[r];
  const int tok = tp != nullptr && slot >= 0 ? tp[slot] : -1;
  const bool valid = tok >= 0 && tok < vocab;
  V8 v{{0u, 0u, 0u, 0u}};
  if (valid) {
    v = ld8_nt(emb + static_cast<long long>(tok) * H + j);
#pragma unroll
    for (int e = 0; e < 4; ++e) v.w[e] = pack_bf16_hw(mult * lo_bf16(v.w[e]), mult * hi_bf16(v.w[e]));
  }
  st8_nt(out + static_cast<long long>(r) * H + j, v);
}
}  // namespace
}  // namespace g4

extern "C" {

int granite4_multi_embed(const GpuMultiRows* d_rows, int rows, const uint16_t* emb, int vocab,
                         int H, float mult, uint16_t* out) {
  if (d_rows == nullptr || emb == nullptr || out == nullptr || rows < 1 ||
      rows > kMaxVerifyRows || vocab <= 0 || H <= 0 || H % 8 != 0 || !std::isfinite(mult)) {
    std::fprintf(stderr, "granite4: granite4_multi_embed: invalid arguments\n");
    return -1;
  }
  hipLaunchKernelGGL(multi_embed_kernel, dim3((H / 8 + kBlock - 1) / kBlock, rows), kBlock, 0,
                     stream(), d_rows, emb, vocab, H, mult, out);
  return launch_status("granite4_multi_embed");
}

int granite4_multi_rope(const uint16_t* x, const float* cos_tbl, const float* sin_tbl,
                        const GpuMultiRows* d_rows, int rows, int heads, int d, uint16_t* out) {
  if (x == nullptr || cos_tbl == nullptr || sin_tbl == nullptr || out == nullptr ||
      d_rows == nullptr || rows < 1 || rows > kMaxVerifyRows || heads <= 0 || d <= 0 || (d & 1) ||
      d > kMaxHeadDim)
    return -1;
  RopeArgs a = rope_args_zero();
  a.q = x;
  a.q_stride = static_cast<long long>(heads) * d;
  a.q_rot = out;
  a.q_rot_stride = a.q_stride;
  a.cos_t = cos_tbl;
  a.sin_t = sin_tbl;
  a.max_pos = table_bound(cos_tbl);
  a.mr = d_rows;
  a.rows = rows;
  a.Hq = heads;
  a.d = d;
  return launch_rope_append(a, 16, d, "granite4_multi_rope");
}

int granite4_multi_rope_append(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                               const float* cos_tbl, const float* sin_tbl,
                               const GpuMultiRows* d_rows, int rows, int Hq, int Hk, int d,
                               int bits, void* cache_k, void* cache_v, float* k_scale,
                               float* v_scale, int stride, uint16_t* q_rot) {
  if (q == nullptr || k == nullptr || v == nullptr || cos_tbl == nullptr || sin_tbl == nullptr ||
      d_rows == nullptr || rows < 1 || rows > kMaxVerifyRows || Hq <= 0 || Hk <= 0 ||
      d > 256 || (d & 63) != 0 || q_rot == nullptr || cache_k == nullptr || cache_v == nullptr ||
      (bits != 16 && bits != 8 && bits != 4 && bits != 5) ||
      (bits != 16 && (k_scale == nullptr || v_scale == nullptr)) || (bits == 5 && d != 128))
    return -1;
  RopeArgs a = rope_args_zero();
  a.q = q;
  a.q_stride = static_cast<long long>(Hq) * d;
  a.k = k;
  a.k_stride = static_cast<long long>(Hk) * d;
  a.v = v;
  a.v_stride = a.k_stride;
  a.cos_t = cos_tbl;
  a.sin_t = sin_tbl;
  a.max_pos = table_bound(cos_tbl);
  a.mr = d_rows;
  a.rows = rows;
  a.Hq = Hq;
  a.Hk = Hk;
  a.d = d;
  a.q_rot = q_rot;
  a.q_rot_stride = a.q_stride;
  a.cache_k = cache_k;
  a.cache_v = cache_v;
  a.k_scale = k_scale;
  a.v_scale = v_scale;
  a.stride = stride;
  a.rotate_k = 1;
  a.k_round = 1;
  a.has_kv = 1;
  return launch_rope_append(a, bits, d, "granite4_multi_rope_append");
}

int granite4_multi_kv_append(const uint16_t* k, const uint16_t* v, int bits, void* cache_k,
                             void* cache_v, float* k_scale, float* v_scale,
                             const GpuMultiRows* d_rows, int rows, int stride, int Hk, int d) {
  if (k == nullptr || v == nullptr || cache_k == nullptr || cache_v == nullptr ||
      d_rows == nullptr || rows < 1 || rows > kMaxVerifyRows || Hk <= 0 || d <= 0 || d > 1024 ||
      (bits != 16 && bits != 8 && bits != 4 && bits != 5) ||
      (bits != 16 && (k_scale == nullptr || v_scale == nullptr)) || (bits == 5 && d != 128) ||
      (bits == 4 && (d & 1)))
    return -1;
  RopeArgs a = rope_args_zero();
  a.k = k;
  a.k_stride = static_cast<long long>(Hk) * d;
  a.v = v;
  a.v_stride = a.k_stride;
  a.mr = d_rows;
  a.rows = rows;
  a.Hk = Hk;
  a.d = d;
  a.cache_k = cache_k;
  a.cache_v = cache_v;
  a.k_scale = k_scale;
  a.v_scale = v_scale;
  a.stride = stride;
  a.has_kv = 1;
  return launch_rope_append(a, bits, d, "granite4_multi_kv_append");
}

// --- generalised fused entry points -----------------------------------------------

int granite4_rope_append(const uint16_t* q, long q_stride, const uint16_t* k, long k_stride,
                         const uint16_t* v, long v_stride, const float* cos_tbl,
                         const float* sin_tbl, int max_pos, int rows, int Hq, int Hk, int d,
                         int base_pos, const int* d_pos_rows, const int* d_pt,
                         const int* d_arena_rows, int bits, int group, int k_round_bf16,
                         int rotate_k, uint16_t* q_rot, long q_rot_stride, void* cache_k,
                         void* cache_v, float* k_scale, float* v_scale, int stride) {
  const bool rot_needed = (q != nullptr && Hq > 0) || rotate_k;
  if (d != 128 || rows <= 0 || Hq < 0 || Hk <= 0 || k == nullptr || v == nullptr ||
      cache_k == nullptr || cache_v == nullptr || stride <= 0 ||
      (q == nullptr) != (Hq == 0) || (Hq > 0 && q_rot == nullptr) ||
      (rot_needed && (cos_tbl == nullptr || sin_tbl == nullptr || max_pos <= 0)) ||
      (bits != 16 && bits != 8 && bits != 4 && bits != 5) ||
      (bits != 16 && (group != 32 && group != 64 && group != 128)) ||
      (bits != 16 && (k_scale == nullptr || v_scale == nullptr)) ||
      (d_pos_rows == nullptr && (base_pos < 0 || base_pos > INT_MAX - rows)) ||
      q_stride < (Hq > 0 ? static_cast<long>(Hq) * d : 0) || k_stride < static_cast<long>(Hk) * d ||
      v_stride < static_cast<long>(Hk) * d) {
    std::fprintf(stderr, "granite4: granite4_rope_append: invalid arguments\n");
    return -1;
  }
  RopeArgs a = rope_args_zero();
  a.q = q;
  a.q_stride = q_stride;
  a.k = k;
  a.k_stride = k_stride;
  a.v = v;
  a.v_stride = v_stride;
  a.cos_t = cos_tbl;
  a.sin_t = sin_tbl;
  a.max_pos = max_pos;
  a.rows = rows;
  a.Hq = Hq;
  a.Hk = Hk;
  a.d = d;
  a.base_pos = base_pos;
  a.pos_rows = d_pos_rows;
  a.pt = d_pt;
  a.arena_rows = d_arena_rows;
  a.q_rot = q_rot;
  a.q_rot_stride = q_rot_stride;
  a.cache_k = cache_k;
  a.cache_v = cache_v;
  a.k_scale = k_scale;
  a.v_scale = v_scale;
  a.stride = stride;
  a.rotate_k = rotate_k ? 1 : 0;
  a.k_round = k_round_bf16 ? 1 : 0;
  a.has_kv = 1;
  return launch_rope_append(a, bits, bits == 16 ? 128 : group, "granite4_rope_append");
}

int granite4_rope_append_at_pos(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                const float* cos_tbl, const float* sin_tbl, int max_pos,
                                const int* d_pos, const int* d_pt, int Hq, int Hk, int d,
                                int bits, int group, uint16_t* q_rot, void* cache_k,
                                void* cache_v, float* k_scale, float* v_scale, int stride) {
  RopeArgs a;
  if (!rope_args_at_pos(a, q, k, v, cos_tbl, sin_tbl, max_pos, d_pos, d_pt, Hq, Hk, d, bits, group,
                        q_rot, cache_k, cache_v, k_scale, v_scale, stride)) {
    std::fprintf(stderr, "granite4: granite4_rope_append_at_pos: invalid arguments\n");
    return -1;
  }
  return launch_rope_append(a, bits, bits == 16 ? 128 : group, "granite4_rope_append_at_pos");
}

}  // extern "C"
