// ref_shim.cc - C entry points over the reference's OWN host math, built from
// the reference sources where they lie (see oracle/Makefile, target `ref`).
//
// TEST INFRASTRUCTURE ONLY: used by tests/golden/gen_golden.py to write the
// golden vectors and by the CPU tests to cross-check the oracle, never by the
// product. Each function only composes reference functions; where the
// reference keeps a formula in an anonymous namespace (gpu_pack.cc:44-51) or
// inside a kernel epilogue (forward_gpu.cu:992-994), the one-line formula is
// restated here with its citation.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

#include "kernel_math.h"
#include "kv_pool.h"

using namespace granite4;

extern "C" {

std::uint16_t ref_f32_to_bf16(float f) { return f32_to_bf16_host(f); }

std::uint8_t ref_fp8_encode(double v) { return fp8_e4m3_encode(v, nullptr); }

std::uint16_t ref_fp8_to_bf16(std::uint8_t c) { return fp8_e4m3_to_bf16(c); }

// gpu_pack.cc:44-51: scale = float(amax / 448); code = encode(double(v) / double(scale)).
float ref_fp8_scale_for(double amax) { return static_cast<float>(amax / kFp8E4M3MaxF); }
std::uint8_t ref_fp8_encode_scaled(float v, float scale) {
  return fp8_e4m3_encode(static_cast<double>(v) / static_cast<double>(scale), nullptr);
}

// rmsnorm_f32 on bf16 rows, bf16 output (kernels_phase2.cu:119-125 rounding).
void ref_rmsnorm_bf16(const std::uint16_t* x, const std::uint16_t* w, float eps, int rows,
                      int cols, std::uint16_t* out) {
  std::vector<float> xf(cols), wf(cols), of(cols);
  for (int i = 0; i < cols; ++i) wf[i] = bf16_to_f32_host(w[i]);
  for (int r = 0; r < rows; ++r) {
    for (int i = 0; i < cols; ++i) xf[i] = bf16_to_f32_host(x[(std::size_t)r * cols + i]);
    rmsnorm_f32(xf.data(), wf.data(), eps, cols, of.data());
    for (int i = 0; i < cols; ++i) out[(std::size_t)r * cols + i] = f32_to_bf16_host(of[i]);
  }
}

// Residual epilogue bf16(res + mult * y) (forward_gpu.cu:992-994,
// kernel_math.h:527-528), y = bf16 branch.
std::uint16_t ref_residual_add(std::uint16_t res, std::uint16_t branch, float mult) {
  return f32_to_bf16_host(bf16_to_f32_host(res) + mult * bf16_to_f32_host(branch));
}

void ref_rope_tables(double theta, int head_dim, int max_pos, float* c, float* s) {
  std::vector<float> vc, vs;
  rope_freqs_f32(theta, head_dim, max_pos, &vc, &vs);
  std::memcpy(c, vc.data(), vc.size() * sizeof(float));
  std::memcpy(s, vs.data(), vs.size() * sizeof(float));
}

// rope_half_f32 on one bf16 head, f32 output (the caller rounds as needed).
void ref_rope_half(const std::uint16_t* x, const float* c, const float* s, int d, float* out) {
  std::vector<float> xf(d);
  for (int i = 0; i < d; ++i) xf[i] = bf16_to_f32_host(x[i]);
  rope_half_f32(xf.data(), c, s, d, out);
}

float ref_silu(float x) { return silu_f32(x); }

float ref_kv8_scale(float a) { return kv8_scale_host(a); }
int ref_kv8_quant(float x, float s) { return kv8_quant_host(x, s); }
float ref_q4_scale(float a) { return q4_scale_host(a); }
int ref_q4_quant(float x, float s) { return q4_quant_host(x, s); }
float ref_k5_scale(float a) { return k5_scale_host(a); }
int ref_k5_quant(float x, float s) { return k5_quant_host(x, s); }
void ref_k5_pack_row(const unsigned char* codes, unsigned char* out) {
  k5_pack_row_host(codes, out);
}

std::uint64_t ref_rng_fill_u64(std::uint64_t seed, int n, std::uint64_t* out) {
  Xorshift64 r(seed);
  for (int i = 0; i < n; ++i) out[i] = r.next();
  return r.s;
}
void ref_rng_fill_range(std::uint64_t seed, double a, int n, float* out) {
  Xorshift64 r(seed);
  for (int i = 0; i < n; ++i) out[i] = r.next_float_range(a);
}

// A PagedKV pool with interleaved sequences, so block tables are not the
// identity. Writes, for `seqs` sequences of `tokens` positions each, the page
// id of every page (blocks[seq][page]) and the row table (rows[seq][pos]).
int ref_paged_row_tables(int seqs, int tokens, int* blocks, int* rows) {
  const std::size_t B = 16;
  ModelConfig mc = kModelConfig;
  const KvLayout l = KvLayout::from_config(mc);
  const std::size_t pages_needed = (std::size_t)seqs * ((tokens + B - 1) / B) + 8;
  KvPoolConfig cfg = KvPoolConfig::from_budget(mc, B, pages_needed * B * l.bytes_per_token);
  PagedKV pool(cfg);
  std::vector<int> ids(seqs);
  for (int s = 0; s < seqs; ++s) ids[s] = pool.create_sequence();
  // Grow the sequences one page at a time, round-robin, so pages interleave.
  const int npages = (tokens + (int)B - 1) / (int)B;
  for (int p = 1; p <= npages; ++p)
    for (int s = 0; s < seqs; ++s) {
      const std::size_t want = std::min<std::size_t>((std::size_t)p * B, (std::size_t)tokens);
      PagedKV::Tokens toks(want, (std::uint32_t)(1000 * s + 7));
      for (std::size_t t = 0; t < want; ++t) toks[t] = (std::uint32_t)(1000 * s + t);
      if (!pool.reserve(ids[s], want, toks)) return -1;
    }
  for (int s = 0; s < seqs; ++s) {
    const std::vector<std::size_t>& bt = pool.block_table(ids[s]);
    if ((int)bt.size() != npages) return -2;
    for (int pg = 0; pg < npages; ++pg) blocks[s * npages + pg] = (int)bt[pg];
    if (!pool.row_table(ids[s], (std::size_t)tokens, rows + (std::size_t)s * tokens)) return -3;
  }
  return npages;
}

// kernel_math.h:312-331: the reference's host GQA decode attention on a
// contiguous bf16 cache k, v [Hk][kv_len][d]; out [Hq][d].
void ref_gqa_attention_bf16(const std::uint16_t* q, const std::uint16_t* k, const std::uint16_t* v,
                            float scale, int Hq, int Hk, int d, int kv_len, std::uint16_t* out) {
  std::vector<std::uint16_t> o;
  gqa_attention_bf16(q, k, v, scale, Hq, Hk, d, kv_len, &o);
  std::memcpy(out, o.data(), o.size() * sizeof(std::uint16_t));
}

}  // extern "C"
