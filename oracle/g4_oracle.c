/*
 * g4_oracle.c - CPU restatement of the reference engine's non-GEMM layer math.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP library and the timed CPU
 * baseline of bench.py. Nothing in the product path links or loads it.
 *
 * Written as plain scalar C (compiled -O2 -ffp-contract=off so that a*b - c*d
 * is two roundings, as in the reference's host math). Each function names the
 * reference lines it follows; DESIGN notes on where the build deliberately
 * extends the reference (FP8 activation outputs, group-32 KV scales) are in
 * the header comments below.
 */
#include "g4_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* bf16 (kernel_math.h:39-55)                                                */
/* ------------------------------------------------------------------------ */

float g4o_bf16_to_f32(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, sizeof f);
  return f;
}

/* Round-to-nearest-even on the low 16 bits: add 0x7fff plus the lowest kept
 * bit, then truncate (the reference's exact formula, NaN patterns included). */
uint16_t g4o_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, sizeof u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

/* ------------------------------------------------------------------------ */
/* xorshift64* (kernel_math.h:637-658)                                       */
/* ------------------------------------------------------------------------ */

static uint64_t rng_seed(uint64_t seed) { return seed ? seed : 0x9e3779b97f4a7c15ull; }

uint64_t g4o_rng_next(uint64_t* s) {
  uint64_t x = *s;
  x ^= x << 13;
  x ^= x >> 7;
  x ^= x << 17;
  *s = x;
  return x * 0x2545F4914F6CDD1Dull;
}

/* Top 23 bits of the output as a float in [0, 1). */
float g4o_rng_float(uint64_t* s) {
  const uint32_t u = (uint32_t)(g4o_rng_next(s) >> 41);
  return (float)u * 0x1p-23f;
}

static float rng_range(uint64_t* s, double a) {
  const float u = g4o_rng_float(s);
  return (u * 2.0f - 1.0f) * (float)a;
}

/* gen_bf16 of test_kernels.cu:240-242 with a general half-width a. */
void g4o_fill_uniform_bf16(uint64_t seed, double a, size_t n, uint16_t* out) {
  uint64_t s = rng_seed(seed);
  for (size_t i = 0; i < n; ++i) out[i] = g4o_f32_to_bf16(rng_range(&s, a));
}

void g4o_fill_uniform_f32(uint64_t seed, double a, size_t n, float* out) {
  uint64_t s = rng_seed(seed);
  for (size_t i = 0; i < n; ++i) out[i] = rng_range(&s, a);
}

/* Box-Muller over two uniforms: the normal draws of the benchmark configs. */
void g4o_fill_normal_bf16(uint64_t seed, double mean, double stddev, size_t n, uint16_t* out) {
  uint64_t s = rng_seed(seed);
  const double two_pi = 6.283185307179586476925;
  for (size_t i = 0; i < n; ++i) {
    const double u1 = 1.0 - (double)g4o_rng_float(&s); /* (0, 1] */
    const double u2 = (double)g4o_rng_float(&s);
    const double z = sqrt(-2.0 * log(u1)) * cos(two_pi * u2);
    out[i] = g4o_f32_to_bf16((float)(mean + stddev * z));
  }
}

void g4o_fill_u32(uint64_t seed, size_t n, uint32_t* out) {
  uint64_t s = rng_seed(seed);
  for (size_t i = 0; i < n; ++i) out[i] = (uint32_t)(g4o_rng_next(&s) >> 32);
}

/* ------------------------------------------------------------------------ */
/* FP8 e4m3                                                                  */
/* ------------------------------------------------------------------------ */

/*
 * Correctly rounded (ties-to-even) e4m3 encode of a double, with the
 * reference's conventions (fp8_convert.cc:47-122): NaN -> 0x7F; the sign is
 * kept for zero and for values that round to zero; |v| >= 464 (and inf)
 * saturates to +-448 (0x7E); the 0x7F slot is never produced for finite input.
 *
 * Restated from the format definition rather than the reference's integer
 * significand arithmetic: below 2^-6 the grid is k * 2^-9 (k = 0..8, and
 * k = 8 is the first normal 0x08); in [2^e, 2^(e+1)) it is k * 2^(e-3),
 * k = 8..16. Scaling by a power of two is exact, so nearbyint() (the default
 * ties-to-even mode) performs the only rounding.
 */
uint8_t g4o_fp8_encode(double v) {
  if (v != v) return 0x7Fu;
  const uint8_t sign = signbit(v) ? 0x80u : 0x00u;
  const double a = fabs(v);
  if (a == 0.0) return sign;
  if (a >= 464.0) return (uint8_t)(sign | 0x7Eu);
  int ex = 0;
  (void)frexp(a, &ex); /* a in [2^(ex-1), 2^ex) */
  const int e2 = ex - 1;
  if (e2 < -6) {
    const double k = nearbyint(ldexp(a, 9)); /* 0..8 */
    return (uint8_t)(sign | (uint8_t)k);
  }
  double k = nearbyint(ldexp(a, 3 - e2)); /* 8..16 */
  int e = e2;
  if (k >= 16.0) {
    k = 8.0;
    e += 1;
  }
  const int E = e + 7;
  const int m = (int)k - 8;
  if (E > 15 || (E == 15 && m == 7)) return (uint8_t)(sign | 0x7Eu);
  return (uint8_t)(sign | (uint8_t)(E << 3) | (uint8_t)m);
}

/* Exact decode (fp8_convert.cc:128-157); 0x7F / 0xFF decode to NaN. */
double g4o_fp8_decode(uint8_t c) {
  const double sgn = (c & 0x80u) ? -1.0 : 1.0;
  const int E = (c >> 3) & 0xF;
  const int m = c & 0x7;
  if (E == 15 && m == 7) return NAN;
  if (E == 0) return sgn * ldexp((double)m, -9);
  return sgn * ldexp(8.0 + m, E - 10);
}

/* scale = float(amax / 448) (gpu_pack.cc:44-46). */
float g4o_fp8_scale_for(double amax) { return (float)(amax / 448.0); }

/* code = encode(double(x) / double(scale)) (gpu_pack.cc:48-51). */
void g4o_fp8_encode_scaled_bf16(const uint16_t* x, size_t n, float scale, uint8_t* codes) {
  for (size_t i = 0; i < n; ++i)
    codes[i] = g4o_fp8_encode((double)g4o_bf16_to_f32(x[i]) / (double)scale);
}

/*
 * Per-tensor quantisation of a bf16 tensor, the reference's pack_fp8
 * (gpu_pack.cc:296-308 with parallel_max_abs :89-103): amax skips NaN
 * (`a > mx`), scale <= 0 gives all-zero codes and scale 0.
 */
float g4o_fp8_quantize_bf16(const uint16_t* x, size_t n, uint8_t* codes) {
  double mx = 0.0;
  for (size_t i = 0; i < n; ++i) {
    const double a = fabs((double)g4o_bf16_to_f32(x[i]));
    if (a > mx) mx = a;
  }
  const float scale = g4o_fp8_scale_for(mx);
  if (scale <= 0.0f) {
    memset(codes, 0, n);
    return 0.0f;
  }
  g4o_fp8_encode_scaled_bf16(x, n, scale, codes);
  return scale;
}

/* ------------------------------------------------------------------------ */
/* Embedding gather: out = bf16(mult * emb[tok]) (kernel_math.h:450-453,      */
/* prefill_gemm.cu:280-290 rounding).                                        */
/* ------------------------------------------------------------------------ */

void g4o_embed_rows(const int32_t* tokens, int rows, const uint16_t* emb, int H, float mult,
                    uint16_t* out) {
  for (int r = 0; r < rows; ++r) {
    const uint16_t* src = emb + (size_t)tokens[r] * (size_t)H;
    uint16_t* dst = out + (size_t)r * (size_t)H;
    for (int j = 0; j < H; ++j) dst[j] = g4o_f32_to_bf16(mult * g4o_bf16_to_f32(src[j]));
  }
}

/* ------------------------------------------------------------------------ */
/* RMSNorm (kernel_math.h:178-184): double sum of squares, r = 1/sqrt(float   */
/* mean + eps), y = x*r*w in float, bf16 output (kernels_phase2.cu:119-125). */
/* ------------------------------------------------------------------------ */

static void rmsnorm_row(const float* x, const uint16_t* w, float eps, int cols, uint16_t* out) {
  double s = 0.0;
  for (int i = 0; i < cols; ++i) s += (double)x[i] * (double)x[i];
  const float r = 1.0f / sqrtf((float)(s / cols) + eps);
  for (int i = 0; i < cols; ++i) out[i] = g4o_f32_to_bf16(x[i] * r * g4o_bf16_to_f32(w[i]));
}

void g4o_rmsnorm(const uint16_t* x, const uint16_t* w, float eps, int rows, int cols,
                 uint16_t* out) {
  float buf[16384];
  for (int r = 0; r < rows; ++r) {
    const uint16_t* xr = x + (size_t)r * (size_t)cols;
    for (int i = 0; i < cols; ++i) buf[i] = g4o_bf16_to_f32(xr[i]);
    rmsnorm_row(buf, w, eps, cols, out + (size_t)r * (size_t)cols);
  }
}

/*
 * Residual add then RMSNorm of the rounded residual: res' = bf16(res + mult *
 * branch) (the O / down epilogue, forward_gpu.cu:992-994 and kernel_math.h:
 * 527-528; the branch arrives as bf16 here), normed = rmsnorm(res').
 * Either output pointer may be NULL.
 */
void g4o_add_rmsnorm(const uint16_t* res, const uint16_t* branch, float mult, const uint16_t* w,
                     float eps, int rows, int cols, uint16_t* res_out, uint16_t* normed) {
  float buf[16384];
  for (int r = 0; r < rows; ++r) {
    const size_t o = (size_t)r * (size_t)cols;
    for (int i = 0; i < cols; ++i) {
      const float sum = g4o_bf16_to_f32(res[o + i]) + mult * g4o_bf16_to_f32(branch[o + i]);
      const uint16_t b = g4o_f32_to_bf16(sum);
      if (res_out) res_out[o + i] = b;
      buf[i] = g4o_bf16_to_f32(b);
    }
    if (normed) rmsnorm_row(buf, w, eps, cols, normed + o);
  }
}

/* ------------------------------------------------------------------------ */
/* SwiGLU: act = bf16(g * (1 / (1 + exp(-g))) * u) (prefill_gemm.cu:1194-1203;*/
/* the decode epilogue kernels_phase2.cu:643-651 has the same shape).         */
/* ------------------------------------------------------------------------ */

static uint16_t swiglu_one(float g, float u) {
  const float sig = 1.0f / (1.0f + expf(-g));
  return g4o_f32_to_bf16(g * sig * u);
}

void g4o_swiglu_bf16(const uint16_t* gu, int rows, int I, uint16_t* act) {
  for (int r = 0; r < rows; ++r) {
    const uint16_t* row = gu + (size_t)r * 2u * (size_t)I;
    for (int i = 0; i < I; ++i)
      act[(size_t)r * I + i] = swiglu_one(g4o_bf16_to_f32(row[i]), g4o_bf16_to_f32(row[I + i]));
  }
}

void g4o_silu_mul_f32(const float* gu, int I, int rows, uint16_t* act) {
  for (int r = 0; r < rows; ++r) {
    const float* row = gu + (size_t)r * 2u * (size_t)I;
    for (int i = 0; i < I; ++i) act[(size_t)r * I + i] = swiglu_one(row[i], row[I + i]);
  }
}

/* ------------------------------------------------------------------------ */
/* FP8 x FP8 GEMM (exact products, double accumulation; test_kernels.cu:     */
/* 1685-1719 pins the reference's GEMM against this form).                  */
/* ------------------------------------------------------------------------ */

void g4o_gemm_fp8(const uint8_t* A, int lda, float a_scale, const uint8_t* W, int M, int N, int K,
                  float scale0, float scale1, float scale2, int seg1, int seg2, float* y) {
  double dec[256];
  for (int c = 0; c < 256; ++c) dec[c] = g4o_fp8_decode((uint8_t)c);
  for (int m = 0; m < M; ++m) {
    const uint8_t* a = A + (size_t)m * (size_t)lda;
    for (int n = 0; n < N; ++n) {
      const uint8_t* w = W + (size_t)n * (size_t)K;
      double acc = 0.0;
      for (int k = 0; k < K; ++k) acc += dec[a[k]] * dec[w[k]];
      const float ws = n < seg1 ? scale0 : (n < seg2 ? scale1 : scale2);
      const float s = a_scale * ws;
      y[(size_t)m * (size_t)N + n] = (float)((double)s * acc);
    }
  }
}

void g4o_gemm_bf16w(const uint16_t* A, int lda, const uint8_t* W, int M, int N, int K,
                    float scale0, float scale1, float scale2, int seg1, int seg2, float* y) {
  double dec[256];
  for (int c = 0; c < 256; ++c) dec[c] = g4o_fp8_decode((uint8_t)c);
  for (int m = 0; m < M; ++m) {
    const uint16_t* a = A + (size_t)m * (size_t)lda;
    for (int n = 0; n < N; ++n) {
      const uint8_t* w = W + (size_t)n * (size_t)K;
      double acc = 0.0;
      for (int k = 0; k < K; ++k) acc += (double)g4o_bf16_to_f32(a[k]) * dec[w[k]];
      const float s = n < seg1 ? scale0 : (n < seg2 ? scale1 : scale2);
      y[(size_t)m * (size_t)N + n] = (float)((double)s * acc);
    }
  }
}

void g4o_gemv_fp8w(const uint16_t* a, const uint8_t* W, int N, int K, float scale, float* y) {
  double dec[256];
  for (int c = 0; c < 256; ++c) dec[c] = g4o_fp8_decode((uint8_t)c);
  for (int n = 0; n < N; ++n) {
    const uint8_t* w = W + (size_t)n * (size_t)K;
    double acc = 0.0;
    for (int k = 0; k < K; ++k) acc += (double)g4o_bf16_to_f32(a[k]) * dec[w[k]];
    y[n] = scale * (float)acc;
  }
}

/* ------------------------------------------------------------------------ */
/* RoPE (kernel_math.h:191-219): Llama half split; tables built in double.   */
/* ------------------------------------------------------------------------ */

void g4o_rope_tables(double theta, int head_dim, int max_pos, float* cos_t, float* sin_t) {
  const int half = head_dim / 2;
  for (int i = 0; i < half; ++i) {
    const double inv_freq = 1.0 / pow(theta, 2.0 * (double)i / head_dim);
    for (int p = 0; p < max_pos; ++p) {
      const double ang = (double)p * inv_freq;
      cos_t[(size_t)p * half + i] = (float)cos(ang);
      sin_t[(size_t)p * half + i] = (float)sin(ang);
    }
  }
}

/* out[i] = a*c - b*s, out[i + half] = b*c + a*s, float arithmetic. */
static void rope_head(const uint16_t* x, const float* c, const float* s, int d, float* out) {
  const int half = d / 2;
  for (int i = 0; i < half; ++i) {
    const float a = g4o_bf16_to_f32(x[i]);
    const float b = g4o_bf16_to_f32(x[i + half]);
    out[i] = a * c[i] - b * s[i];
    out[i + half] = b * c[i] + a * s[i];
  }
}

void g4o_rope_rows(const uint16_t* x, int rows, int heads, int d, const int* pos,
                   const float* cos_t, const float* sin_t, uint16_t* out) {
  float tmp[1024];
  const int half = d / 2;
  for (int r = 0; r < rows; ++r)
    for (int h = 0; h < heads; ++h) {
      const size_t o = ((size_t)r * heads + h) * (size_t)d;
      rope_head(x + o, cos_t + (size_t)pos[r] * half, sin_t + (size_t)pos[r] * half, d, tmp);
      for (int i = 0; i < d; ++i) out[o + i] = g4o_f32_to_bf16(tmp[i]);
    }
}

/* ------------------------------------------------------------------------ */
/* KV quantisation (kernel_math.h:71-173): s = amax / qmax in float; code =  */
/* clamp(round_half_away(x / s), -qmax, qmax); s == 0 gives code 0.          */
/* ------------------------------------------------------------------------ */

float g4o_kv_scale(float amax, int qmax) { return amax / (float)qmax; }

int g4o_kv_code(float x, float scale, int qmax) {
  if (scale == 0.0f) return 0;
  const float r = roundf(x / scale);
  if (r > (float)qmax) return qmax;
  if (r < -(float)qmax) return -qmax;
  return (int)r;
}

/* 80-byte K5 row: low nibbles two per byte (even dim low), then bit 4 of dim
 * j at bit j%8 of byte 64 + j/8 (kernel_math.h:156-165). */
void g4o_k5_pack_row(const uint8_t* codes, uint8_t* out) {
  for (int j = 0; j < 64; ++j)
    out[j] = (uint8_t)((codes[2 * j] & 0xFu) | ((codes[2 * j + 1] & 0xFu) << 4));
  for (int b = 0; b < 16; ++b) {
    unsigned plane = 0;
    for (int bit = 0; bit < 8; ++bit) plane |= ((codes[8 * b + bit] >> 4) & 1u) << bit;
    out[64 + b] = (uint8_t)plane;
  }
}

static int kv_row_bytes(int bits, int d, int is_k) {
  switch (bits) {
    case 16: return 2 * d;
    case 8: return d;
    case 4: return d / 2;
    case 5: return is_k ? d / 2 + d / 8 : d / 2;
    default: return 0;
  }
}

/* Quantise one d-wide row in groups and store codes + scales. */
static void kv_store_row(const float* val, int d, int bits, int is_k, int group, uint8_t* row,
                         float* scales) {
  const int qmax = bits == 8 ? 127 : ((bits == 5 && is_k) ? 15 : 7);
  const int off = bits == 8 ? 0 : qmax + 1;
  uint8_t codes[1024];
  for (int g0 = 0; g0 < d; g0 += group) {
    float amax = 0.0f;
    for (int j = g0; j < g0 + group; ++j) amax = fmaxf(amax, fabsf(val[j]));
    const float s = g4o_kv_scale(amax, qmax);
    scales[g0 / group] = s;
    for (int j = g0; j < g0 + group; ++j) codes[j] = (uint8_t)(g4o_kv_code(val[j], s, qmax) + off);
  }
  if (bits == 8) {
    memcpy(row, codes, (size_t)d);
  } else if (bits == 5 && is_k) {
    g4o_k5_pack_row(codes, row);
  } else {
    for (int j = 0; j < d / 2; ++j)
      row[j] = (uint8_t)((codes[2 * j] & 0xFu) | ((codes[2 * j + 1] & 0xFu) << 4));
  }
}

void g4o_rope_append(const uint16_t* q, long q_stride, const uint16_t* k, long k_stride,
                     const uint16_t* v, long v_stride, const float* cos_t, const float* sin_t,
                     int rows, int Hq, int Hk, int d, const int* pos, const int* arena_row,
                     int bits, int group, int rotate_k, int k_round_bf16, uint16_t* q_rot,
                     long q_rot_stride, void* cache_k, void* cache_v, float* k_scale,
                     float* v_scale, int stride) {
  const int half = d / 2;
  const int ng = d / group;
  const int kb = kv_row_bytes(bits, d, 1), vb = kv_row_bytes(bits, d, 0);
  float tmp[1024], kval[1024], vval[1024];
  for (int r = 0; r < rows; ++r) {
    const float* c = cos_t + (size_t)pos[r] * half;
    const float* s = sin_t + (size_t)pos[r] * half;
    if (q != NULL)
      for (int h = 0; h < Hq; ++h) {
        rope_head(q + (size_t)r * q_stride + (size_t)h * d, c, s, d, tmp);
        for (int i = 0; i < d; ++i)
          q_rot[(size_t)r * q_rot_stride + (size_t)h * d + i] = g4o_f32_to_bf16(tmp[i]);
      }
    for (int h = 0; h < Hk; ++h) {
      const uint16_t* kx = k + (size_t)r * k_stride + (size_t)h * d;
      const uint16_t* vx = v + (size_t)r * v_stride + (size_t)h * d;
      uint16_t kbits[1024];
      if (rotate_k) {
        rope_head(kx, c, s, d, tmp);
        for (int i = 0; i < d; ++i) {
          kbits[i] = g4o_f32_to_bf16(tmp[i]);
          kval[i] = k_round_bf16 ? g4o_bf16_to_f32(kbits[i]) : tmp[i];
        }
      } else {
        for (int i = 0; i < d; ++i) {
          kbits[i] = kx[i];
          kval[i] = g4o_bf16_to_f32(kx[i]);
        }
      }
      for (int i = 0; i < d; ++i) vval[i] = g4o_bf16_to_f32(vx[i]);
      const size_t slot = (size_t)h * (size_t)stride + (size_t)arena_row[r];
      uint8_t* krow = (uint8_t*)cache_k + slot * (size_t)kb;
      uint8_t* vrow = (uint8_t*)cache_v + slot * (size_t)vb;
      if (bits == 16) {
        memcpy(krow, kbits, (size_t)kb);
        memcpy(vrow, vx, (size_t)vb);
        continue;
      }
      kv_store_row(kval, d, bits, 1, group, krow, k_scale + slot * (size_t)ng);
      kv_store_row(vval, d, bits, 0, group, vrow, v_scale + slot * (size_t)ng);
    }
  }
}

/* row(p) = block_table[p / page] * page + p % page (kv_pool.cc:285-297). */
void g4o_row_table(const int32_t* block_table, int n, int page, int32_t* out) {
  for (int p = 0; p < n; ++p) out[p] = block_table[p / page] * page + p % page;
}

/* ------------------------------------------------------------------------ */
/* Split-KV decode attention (attention_split.cu:791-1074).                  */

/* Value of element i of a cached row: bf16 value, or the integer code (the
 * stored byte / nibble / 5-bit value minus its offset). */
static float kv_elem(const uint8_t* row, int bits, int is_k, int d, int i) {
  switch (bits) {
    case 16: return g4o_bf16_to_f32(((const uint16_t*)row)[i]);
    case 8: return (float)(int8_t)row[i];
    case 4: return (float)((int)((row[i / 2] >> (4 * (i & 1))) & 0xFu) - 8);
    case 5:
      if (!is_k) return (float)((int)((row[i / 2] >> (4 * (i & 1))) & 0xFu) - 8);
      return (float)((int)(((row[i / 2] >> (4 * (i & 1))) & 0xFu) |
                           (((row[d / 2 + i / 8] >> (i & 7)) & 1u) << 4)) - 16);
    default: return 0.0f;
  }
}

/* Element i of a cached row as the attention reads it: the code (or bf16
 * value), or for scale groups smaller than the row (this build's group-32 /
 * 64 pools) the element dequantised to bf16, bf16(code * scale_g). */
static float kv_att(const uint8_t* row, int bits, int is_k, int d, int i, const float* sc,
                    int group) {
  const float c = kv_elem(row, bits, is_k, d, i);
  if (bits == 16 || group >= d) return c;
  return g4o_bf16_to_f32(g4o_f32_to_bf16(c * sc[i / group]));
}

void g4o_attn_split(const uint16_t* q, int rows, int Hq, int Hk, int d, float scale,
                    const void* cache_k, const void* cache_v, const float* k_scale,
                    const float* v_scale, int bits, int group, int stride, const int* pos,
                    const int* const* pt, int window, int tps, uint16_t* out) {
  const int G = Hq / Hk, ngrp = d / group, tile = 64, span = tps * tile;
  const int kb = kv_row_bytes(bits, d, 1), vb = kv_row_bytes(bits, d, 0);
  const int quant = bits != 16;
  float qf[1024], oacc[1024], acc[1024], logit[64], pbf[64];
  float *ms = NULL, *ls = NULL, *os = NULL;
  for (int r = 0; r < rows; ++r) {
    const int len = pos[r] + 1;
    const int lo = window > 0 ? (len - window > 0 ? len - window : 0) : 0;
    const int nsplit = (len + span - 1) / span;
    ms = (float*)realloc(ms, sizeof(float) * nsplit);
    ls = (float*)realloc(ls, sizeof(float) * nsplit);
    os = (float*)realloc(os, sizeof(float) * (size_t)nsplit * d);
    for (int h = 0; h < Hq; ++h) {
      const int hk = h / G;
      for (int i = 0; i < d; ++i) qf[i] = g4o_bf16_to_f32(q[((size_t)r * Hq + h) * d + i]);
      int used0 = -1, used1 = -1;
      for (int sp = 0; sp < nsplit; ++sp) {
        const int t_begin = sp * span;
        const int t_end = len < t_begin + span ? len : t_begin + span;
        if (t_end <= lo) continue; /* the whole split is below the window */
        if (used0 < 0) used0 = sp;
        used1 = sp;
        const int t_first = t_begin > (lo / tile) * tile ? t_begin : (lo / tile) * tile;
        float m = -INFINITY, l = 0.0f;
        for (int i = 0; i < d; ++i) oacc[i] = 0.0f;
        for (int t0 = t_first; t0 < t_end; t0 += tile) {
          float mx = m;
          for (int j = 0; j < tile; ++j) {
            const int p = t0 + j;
            if (p >= t_end || p < lo) {
              logit[j] = -INFINITY;
              continue;
            }
            const int arow = pt != NULL && pt[r] != NULL ? pt[r][p] : p;
            if (arow < 0 || arow >= stride) { /* unmapped position: skipped, as the kernels do */
              logit[j] = -INFINITY;
              continue;
            }
            const uint8_t* krow = (const uint8_t*)cache_k + ((size_t)hk * stride + arow) * kb;
            const float* ks = quant ? k_scale + ((size_t)hk * stride + arow) * ngrp : NULL;
            float dot = 0.0f;
            if (!quant || ngrp > 1) {
              for (int i = 0; i < d; ++i) dot += qf[i] * kv_att(krow, bits, 1, d, i, ks, group);
            } else {
              for (int i = 0; i < d; ++i) dot += qf[i] * kv_elem(krow, bits, 1, d, i);
              dot *= ks[0];
            }
            logit[j] = g4o_bf16_to_f32(g4o_f32_to_bf16(scale * dot));
            if (logit[j] > mx) mx = logit[j];
          }
          const float alpha = mx == -INFINITY ? 1.0f : expf(m - mx);
          l *= alpha;
          m = mx;
          for (int i = 0; i < d; ++i) oacc[i] *= alpha;
          for (int j = 0; j < tile; ++j) {
            const float e = m == -INFINITY || logit[j] == -INFINITY ? 0.0f : expf(logit[j] - m);
            l += e;
            const int p = t0 + j;
            const int valid = logit[j] != -INFINITY;
            const int arow = valid ? (pt != NULL && pt[r] != NULL ? pt[r][p] : p) : 0;
            const float sv = quant && ngrp == 1 && valid ? v_scale[(size_t)hk * stride + arow] : 1.0f;
            pbf[j] = g4o_bf16_to_f32(g4o_f32_to_bf16(e * sv));
          }
          for (int j = 0; j < tile; ++j) {
            if (logit[j] == -INFINITY) continue;
            const int p = t0 + j;
            const int arow = pt != NULL && pt[r] != NULL ? pt[r][p] : p;
            const uint8_t* vrow = (const uint8_t*)cache_v + ((size_t)hk * stride + arow) * vb;
            const float* vs = quant ? v_scale + ((size_t)hk * stride + arow) * ngrp : NULL;
            for (int i = 0; i < d; ++i) oacc[i] += pbf[j] * kv_att(vrow, bits, 0, d, i, vs, group);
          }
        }
        ms[sp] = m;
        ls[sp] = l;
        memcpy(os + (size_t)sp * d, oacc, sizeof(float) * d);
      }
      float M = -INFINITY;
      for (int sp = used0; sp <= used1; ++sp) M = ms[sp] > M ? ms[sp] : M;
      float L = 0.0f;
      for (int i = 0; i < d; ++i) acc[i] = 0.0f;
      for (int sp = used0; sp <= used1; ++sp) {
        const float w = expf(ms[sp] - M);
        L += ls[sp] * w;
        for (int i = 0; i < d; ++i) acc[i] += os[(size_t)sp * d + i] * w;
      }
      for (int i = 0; i < d; ++i) out[((size_t)r * Hq + h) * d + i] = g4o_f32_to_bf16(acc[i] / L);
    }
  }
  free(ms);
  free(ls);
  free(os);
}

/* One head's online softmax over the 64-position tiles [t_first, t_end) of
 * positions, keys masked outside [lo, len): the state the split and prefill
 * kernels keep (attention_split.cu:873-1020, prefill_gemm.cu:878-928). */
static void attn_tiles(const float* qf, int hk, float scale, const void* cache_k,
                       const void* cache_v, const float* k_scale, const float* v_scale, int bits,
                       int group, int d, int stride, const int* pt, int t_first, int t_end, int lo,
                       float* m_out, float* l_out, float* oacc) {
  const int ngrp = d / group, tile = 64, quant = bits != 16;
  const int kb = kv_row_bytes(bits, d, 1), vb = kv_row_bytes(bits, d, 0);
  float logit[64], pbf[64];
  float m = -INFINITY, l = 0.0f;
  for (int i = 0; i < d; ++i) oacc[i] = 0.0f;
  for (int t0 = t_first; t0 < t_end; t0 += tile) {
    float mx = m;
    for (int j = 0; j < tile; ++j) {
      const int p = t0 + j;
      if (p >= t_end || p < lo) {
        logit[j] = -INFINITY;
        continue;
      }
      const int arow = pt != NULL ? pt[p] : p;
      const uint8_t* krow = (const uint8_t*)cache_k + ((size_t)hk * stride + arow) * kb;
      const float* ks = quant ? k_scale + ((size_t)hk * stride + arow) * ngrp : NULL;
      float dot = 0.0f;
      if (!quant || ngrp > 1) {
        for (int i = 0; i < d; ++i) dot += qf[i] * kv_att(krow, bits, 1, d, i, ks, group);
      } else {
        for (int i = 0; i < d; ++i) dot += qf[i] * kv_elem(krow, bits, 1, d, i);
        dot *= ks[0];
      }
      logit[j] = g4o_bf16_to_f32(g4o_f32_to_bf16(scale * dot));
      if (logit[j] > mx) mx = logit[j];
    }
    const float alpha = mx == -INFINITY ? 1.0f : expf(m - mx);
    l *= alpha;
    m = mx;
    for (int i = 0; i < d; ++i) oacc[i] *= alpha;
    for (int j = 0; j < tile; ++j) {
      const float e = m == -INFINITY || logit[j] == -INFINITY ? 0.0f : expf(logit[j] - m);
      l += e;
      const int valid = logit[j] != -INFINITY;
      const int arow = valid ? (pt != NULL ? pt[t0 + j] : t0 + j) : 0;
      const float sv = quant && ngrp == 1 && valid ? v_scale[(size_t)hk * stride + arow] : 1.0f;
      pbf[j] = g4o_bf16_to_f32(g4o_f32_to_bf16(e * sv));
    }
    for (int j = 0; j < tile; ++j) {
      if (logit[j] == -INFINITY) continue;
      const int arow = pt != NULL ? pt[t0 + j] : t0 + j;
      const uint8_t* vrow = (const uint8_t*)cache_v + ((size_t)hk * stride + arow) * vb;
      const float* vs = quant ? v_scale + ((size_t)hk * stride + arow) * ngrp : NULL;
      for (int i = 0; i < d; ++i) oacc[i] += pbf[j] * kv_att(vrow, bits, 0, d, i, vs, group);
    }
  }
  *m_out = m;
  *l_out = l;
}

void g4o_prefill_attn(const uint16_t* q, int rows, int Hq, int Hk, int d, float scale,
                      const void* cache_k, const void* cache_v, const float* k_scale,
                      const float* v_scale, int bits, int group, int stride, int base_pos,
                      const int* pt, int window, uint16_t* out) {
  const int G = Hq / Hk;
  float qf[1024], oacc[1024];
  for (int r = 0; r < rows; ++r) {
    const int len = base_pos + r + 1;
    const int lo = window > 0 ? (len - window > 0 ? len - window : 0) : 0;
    for (int h = 0; h < Hq; ++h) {
      for (int i = 0; i < d; ++i) qf[i] = g4o_bf16_to_f32(q[((size_t)r * Hq + h) * d + i]);
      float m, l;
      attn_tiles(qf, h / G, scale, cache_k, cache_v, k_scale, v_scale, bits, group, d, stride, pt,
                 (lo / 64) * 64, len, lo, &m, &l, oacc);
      const float inv = 1.0f / l;
      for (int i = 0; i < d; ++i) out[((size_t)r * Hq + h) * d + i] = g4o_f32_to_bf16(oacc[i] * inv);
    }
  }
}
