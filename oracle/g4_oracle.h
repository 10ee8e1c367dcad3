/*
 * g4_oracle.h - CPU restatement of the reference engine's non-GEMM layer math.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or the timed CPU baseline). The product path (libgranite4_layerops.so)
 * never links, loads or calls it.
 *
 * Every function cites the reference file:line whose behaviour it restates
 * (paths relative to the reference repo root). Element types: bf16 values
 * travel as uint16_t bit patterns, FP8 e4m3 as uint8_t codes.
 *
 * KV formats (the reference's `bits` argument, forward_gpu.cu:731-750):
 *   16 = bf16 rows, 8 = int8 + f32 scale, 4 = int4 (two codes per byte) +
 *   scale, 5 = K 5-bit (80-byte row: 64 nibble bytes + 16-byte high-bit plane)
 *   with V int4. `group` is the number of head-dim elements sharing one scale
 *   (the reference uses the whole 128-dim row; 32 is this build's group-32
 *   extension), so a row carries d/group scales.
 */
#ifndef G4_ORACLE_H
#define G4_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* bf16 <-> f32, round-to-nearest-even (kernel_math.h:39-55). */
float g4o_bf16_to_f32(uint16_t b);
uint16_t g4o_f32_to_bf16(float f);

/* xorshift64* test-input generator (kernel_math.h:637-658). */
uint64_t g4o_rng_next(uint64_t* state);
float g4o_rng_float(uint64_t* state);
void g4o_fill_uniform_bf16(uint64_t seed, double a, size_t n, uint16_t* out);
void g4o_fill_uniform_f32(uint64_t seed, double a, size_t n, float* out);
void g4o_fill_normal_bf16(uint64_t seed, double mean, double stddev, size_t n, uint16_t* out);
void g4o_fill_u32(uint64_t seed, size_t n, uint32_t* out);

/* FP8 e4m3 (fp8_convert.cc:47-157, gpu_pack.cc:44-51, gpu_pack.cc:296-308). */
uint8_t g4o_fp8_encode(double v);
double g4o_fp8_decode(uint8_t code);
float g4o_fp8_scale_for(double amax);
void g4o_fp8_encode_scaled_bf16(const uint16_t* x, size_t n, float scale, uint8_t* codes);
float g4o_fp8_quantize_bf16(const uint16_t* x, size_t n, uint8_t* codes);

/* Embedding gather (kernel_math.h:450-453, prefill_gemm.cu:280-301). */
void g4o_embed_rows(const int32_t* tokens, int rows, const uint16_t* emb, int H, float mult,
                    uint16_t* out);

/* RMSNorm and the fused residual add (kernel_math.h:178-184, 527-528;
 * kernels_phase2.cu:51-132; forward_gpu.cu:992-994). */
void g4o_rmsnorm(const uint16_t* x, const uint16_t* w, float eps, int rows, int cols,
                 uint16_t* out);
void g4o_add_rmsnorm(const uint16_t* res, const uint16_t* branch, float mult, const uint16_t* w,
                     float eps, int rows, int cols, uint16_t* res_out, uint16_t* normed);

/* SwiGLU (prefill_gemm.cu:1194-1203, kernels_phase2.cu:643-651). gu is
 * [rows][2I]: gate at [r][i], up at [r][I + i]. */
void g4o_swiglu_bf16(const uint16_t* gu, int rows, int I, uint16_t* act);
void g4o_silu_mul_f32(const float* gu, int I, int rows, uint16_t* act);

/* FP8 x FP8 GEMM value before the epilogue's rounding:
 * y[m][n] = (float)((double)(a_scale * w_scale(n)) * S[m][n]), with
 * S = sum_k dec(A[m][k]) * dec(W[n][k]) accumulated in double (every product
 * of two e4m3 values is exact) and w_scale(n) = scale0 / scale1 / scale2 split
 * at seg1 / seg2 (the reference's GemmEpilogue, prefill_gemm.h:12-28,
 * epi_scale prefill_gemm.cu:65-67). The reference checks its GEMM the same
 * way: against the double-accumulated exact product, within 2 bf16 ulp of
 * the rounded epilogue value (test_kernels.cu:1685-1719). A is [M][lda]
 * bytes, W [N][K], y [M][N]. */
void g4o_gemm_fp8(const uint8_t* A, int lda, float a_scale, const uint8_t* W, int M, int N, int K,
                  float scale0, float scale1, float scale2, int seg1, int seg2, float* y);

/* The reference's prefill GEMM value before its epilogue rounding
 * (prefill_gemm.h:34-39, epi_store prefill_gemm.cu:69-89): bf16 A [M][lda]
 * times fp8 e4m3 W [N][K]^T, y[m][n] = (float)((double)scale(n) * S), S the
 * exact sum of bf16(a) * fp8(w) products (each exact) accumulated in double;
 * scale(n) as g4o_gemm_fp8's. */
void g4o_gemm_bf16w(const uint16_t* A, int lda, const uint8_t* W, int M, int N, int K,
                    float scale0, float scale1, float scale2, int seg1, int seg2, float* y);

/* Decode GEMV value before rounding (gemv_row_dequant forward_gpu.cu:934-994):
 * y[n] = scale * (float)S[n], S = sum_k bf16(a[k]) * fp8(W[n][k]) in double
 * (products exact). a bf16 [K], W [N][K], y [N]. */
void g4o_gemv_fp8w(const uint16_t* a, const uint8_t* W, int N, int K, float scale, float* y);

/* RoPE (kernel_math.h:191-219, kernels_phase2.cu:138-162). */
void g4o_rope_tables(double theta, int head_dim, int max_pos, float* cos_t, float* sin_t);
void g4o_rope_rows(const uint16_t* x, int rows, int heads, int d, const int* pos,
                   const float* cos_t, const float* sin_t, uint16_t* out);

/* KV quantisation (kernel_math.h:71-173, device_math.cuh:105-210). qmax is
 * 127 (int8), 7 (int4) or 15 (K5). Returns the signed code before offset. */
float g4o_kv_scale(float amax, int qmax);
int g4o_kv_code(float x, float scale, int qmax);
void g4o_k5_pack_row(const uint8_t* codes128, uint8_t* out80);

/* RoPE of q/k fused with the quantised KV write (forward_gpu.cu:598-729,
 * prefill_gemm.cu:306-624, kernels_phase2.cu:381-577). Row r sits at RoPE
 * position pos[r] and writes arena row arena_row[r]. rotate_k = 0 appends K
 * as given (the standalone kv_append kernels); k_round_bf16 = 1 quantises the
 * bf16-rounded rotated K (decode / multi kernels), 0 the f32 value (prefill).
 * q may be NULL (no query heads). Caches are [Hk][stride][row bytes]; scales
 * [Hk][stride][d / group]. */
void g4o_rope_append(const uint16_t* q, long q_stride, const uint16_t* k, long k_stride,
                     const uint16_t* v, long v_stride, const float* cos_t, const float* sin_t,
                     int rows, int Hq, int Hk, int d, const int* pos, const int* arena_row,
                     int bits, int group, int rotate_k, int k_round_bf16, uint16_t* q_rot,
                     long q_rot_stride, void* cache_k, void* cache_v, float* k_scale,
                     float* v_scale, int stride);

/* Split-KV decode attention over the paged pool (attention_split.cu: the
 * tensor-core kernel :791-1047 and attn_combine_kernel :1049-1074, launched
 * by attn_split :1083-1255). Row r (query q[r][Hq][d], Hq = 4 Hk, query head h
 * reads KV head h / 4) sits at position pos[r] and attends to positions
 * [lo, pos[r]], lo = max(0, pos[r] + 1 - window) when window > 0 else 0,
 * found at arena row pt[r][position] (pt[r] NULL: row = position); a
 * position whose row is outside [0, stride) is skipped (this library's rule
 * for unmapped pages; the reference never passes one). Cache formats as
 * g4o_rope_append's. Positions are cut into 64-position tiles and
 * the tiles into splits of tps tiles; each split keeps its own online
 * softmax, and the splits are combined, as the kernels do:
 *   logit  = bf16(scale * dot), dot = q . k (bf16 K), (q . codes) * k_scale
 *            (quantised K with the reference's one scale per row, group =
 *            d), or q . bf16(code * k_scale_g) (scale groups of 32 or 64,
 *            this build's extension: each element dequantised to bf16 with
 *            its group's scale, then the bf16 path)
 *   p      = exp(logit - m) (f32, m = the split's running maximum), summed
 *            unrounded into l; the value product uses bf16(p * v_scale)
 *            against the code (one scale per row), or bf16(p) against the
 *            bf16 value (bf16 V; scale groups: bf16(code * v_scale_g))
 *   out    = bf16(sum_s o_s w_s / sum_s l_s w_s), w_s = exp(m_s - max_s m_s).
 * Sums run in f32 in key / dim order. */
void g4o_attn_split(const uint16_t* q, int rows, int Hq, int Hk, int d, float scale,
                    const void* cache_k, const void* cache_v, const float* k_scale,
                    const float* v_scale, int bits, int group, int stride, const int* pos,
                    const int* const* pt, int window, int tps, uint16_t* out);

/* Causal prefill attention over the paged pool (prefill_gemm.cu:626-1188,
 * prefill_attention :1392-1474; the quantised-cache form keeps the codes and
 * applies the scales to the logits and probabilities, :942-1188). Query rows
 * q [rows][Hq][d] sit at positions base_pos + r and attend to positions
 * [lo, base_pos + r] (lo as g4o_attn_split's window rule) through pt (NULL:
 * row = position), in one pass of 64-position tiles from position 0: the
 * same logits, online softmax and value product as g4o_attn_split, and
 * out = bf16(o * (1 / l)). */
void g4o_prefill_attn(const uint16_t* q, int rows, int Hq, int Hk, int d, float scale,
                      const void* cache_k, const void* cache_v, const float* k_scale,
                      const float* v_scale, int bits, int group, int stride, int base_pos,
                      const int* pt, int window, uint16_t* out);

/* Paged pool: position -> arena row (kv_pool.cc:285-297). */
void g4o_row_table(const int32_t* block_table, int n, int page, int32_t* out);

/* bench.py's CPU baseline (g4_cpu_step.c): the T-token one-layer step of
 * BASELINE config 3 (embed from the full 100352-row table, add+RMSNorm ->
 * FP8, SwiGLU -> FP8, RoPE + int8 KV) with the functions above, split by rows
 * over `threads` host threads, repeated for about `seconds`. Returns the
 * steps done and their wall time in *wall_s; -1 on bad arguments. */
int g4o_cpu_step_bench(int T, int threads, double seconds, double* wall_s);

#ifdef __cplusplus
}
#endif

#endif /* G4_ORACLE_H */
