/*
 * granite4_layerops.h - C ABI of the MI355X (gfx950) non-GEMM layer ops of the
 * Granite 4.2 8B engine: embedding gather, residual add + RMSNorm (bf16 or
 * FP8 e4m3 output), SwiGLU (bf16 or FP8), RoPE on Q/K fused with the
 * quantised write into the paged KV arena.
 *
 * Conventions (the reference engine's, kernels_phase2.cu:822-836,
 * engine/CMakeLists.txt:39-48):
 *   - every pointer is device memory owned by the caller, except where a
 *     function says it allocates (granite4_rope_tables_build);
 *   - return 0 on success, -1 on invalid arguments or a launch error, with a
 *     diagnostic on stderr; outputs are untouched when -1 comes from argument
 *     validation;
 *   - launches are asynchronous on the calling host thread's current stream
 *     (hipStreamPerThread unless granite4_set_stream chose another), never
 *     synchronise and never allocate, so a caller may capture them in a HIP
 *     graph;
 *   - decode variants read the position from device memory (d_pos).
 *
 * Shapes of the Granite 4.2 8B model: H = 4096, I = 12800, Hq = 32, Hk = 8,
 * d = 128, 16-token KV pages.
 *
 * KV arena (per layer, forward_gpu.cu:1315-1343): K and V are
 * [Hk][stride][row bytes] with row bytes 256 (bf16), 128 (int8), 64 (int4),
 * 80 (K5: 64 nibble bytes + 16-byte high-bit plane; V stays int4). Scales
 * are f32 [Hk][stride][d / group]; group = d reproduces the reference's one
 * scale per (head, token) row, group = 32 is the group-32 format. Logical
 * position p lives in arena row d_pt[p] (d_pt == NULL: row p), with
 * d_pt[p] = block_table[p / 16] * 16 + p % 16 (kv_pool.cc:285-297).
 * A row index outside [0, stride) or a position outside the cos/sin table is
 * skipped by the kernels (no write) instead of faulting.
 */
#ifndef GRANITE4_LAYEROPS_H
#define GRANITE4_LAYEROPS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------------------
 * Stream selection (the reference builds with the per-thread default stream;
 * this keeps that default and lets a caller such as a PyTorch harness name
 * its own stream). `stream` is a hipStream_t; NULL restores the default.
 * ------------------------------------------------------------------------- */
int granite4_set_stream(void* stream);
void* granite4_get_stream(void);

/* Library / device identification for harnesses: writes the gfx arch name of
 * the current device (e.g. "gfx950") into buf; 0 on success. */
int granite4_device_arch(char* buf, int buf_len);

/* ===========================================================================
 * Entry points with the reference's names and signatures (drop-in).
 * ========================================================================= */

/* kernels_phase2.cu:868. Builds cos/sin [max_pos][head_dim/2] f32 tables on
 * the host in double (kernel_math.h:191-206), allocates them with hipMalloc
 * and uploads them; the caller frees both (hipFree or
 * granite4_rope_tables_free). Synchronous. */
int granite4_rope_tables_build(double theta, int head_dim, int max_pos, float** d_cos,
                               float** d_sin);
/* Frees tables from granite4_rope_tables_build (no reference counterpart). */
int granite4_rope_tables_free(float* d_cos, float* d_sin);

/* kernels_phase2.cu:910 / :922. y = bf16(x * rsqrt(mean(x^2) + eps) * w) per
 * row; the _batched form also requires rows <= 16 (kMaxVerifyRows). */
int granite4_kernel_rmsnorm(const uint16_t* d_x, const uint16_t* d_w, float eps, int rows,
                            int cols, uint16_t* d_out);
int granite4_kernel_rmsnorm_batched(const uint16_t* d_x, const uint16_t* d_w, float eps,
                                    int rows, int cols, uint16_t* d_out);

/* kernels_phase2.cu:938. Row r of x ([rows][head_dim]) is rotated with table
 * row r (the row index is the position). */
int granite4_kernel_rope(const uint16_t* d_x, const float* d_cos, const float* d_sin, int rows,
                         int head_dim, uint16_t* d_out);

/* forward_gpu.cu:3814. Every head of x ([heads][d]) rotated with one table row
 * (d_cos_row / d_sin_row point at that position's d/2 entries). */
int granite4_kernel_rope_at_pos(const uint16_t* d_x, const float* d_cos_row,
                                const float* d_sin_row, int heads, int d, uint16_t* d_out);

/* forward_gpu.cu:3829. Row r ([rows][heads][d]) rotated with table row r of
 * d_cos / d_sin; rows <= 16. */
int granite4_kernel_rope_at_pos_batched(const uint16_t* d_x, const float* d_cos,
                                        const float* d_sin, int rows, int heads, int d,
                                        uint16_t* d_out);

/* kernels_phase2.cu:1087 / :1107 / :1133 / :1159. Append `rows` consecutive
 * positions base_pos.. of already-rotated K and raw V ([rows][Hk][d] bf16) to
 * the caches through d_pt; rows <= 16, stride >= base_pos + rows. Quantised
 * forms store one f32 scale per (head, row); k5v4 needs d == 128. */
int granite4_kernel_kv_append_batched(const uint16_t* d_src_k, const uint16_t* d_src_v,
                                      uint16_t* d_cache_k, uint16_t* d_cache_v, int base_pos,
                                      int rows, int stride, int Hk, int d, const int* d_pt);
int granite4_kernel_kv_append_int8_batched(const uint16_t* d_src_k, const uint16_t* d_src_v,
                                           int8_t* d_cache_k, int8_t* d_cache_v,
                                           float* d_cache_k_scale, float* d_cache_v_scale,
                                           int base_pos, int rows, int stride, int Hk, int d,
                                           const int* d_pt);
int granite4_kernel_kv_append_int4_batched(const uint16_t* d_src_k, const uint16_t* d_src_v,
                                           uint8_t* d_cache_k, uint8_t* d_cache_v,
                                           float* d_cache_k_scale, float* d_cache_v_scale,
                                           int base_pos, int rows, int stride, int Hk, int d,
                                           const int* d_pt);
int granite4_kernel_kv_append_k5v4_batched(const uint16_t* d_src_k, const uint16_t* d_src_v,
                                           uint8_t* d_cache_k, uint8_t* d_cache_v,
                                           float* d_cache_k_scale, float* d_cache_v_scale,
                                           int base_pos, int rows, int stride, int Hk, int d,
                                           const int* d_pt);

/* forward_gpu.cu:3847. RoPE q and k of `rows` verify rows (table row r of
 * d_cos / d_sin for row r) into d_q_rot / d_k_rot, then append rotated K and
 * raw V at positions base_pos.. (bf16 cache); rows <= 16. */
int granite4_kernel_verify_qkv_stage(const uint16_t* d_q, const uint16_t* d_k,
                                     const uint16_t* d_v, const float* d_cos,
                                     const float* d_sin, int base_pos, int rows, int Hq, int Hk,
                                     int d, int cache_stride, uint16_t* d_q_rot,
                                     uint16_t* d_k_rot, uint16_t* d_cache_k,
                                     uint16_t* d_cache_v, const int* d_pt);

/* C-linkage twins of the reference's C++ `granite4::prefill_*` launchers
 * (prefill_gemm.h:41-105); the C++ wrappers at the end of this header keep the
 * reference's names. */

/* prefill_gemm.cu:1300. out[r] = bf16(mult * emb[d_tokens[start + r]]). */
int granite4_prefill_embed_rows(const int32_t* d_tokens, int start, int rows,
                                const uint16_t* emb, float mult, uint16_t* out, int H);

/* prefill_gemm.cu:1311 / :1331 / :1356 / :1378. qkv is token-major
 * [rows][(Hq + 2 Hk) d]; row r sits at position base_pos + r. q is rotated
 * into q_rot [rows][Hq d]; k is rotated and, with v, written through d_pt.
 * The quantised forms quantise the f32 rotated K (not its bf16 rounding),
 * one scale per (head, row), and need d == 128. */
int granite4_prefill_rope_split_append(const uint16_t* qkv, const float* cos_tbl,
                                       const float* sin_tbl, int base_pos, int rows, int Hq,
                                       int Hk, int d, int stride, uint16_t* q_rot,
                                       uint16_t* cache_k, uint16_t* cache_v, const int* d_pt);
int granite4_prefill_rope_split_append_int8(const uint16_t* qkv, const float* cos_tbl,
                                            const float* sin_tbl, int base_pos, int rows,
                                            int Hq, int Hk, int d, int stride, uint16_t* q_rot,
                                            int8_t* cache_k, int8_t* cache_v,
                                            float* cache_k_scale, float* cache_v_scale,
                                            const int* d_pt);
int granite4_prefill_rope_split_append_int4(const uint16_t* qkv, const float* cos_tbl,
                                            const float* sin_tbl, int base_pos, int rows,
                                            int Hq, int Hk, int d, int stride, uint16_t* q_rot,
                                            uint8_t* cache_k, uint8_t* cache_v,
                                            float* cache_k_scale, float* cache_v_scale,
                                            const int* d_pt);
int granite4_prefill_rope_split_append_k5v4(const uint16_t* qkv, const float* cos_tbl,
                                            const float* sin_tbl, int base_pos, int rows,
                                            int Hq, int Hk, int d, int stride, uint16_t* q_rot,
                                            uint8_t* cache_k, uint8_t* cache_v,
                                            float* cache_k_scale, float* cache_v_scale,
                                            const int* d_pt);

/* prefill_gemm.cu:1468. act[r][i] = bf16(g * sigmoid(g) * u) with f32
 * gu [rows][2I] (gate at [r][i], up at [r][I + i]). */
int granite4_prefill_silu_mul(const float* gu, int I, int rows, uint16_t* act);

/* Multi-session descriptor (forward_gpu_api.h:163-182), layout-identical. */
#define GRANITE4_MAX_VERIFY_ROWS 16
#define GRANITE4_MAX_TREE_DEPTH 8
typedef struct GpuMultiRows {
  int n;
  int pos[GRANITE4_MAX_VERIFY_ROWS];
  const int* pt[GRANITE4_MAX_VERIFY_ROWS];
  int32_t* tok[GRANITE4_MAX_VERIFY_ROWS];
  int grp[GRANITE4_MAX_VERIFY_ROWS];
  int tree;
  int slot[GRANITE4_MAX_VERIFY_ROWS];
  int tbase[GRANITE4_MAX_VERIFY_ROWS];
  int tail[GRANITE4_MAX_VERIFY_ROWS][GRANITE4_MAX_TREE_DEPTH];
} GpuMultiRows;

/* forward_gpu.cu:3891 / :3907 / :3914 (C-linkage twins of gpu_multi_rope,
 * gpu_multi_rope_append, gpu_multi_kv_append). Row r is position
 * d_rows->pos[r]; its KV goes to arena row d_rows->pt[r][slot] with slot =
 * tree ? d_rows->slot[r] : pos[r]. bits: 16 / 8 / 4 / 5 (K5V4). The multi
 * forms quantise the bf16-rounded rotated K, as the reference's decode path. */
int granite4_multi_rope(const uint16_t* x, const float* cos_tbl, const float* sin_tbl,
                        const GpuMultiRows* d_rows, int rows, int heads, int d, uint16_t* out);
int granite4_multi_rope_append(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                               const float* cos_tbl, const float* sin_tbl,
                               const GpuMultiRows* d_rows, int rows, int Hq, int Hk, int d,
                               int bits, void* cache_k, void* cache_v, float* k_scale,
                               float* v_scale, int stride, uint16_t* q_rot);
int granite4_multi_kv_append(const uint16_t* k, const uint16_t* v, int bits, void* cache_k,
                             void* cache_v, float* k_scale, float* v_scale,
                             const GpuMultiRows* d_rows, int rows, int stride, int Hk, int d);
/* embed_multi_v8_kernel (forward_gpu.cu:370-378, the embedding of
 * forward_multi_step :2517-2524): out[r] = bf16(mult * emb[tok]) with tok =
 * d_rows->tok[r][tree ? slot[r] : pos[r]]; a token outside [0, vocab) (or a
 * NULL token array) writes a zero row. H % 8 == 0, rows <= 16. */
int granite4_multi_embed(const GpuMultiRows* d_rows, int rows, const uint16_t* emb, int vocab,
                         int H, float mult, uint16_t* out);

/* ===========================================================================
 * Fused entry points the MI355X build adds (no single reference function;
 * each cites the reference pieces it fuses).
 * ========================================================================= */

/* Non-allocating twin of granite4_rope_tables_build: fills caller-owned
 * device tables [max_pos][head_dim / 2]. Synchronous. */
int granite4_rope_tables_fill(double theta, int head_dim, int max_pos, float* d_cos,
                              float* d_sin);

/* Embedding gather with a bounds check (forward_gpu.cu:84-101,
 * prefill_gemm.cu:292-301): out[r] = bf16(mult * emb[tokens[r]]); a token
 * outside [0, vocab) writes a zero row. */
int granite4_embed_rows(const int32_t* d_tokens, int rows, const uint16_t* emb, int vocab,
                        int H, float mult, uint16_t* out);
/* Decode form: one row, token d_tokens[*d_pos] (embed_v8_kernel). */
int granite4_embed_at_pos(const int32_t* d_tokens, const int* d_pos, const uint16_t* emb,
                          int vocab, int H, float mult, uint16_t* out);

/* Residual add + RMSNorm (forward_gpu.cu:992-994 epilogue + rmsnorm_kernel
 * kernels_phase2.cu:51-132):
 *   res'   = bf16(float(res) + resid_mult * float(branch))   (written to d_res_out)
 *   normed = bf16(float(res') * rsqrt(mean(res'^2) + eps) * float(w))
 * d_branch == NULL skips the add (normed = rmsnorm(res)); d_res_out may alias
 * d_res; d_res_out == NULL skips that write. */
int granite4_add_rmsnorm(const uint16_t* d_res, const uint16_t* d_branch, float resid_mult,
                         const uint16_t* d_w, float eps, int rows, int cols, uint16_t* d_res_out,
                         uint16_t* d_normed);

/* As granite4_add_rmsnorm, with the normed output as FP8 e4m3 codes under one
 * per-tensor scale: scale = float(amax / 448) over all |normed| (bf16 values),
 * code = RNE_e4m3(normed / scale) (the reference's weight quantiser
 * gpu_pack.cc:44-51, 296-308 applied to the bf16 normed tensor). One launch
 * when the tensor fits in the registers of one resident grid (its workgroups
 * meet once to agree on the maximum), otherwise two launches
 * (amax, then encode). d_work: caller-owned device workspace of at least
 * GRANITE4_FP8_WORK_BYTES(rows) bytes (= granite4_fp8_work_bytes(rows)): the
 * two-launch form's per-workgroup partial maxima and per-row 1 / rms, and
 * the single-launch form's synchronisation slots. Zero-fill it once after
 * allocating it; the ops keep it valid from then on. Calls that share one
 * workspace must be ordered on one stream. */
#define GRANITE4_FP8_MAX_PARTIALS 1024
#define GRANITE4_FP8_WORK_BYTES(rows) (12544 + 4 * (rows))
size_t granite4_fp8_work_bytes(int rows);
/* FP8 launch form for granite4_add_rmsnorm_fp8 / granite4_swiglu_fp8, process
 * wide: 0 (default) = one launch when the tensor fits the registers of one
 * resident grid, else two; 1 = always two launches; 2 = as 0, with the single
 * launch made through hipLaunchCooperativeKernel, so that the runtime
 * guarantees the co-residency instead of the occupancy query (measured on
 * MI355X: about 92 us more per launch than mode 0, in a HIP graph or not, and
 * graph-capturable). Every form gives identical codes and scales. Returns the
 * previous mode, -1 for another value. No reference counterpart (a tuning
 * switch).
 *
 * The single-launch form's workgroups meet once inside the launch, so it
 * needs every workgroup of its grid resident at the same time. The library
 * sizes the grid from the occupancy query, which holds when the call has the
 * device to itself. Another stream's kernels (or another process's) holding
 * CUs for longer than the bounded wait (about 2^20 polls), or two
 * single-launch calls in flight at once on different streams, break that.
 * The wait then gives up instead of hanging: the scale written is NaN, and
 * the workspace's sticky error word is set. A caller that overlaps streams on
 * one device selects mode 1, whose two launches need no co-residency. */
int granite4_set_fp8_launch_mode(int mode);
/* Reads the workspace's sticky synchronisation-error word: 0 if no
 * single-launch FP8 call on d_work gave up waiting since the last clear, 1
 * if one did (that call's codes and scale are invalid; its scale is NaN where
 * the give-up reached workgroup 0), -1 on a HIP error. Every call advances
 * the workspace's generation, give-ups included, so later calls are correct
 * without a clear. clear != 0 resets the word and the synchronisation slots
 * to their zero-filled start. Synchronises the calling thread's stream (not
 * for use inside graph capture). d_work NULL reads the current device's static scratch of
 * granite4_add_rmsnorm_fp8_noalloc. No reference counterpart. */
int granite4_fp8_sync_status(void* d_work, int clear);
/* Test hook: sets the process-wide poll limit of the single-launch forms'
 * bounded waits and of the attention's fused-combine wait (default 2^20)
 * and returns the previous one, -1 for a negative limit. 0 makes every wait
 * give up at once, so a test can drive
 * the error path while every kernel still exits normally. No reference
 * counterpart. */
int granite4_debug_set_sync_spin_limit(int limit);
int granite4_add_rmsnorm_fp8(const uint16_t* d_res, const uint16_t* d_branch, float resid_mult,
                             const uint16_t* d_w, float eps, int rows, int cols,
                             uint16_t* d_res_out, uint8_t* d_codes, float* d_scale,
                             void* d_work);

/* No reference counterpart: for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). granite4_add_rmsnorm_fp8 without the d_work argument: its
 * workspace is a static device array in the library (274,688 bytes per GPU,
 * held until the process ends), so the call allocates nothing. rows <= 65536
 * (-1 with a message beyond that). Every call on one GPU shares that array:
 * calls that overlap on one GPU (other streams, other host threads) race and
 * must be serialised by the caller. The first call on a device zero-fills
 * the array's synchronisation area with a kernel on the calling stream.
 * granite4_fp8_sync_status(NULL, clear) reads its error word. */
int granite4_add_rmsnorm_fp8_noalloc(const uint16_t* d_res, const uint16_t* d_branch,
                                     float resid_mult, const uint16_t* d_w, float eps, int rows,
                                     int cols, uint16_t* d_res_out, uint8_t* d_codes,
                                     float* d_scale);

/* SwiGLU from bf16 gate|up rows gu [rows][2I] (gate at [r][i], up at
 * [r][I + i]; prefill_gemm.cu:1194-1203 with bf16 inputs):
 * act = bf16(g * (1 / (1 + exp(-g))) * u). */
int granite4_swiglu(const uint16_t* d_gu, int rows, int I, uint16_t* d_act);

/* SwiGLU with FP8 requantisation of act (per-tensor scale, as
 * granite4_add_rmsnorm_fp8; d_work needs GRANITE4_FP8_WORK_BYTES(0)). d_act
 * may be NULL; when given it receives the bf16 act, and the encode launch
 * reads it back (2 B / element) instead of re-reading gate|up (4 B) and
 * re-evaluating the SiLU. */
int granite4_swiglu_fp8(const uint16_t* d_gu, int rows, int I, uint8_t* d_codes,
                        float* d_scale, void* d_work, uint16_t* d_act);

/* RoPE of q / k fused with the KV write (rope_append_multi_kernel
 * forward_gpu.cu:598-729 and rope_split_append_*_kernel prefill_gemm.cu:
 * 306-624, generalised).
 *   q, k, v      bf16 rows with element strides q_stride / k_stride / v_stride
 *                (prefill: one qkv buffer, q = qkv, k = qkv + Hq d,
 *                v = qkv + (Hq + Hk) d, all strides (Hq + 2 Hk) d); q may be
 *                NULL (no query heads).
 *   position     row r uses RoPE position d_pos_rows[r] when given, else
 *                base_pos + r; its arena row is d_arena_rows[r] when given,
 *                else d_pt[pos] (d_pt NULL: pos).
 *   bits / group 16, 8, 4 or 5 (K5V4); group 32, 64 or 128 (= d) elements per
 *                scale.
 *   k_round_bf16 1: quantise the bf16-rounded rotated K (decode / multi
 *                semantics); 0: the f32 value (prefill semantics).
 *   rotate_k     0: K is already rotated (the kv_append kernels).
 * d must be 128. max_pos bounds the cos/sin tables. */
int granite4_rope_append(const uint16_t* q, long q_stride, const uint16_t* k, long k_stride,
                         const uint16_t* v, long v_stride, const float* cos_tbl,
                         const float* sin_tbl, int max_pos, int rows, int Hq, int Hk, int d,
                         int base_pos, const int* d_pos_rows, const int* d_pt,
                         const int* d_arena_rows, int bits, int group, int k_round_bf16,
                         int rotate_k, uint16_t* q_rot, long q_rot_stride, void* cache_k,
                         void* cache_v, float* k_scale, float* v_scale, int stride);

/* Decode form (rope_at_pos_qk_kernel forward_gpu.cu:857-886 + the
 * kv_append_* kernels :104-277 in one launch): one row at position *d_pos,
 * separate q [Hq d], k, v [Hk d]; K quantised from its bf16 rounding. */
int granite4_rope_append_at_pos(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                const float* cos_tbl, const float* sin_tbl, int max_pos,
                                const int* d_pos, const int* d_pt, int Hq, int Hk, int d,
                                int bits, int group, uint16_t* q_rot, void* cache_k,
                                void* cache_v, float* k_scale, float* v_scale, int stride);

/* Host-side paged-pool index math (kv_pool.cc:285-297): out[p] =
 * block_table[p / page] * page + p % page for p < n. Pure host code. */
int granite4_row_table(const int32_t* block_table, int n, int page, int32_t* out);

/* Host-side self-test of the device FP8 / KV arithmetic: runs the exact
 * inline code the kernels use, on the CPU (no GPU needed). */
int granite4_host_fp8_encode(const float* y, size_t n, float scale, uint8_t* codes);
int granite4_host_kv_codes(const float* x, size_t n, float scale, int qmax, int32_t* codes);

/* Streaming bandwidth probe (kernels_bench.cu:36-53 pattern): mode 1 copies
 * `bytes` (multiple of 16) from src to dst, mode 0 only reads src (dst: a
 * 4-byte sink); modes 2 / 3 are the read / copy with non-temporal accesses,
 * 4 a copy with one vector per lane per iteration, 5 a non-temporal copy with
 * eight; `blocks` 256-thread workgroups in a grid-stride loop. */
int granite4_bw_probe(const void* src, void* dst, size_t bytes, int mode, int blocks);
/* The floor of a one-launch layer op (bench infrastructure, no reference
 * counterpart). mode 0: an empty kernel of `blocks` workgroups. mode 1: each
 * lane of `blocks` 256-thread workgroups loads its share of read_bytes (at
 * most 8 16-byte vectors per lane), then writes its share of write_bytes.
 * mode 2: as 1 with one grid synchronisation between the loads and the
 * stores (d_work: an FP8 workspace), the single-launch FP8 forms' structure.
 * blocks must not exceed the resident grid (at most 1024). */
int granite4_floor_probe(const void* src, size_t read_bytes, void* dst, size_t write_bytes,
                         void* d_work, int mode, int blocks);

/* Device self-tests of the hardware conversions the kernels use, against the
 * library's exact software arithmetic (the pattern of the reference's
 * granite4_fp8_decode_all probe, kernels_phase2.cu:844). d_result: two
 * zero-initialised device uint64 (mismatch count, first mismatching input
 * bits). _bf16 sweeps every non-NaN f32 through v_cvt_pk_bf16_f32; _fp8 every
 * f32 y in [0, 470 * scale] (and -y) through the FP8 pair encoder. */
int granite4_selftest_bf16(unsigned long long* d_result);
int granite4_selftest_fp8(float scale, unsigned long long* d_result);


/* ---------------------------------------------------------------------------
 * Split-KV decode attention over the paged KV pool (attention_split.cu,
 * attention_gpu.h:14-60).
 * ------------------------------------------------------------------------- */

/* Scratch bytes for `rows` query rows at cache stride `stride`
 * (attention_gpu.h:17 attn_split_scratch_bytes; the split layout follows
 * stride, or max_len when a call passes one). */
size_t granite4_attn_split_scratch_bytes(int Hq, int rows, int stride);

/* Where the split blocks' partials are combined (no counterpart in the
 * reference, which always launches attn_combine_kernel): 0 (the default)
 * inside the split launch, by the last block of each (row group, KV head) to
 * finish; 1 as a second launch. Both give identical outputs. The fused form
 * keeps arrival tags in the scratch that the combining block re-zeroes, so
 * a scratch buffer must not be shared by calls in flight at once (as for
 * the partials in either form). Process-wide; returns the previous mode, or
 * -1 for another value. */
int granite4_set_attn_combine_mode(int mode);

/* Status of the fused combine's bounded wait on one attention scratch buffer
 * (no counterpart in the reference, whose combine is always a second
 * launch): 0 if no combining block gave up waiting since the last clear (or
 * the zero fill of the scratch), 1 if one did; then that call's outputs are
 * NaN, and tags of late blocks may remain in the scratch, so zero-fill the
 * whole scratch before reusing it. clear != 0 resets the error word.
 * Synchronises the calling thread's stream; -1 on a null scratch or a HIP
 * error. The error word is the scratch's first 4 bytes, valid once the
 * scratch was zero-filled after allocation. */
int granite4_attn_sync_status(void* scratch, int clear);

/* The reference's attn_split (attention_gpu.h:53-60, bools as int). Causal
 * GQA for rows (1..16) query rows q [rows][Hq * d]: row r sits at position
 * p + r (p = *d_pos when d_pos is non-NULL, else kv_base; or row_pos[r] for
 * multi-sequence rows with their own tables row_pt[r]) and attends to
 * positions [0, p + r] (the last `window` of them when window > 0), read
 * through d_pt (position -> arena row; NULL = contiguous). Caches are
 * [Hk][stride][row bytes]: bf16 (cache_k / cache_v), int8 (cache_k8 /
 * cache_v8 with per-row scales, int8 = 1), int4 (cache_k4 / cache_v4,
 * int4 = 1) or K5 K + int4 V (k5 = 1). d = 128 and Hq = 4 Hk only; out is
 * [rows][Hq * d]. row_grp / ngroups (rows of one sequence sharing tiles) and
 * kv_hint only shape the reference's launch: results are identical without
 * them. Draft-tree rows (row_tbase / row_tail) are not supported: -1.
 * Arena rows outside [0, stride) are skipped (their keys are masked). */
int granite4_attn_split(const uint16_t* q, const uint16_t* cache_k, const uint16_t* cache_v,
                        float scale, int Hq, int Hk, int d, int kv_base, const int* d_pos,
                        int rows, int stride, void* scratch, uint16_t* out,
                        const int8_t* cache_k8, const int8_t* cache_v8,
                        const float* cache_k_scale, const float* cache_v_scale, int int8,
                        const uint8_t* cache_k4, const uint8_t* cache_v4, int int4,
                        const int* d_pt, int max_len, const int* row_pos,
                        const int* const* row_pt, const int* row_grp, int ngroups,
                        const int* row_tbase, const int* row_tail, int kv_hint, int k5,
                        int window);

/* Causal prefill attention over the pool (prefill_gemm.h:87-101
 * prefill_attention; bools as int): query rows q_rot [rows][Hq * d] at
 * positions [base_pos, base_pos + rows) attend to positions [0, position]
 * (the last `window` when window > 0) through d_pt (NULL: contiguous);
 * out [rows][Hq * d]. d = 128, Hq = 4 Hk only; stride >= base_pos + rows. */
int granite4_prefill_attention(const uint16_t* q_rot, const uint16_t* cache_k,
                               const uint16_t* cache_v, float scale, int Hq, int Hk, int d,
                               int base_pos, int rows, int stride, uint16_t* out,
                               const int8_t* cache_k8, const int8_t* cache_v8,
                               const float* k_scale, const float* v_scale, int int8,
                               const uint8_t* cache_k4, const uint8_t* cache_v4, int int4,
                               const int* d_pt, int k5, int window);

/* granite4_prefill_attention for every pool format of this library (bits 16
 * / 8 / 4 / 5, group 32 / 64 / 128 scales; groups of 32 / 64 read as
 * granite4_attn_paged reads them). New entry point. */
int granite4_prefill_attn(const uint16_t* q_rot, int rows, int Hq, int Hk, int d, float scale,
                          const void* cache_k, const void* cache_v, const float* k_scale,
                          const float* v_scale, int bits, int group, int stride, int base_pos,
                          const int* d_pt, int window, uint16_t* out);

/* The same attention for any pool format of this library, including the
 * group scales of granite4_rope_append: bits 16 / 8 / 4 / 5 (K5 K + int4 V),
 * group 32 / 64 / 128 (scales [Hk][stride][128 / group]; ignored for bf16).
 * New entry point (the reference's attention reads per-row scales only).
 * Group 128 keeps the reference's numerics (codes in the products, the row
 * scales on the dot and on p); groups of 32 / 64 are the bf16 attention over
 * the cache dequantised element by element, bf16(code * scale_g). */
int granite4_attn_paged(const uint16_t* q, int rows, int Hq, int Hk, int d, float scale,
                        const void* cache_k, const void* cache_v, const float* k_scale,
                        const float* v_scale, int bits, int group, int stride, int kv_base,
                        const int* d_pos, const int* d_pt, const int* row_pos,
                        const int* const* row_pt, int max_len, int window, void* scratch,
                        uint16_t* out);

/* ---------------------------------------------------------------------------
 * FP8 x FP8 GEMM with the layer epilogues fused in (gfx950 matrix cores).
 *
 * C[m][n] = a_scale * w_scale(n) * sum_k A[m][k] W[n][k]: A e4m3 codes [M][K]
 * (row pitch lda bytes, the FP8 output of granite4_add_rmsnorm_fp8 /
 * granite4_swiglu_fp8), a_scale its per-tensor scale read from device memory
 * (d_a_scale: the d_scale those ops write, so no host round trip and the
 * calls stay graph-capturable), W e4m3 [N][K] row-major.
 * The epilogue kinds and the per-segment weight scales are the reference's
 * GemmOut / GemmEpilogue (prefill_gemm.h:12-28, epi_store
 * prefill_gemm.cu:69-89); the reference's GEMM takes a bf16 A, this one the
 * FP8 activations of this library. y = acc * (a_scale * w_scale(n)) in f32.
 * Needs K % 128 == 0, lda >= K, lda % 16 == 0, N % 8 == 0, ldc >= N,
 * ldc % 8 == 0, and 16-byte aligned A, W and outputs (the reference needs
 * K % 32 == 0 and even N, prefill_gemm.cu:1263-1268; every Granite
 * projection meets both).
 * ------------------------------------------------------------------------- */
enum {
  GRANITE4_GEMM_BF16 = 0,     /* out_bf16[m][n] = bf16(y) */
  GRANITE4_GEMM_F32 = 1,      /* out_f32[m][n] = y */
  GRANITE4_GEMM_RESIDUAL = 2  /* out_bf16[m][n] = bf16(residual[m][n] + resid_scale * y) */
};

typedef struct Granite4GemmEpilogue {
  float scale0, scale1, scale2; /* w_scale(n): scale0 for n < seg1, scale1 for n < seg2, else scale2 */
  int seg1, seg2;
  uint16_t* out_bf16;
  float* out_f32;
  const uint16_t* residual;     /* may alias out_bf16 */
  float resid_scale;
  int ldc;                      /* output (and residual) row pitch, elements */
} Granite4GemmEpilogue;

/* Replaces: granite4::prefill_gemm (prefill_gemm.h:37-39) for FP8
 * activations; `out` is one of GRANITE4_GEMM_*. */
int granite4_gemm_fp8(int out, const uint8_t* A, int lda, const float* d_a_scale, const uint8_t* W,
                      int M, int N, int K, const Granite4GemmEpilogue* ep);

/* Replaces: granite4::prefill_gemm (prefill_gemm.h:34-39, prefill_gemm.cu:
 * 1260-1298), the reference's own form: C[m][n] = w_scale(n) * sum_k A[m][k]
 * W[n][k] with A bf16 [M][lda] and W e4m3 [N][K]; `out` one of
 * GRANITE4_GEMM_* (kBf16 / kF32 / kResidual, the reference's epi_store,
 * prefill_gemm.cu:69-89, y = w_scale(n) * acc in f32). The reference's
 * requirements: K % 32 == 0, lda % 8 == 0, lda >= K, even N and ldc,
 * ldc >= N, 16-byte aligned A and W (outputs whose pitch or width is not a
 * multiple of 8 are written element by element). ws / ws_bytes are accepted
 * and unused: the grid is persistent over 128 x 128 tiles, with no split-K
 * workspace. */
int granite4_prefill_gemm(int out, const uint16_t* A, int lda, const uint8_t* W, int M, int N,
                          int K, const Granite4GemmEpilogue* ep, float* ws, size_t ws_bytes);
/* prefill_gemm.h:42 (prefill_gemm_workspace_bytes): 0, no workspace is used. */
size_t granite4_prefill_gemm_workspace_bytes(int M, int N);

/* Replaces: the gate|up GEMM with the kF32 epilogue followed by
 * granite4::prefill_silu_mul (forward_gpu.cu:2837-2839, prefill_gemm.cu:
 * 1194-1203), fused: W_gu is [2I][K] (gate rows, then up rows), act[m][i] =
 * bf16(silu(g) * u) with g = acc_gate * (a_scale * gate_scale), u = acc_up *
 * (a_scale * up_scale); act [M][I] bf16 is always written. With codes != NULL
 * it is also quantised to FP8 e4m3 under the per-tensor scale amax / 448
 * (written to d_scale), exactly as granite4_swiglu_fp8 quantises its act.
 * d_work: the FP8 workspace (GRANITE4_FP8_WORK_BYTES(0) bytes at least). */
int granite4_gemm_fp8_swiglu(const uint8_t* A, int lda, const float* d_a_scale,
                             const uint8_t* W_gu, int M, int I, int K, float gate_scale,
                             float up_scale, uint16_t* act, uint8_t* codes, float* d_scale,
                             void* d_work);

/* Replaces: the O / down GEMM with the kResidual epilogue followed by the
 * next RMSNorm (forward_gpu.cu:2834-2836: prefill_gemm(kResidual) +
 * granite4_kernel_rmsnorm), with the norm's output FP8 for the next GEMM:
 * hidden[m][n] = bf16(hidden + resid_scale * acc * (a_scale * w_scale)) in
 * place, then codes / d_scale = the per-tensor FP8 RMSNorm of the updated
 * hidden (as granite4_add_rmsnorm_fp8 with no branch). H % 8 == 0. */
int granite4_gemm_fp8_residual_rmsnorm_fp8(const uint8_t* A, int lda, const float* d_a_scale,
                                           const uint8_t* W, int M, int H, int K, float w_scale,
                                           uint16_t* hidden, float resid_scale,
                                           const uint16_t* gamma, float eps, uint8_t* codes,
                                           float* d_scale, void* d_work);

/* ---------------------------------------------------------------------------
 * Batch-1 decode GEMVs (bf16 activation x fp8 e4m3 weight rows [N][K]) with
 * the decode step's non-GEMM ops fused in. y[n] = scale * sum_k fp8(W[n][k])
 * * a[k] in f32, as the reference's gemv_row_dequant (forward_gpu.cu:
 * 934-994). K % 64 == 0, K <= 16384, 16-byte aligned a and W.
 * ------------------------------------------------------------------------- */

/* Replaces: row_gemm_dequant_kernel launches (forward_gpu.cu:997-1002):
 * out[n] = bf16(y). */
int granite4_gemv_fp8w(const uint16_t* d_a, const uint8_t* d_w, float scale, int N, int K,
                       uint16_t* d_out);

/* Replaces: row_gemm_dequant_resid_kernel (forward_gpu.cu:1004-1013), the O /
 * down projection: out[n] = bf16(residual[n] + resid_scale * y); out may be
 * the residual (in place). */
int granite4_gemv_fp8w_resid(const uint16_t* d_a, const uint8_t* d_w, float scale,
                             const uint16_t* d_residual, float resid_scale, int N, int K,
                             uint16_t* d_out);

/* Replaces: row_gemm_dequant_qkv_kernel (forward_gpu.cu:1034-1057): the q, k,
 * v projections in one launch, each with its own weight, scale and output. */
int granite4_gemv_qkv(const uint16_t* d_a, const uint8_t* d_wq, const uint8_t* d_wk,
                      const uint8_t* d_wv, float sq, float sk, float sv, int Nq, int Nk, int Nv,
                      int K, uint16_t* d_q, uint16_t* d_k, uint16_t* d_v);

/* Replaces: granite4_kernel_rmsnorm (kernels_phase2.cu:910) followed by the
 * q / k / v GEMV (forward_gpu.cu:2115-2131): d_x is the residual row; every
 * workgroup computes bf16(x * r * gamma) itself (r from the double sum of
 * squares, as granite4_kernel_rmsnorm) and multiplies it. */
int granite4_gemv_rmsnorm_qkv(const uint16_t* d_x, const uint16_t* d_gamma, float eps,
                              const uint8_t* d_wq, const uint8_t* d_wk, const uint8_t* d_wv,
                              float sq, float sk, float sv, int Nq, int Nk, int Nv, int K,
                              uint16_t* d_q, uint16_t* d_k, uint16_t* d_v);

/* Replaces: granite4_kernel_silu_gate_up (kernels_phase2.cu:1217, the same
 * signature): act[i] = bf16(g * (1 / (1 + exp(-g))) * u), g = scale_g * (gate
 * row i . x), u = scale_u * (up row i . x). */
int granite4_kernel_silu_gate_up(const uint8_t* d_wg, const uint8_t* d_wu, const uint16_t* d_x,
                                 float scale_g, float scale_u, int N, int K, uint16_t* d_out);

/* Replaces: granite4_kernel_rmsnorm followed by granite4_kernel_silu_gate_up
 * (forward_gpu.cu:2227-2234): d_x is the residual row, normalised in every
 * workgroup as granite4_gemv_rmsnorm_qkv does. */
int granite4_gemv_rmsnorm_silu_gate_up(const uint16_t* d_x, const uint16_t* d_gamma, float eps,
                                       const uint8_t* d_wg, const uint8_t* d_wu, float scale_g,
                                       float scale_u, int N, int K, uint16_t* d_out);

/* Replaces: granite4_kernel_rmsnorm + the q / k / v GEMV + the RoPE and KV
 * append of the decode step (forward_gpu.cu:2115-2157), in one launch: the
 * residual row d_x (K = 4096) is normalised in every workgroup, the q|k|v
 * projections (Hq / Hk / Hk heads of 128 rows) are computed one head per
 * workgroup, and each head is rotated at *d_pos and written exactly as
 * granite4_rope_append_at_pos writes it (q_rot; K / V into the pool row
 * d_pt[*d_pos], quantised per bits / group). Outputs are bit-identical to
 * granite4_gemv_rmsnorm_qkv followed by granite4_rope_append_at_pos. */
int granite4_gemv_rmsnorm_qkv_rope_append(const uint16_t* d_x, const uint16_t* d_gamma,
                                          float eps, const uint8_t* d_wq, const uint8_t* d_wk,
                                          const uint8_t* d_wv, float sq, float sk, float sv,
                                          const float* cos_tbl, const float* sin_tbl, int max_pos,
                                          const int* d_pos, const int* d_pt, int Hq, int Hk,
                                          int bits, int group, uint16_t* q_rot, void* cache_k,
                                          void* cache_v, float* k_scale, float* v_scale,
                                          int stride);

/* Replaces: the decode step's RoPE + KV append (forward_gpu.cu:2132-2157)
 * followed by the split-KV attention (attention_split.cu:1083-1255), in the
 * attention launches: q / k / v are the raw bf16 projections of one token
 * at *d_pos; q is rotated in registers, and the workgroup whose split holds
 * the position rotates, quantises and writes that position's K / V row into
 * the pool (row d_pt[*d_pos]) before reading it. The pool and the output
 * are bit-identical to granite4_rope_append_at_pos followed by
 * granite4_attn_paged (rows = 1). scratch: granite4_attn_split_scratch_bytes
 * (Hq, 1, stride) bytes. */
int granite4_attn_decode_append(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                const float* cos_tbl, const float* sin_tbl, int max_pos,
                                const int* d_pos, const int* d_pt, int Hq, int Hk, float scale,
                                void* cache_k, void* cache_v, float* k_scale, float* v_scale,
                                int bits, int group, int stride, void* scratch, uint16_t* out);

/* Replaces: granite4_kernel_rmsnorm + the q / k / v GEMV + the RoPE of the
 * decode step (forward_gpu.cu:2115-2131, rope_at_pos_qk_kernel :857-886):
 * q_rot and k_rot are the q and k projections (Hq / Hk heads of 128 rows)
 * rotated at *d_pos, v the v projection; each rotation pair (dims i, i + 64)
 * is computed in one workgroup from the bf16 projections, with the append
 * kernels' products and roundings, so the outputs are bit-identical to the
 * GEMV followed by the rotation. A position outside [0, max_pos) leaves
 * q_rot and k_rot unwritten (as granite4_rope_append_at_pos leaves q_rot). */
int granite4_gemv_rmsnorm_qkv_rope(const uint16_t* d_x, const uint16_t* d_gamma, float eps,
                                   const uint8_t* d_wq, const uint8_t* d_wk, const uint8_t* d_wv,
                                   float sq, float sk, float sv, const float* cos_tbl,
                                   const float* sin_tbl, int max_pos, const int* d_pos, int Hq,
                                   int Hk, int K, uint16_t* d_q_rot, uint16_t* d_k_rot,
                                   uint16_t* d_v);
/* The same without the norm prologue: d_a is the GEMV input itself. */
int granite4_gemv_qkv_rope(const uint16_t* d_a, const uint8_t* d_wq, const uint8_t* d_wk,
                           const uint8_t* d_wv, float sq, float sk, float sv, const float* cos_tbl,
                           const float* sin_tbl, int max_pos, const int* d_pos, int Hq, int Hk,
                           int K, uint16_t* d_q_rot, uint16_t* d_k_rot, uint16_t* d_v);

/* Replaces: the decode step's embedding (forward_gpu.cu:2100, embed of the
 * token d_tokens[*d_pos]) + granite4_gemv_rmsnorm_qkv_rope of the first
 * layer, in one launch: x = bf16(emb_mult * emb[token]) (a zero row for a
 * token outside [0, vocab) or a negative position) is the GEMV's input row,
 * stored to d_hidden_out (the residual stream the step continues with).
 * Outputs bit-identical to granite4_embed_at_pos then
 * granite4_gemv_rmsnorm_qkv_rope. No reference counterpart as one call: it
 * saves the embedding's launch in the decode step. */
int granite4_gemv_embed_rmsnorm_qkv_rope(const int32_t* d_tokens, const uint16_t* d_emb,
                                         int vocab, float emb_mult, uint16_t* d_hidden_out,
                                         const uint16_t* d_gamma, float eps, const uint8_t* d_wq,
                                         const uint8_t* d_wk, const uint8_t* d_wv, float sq,
                                         float sk, float sv, const float* cos_tbl,
                                         const float* sin_tbl, int max_pos, const int* d_pos,
                                         int Hq, int Hk, int K, uint16_t* d_q_rot,
                                         uint16_t* d_k_rot, uint16_t* d_v);

/* Replaces: the KV append of the decode step (kv_append_*_kernel,
 * forward_gpu.cu:104-277) followed by granite4_attn_split (rows = 1), in one
 * attention launch, for q and k already rotated (granite4_gemv_rmsnorm_qkv_rope):
 * the split holding *d_pos quantises k_rot and v into that position's pool
 * row (the decode append's codes of the bf16 rotated K) and attends with it.
 * Bit-identical to granite4_kernel_kv_append*_batched at *d_pos then
 * granite4_attn_paged. A position outside [0, max_pos) writes V only, as the
 * append kernels do. scratch: granite4_attn_split_scratch_bytes(Hq, 1, stride). */
int granite4_attn_decode_append_rotated(const uint16_t* q_rot, const uint16_t* k_rot,
                                        const uint16_t* v, int max_pos, const int* d_pos,
                                        const int* d_pt, int Hq, int Hk, float scale,
                                        void* cache_k, void* cache_v, float* k_scale,
                                        float* v_scale, int bits, int group, int stride,
                                        void* scratch, uint16_t* out);

/* ---------------------------------------------------------------------------
 * The batch-1 decode step of the whole model (the reference's
 * forward_position, forward_gpu.cu:2066-2285, captured once by
 * capture_decode_graph :2934-2964 and replayed per token).
 * ------------------------------------------------------------------------- */

/* One layer's weights (fp8 e4m3 rows [N][K] with per-tensor scales, the
 * reference's LayerView and its sc[0..6]), RMSNorm gammas (bf16 [H]) and KV
 * arena (as granite4_attn_paged reads it; scales NULL for bits 16). */
typedef struct Granite4DecodeLayer {
  const uint16_t* attn_norm;
  const uint8_t* wq;  /* [Hq * 128][H] */
  const uint8_t* wk;  /* [Hk * 128][H] */
  const uint8_t* wv;  /* [Hk * 128][H] */
  const uint8_t* wo;  /* [H][Hq * 128] */
  const uint16_t* ffn_norm;
  const uint8_t* wg;  /* [I][H] */
  const uint8_t* wu;  /* [I][H] */
  const uint8_t* wd;  /* [H][I] */
  float sq, sk, sv, so, sg, su, sd;
  void* cache_k;
  void* cache_v;
  float* k_scale;
  float* v_scale;
} Granite4DecodeLayer;

/* The model: dimensions (head_dim 128, Hq a multiple of Hk), the multipliers
 * of the Granite config (embedding, residual, attention scale), eps, the
 * embedding table, a host array of `layers` layers, the optional final norm
 * and LM head, the RoPE tables and the KV format of every layer's arena
 * (bits 16 / 8 / 4 / 5, group, row stride). */
typedef struct Granite4DecodeModel {
  int layers, H, I, Hq, Hk, vocab;
  float eps, emb_mult, resid_mult, attn_scale;
  const uint16_t* emb;                /* [vocab][H] bf16 */
  const Granite4DecodeLayer* layer;   /* host array [layers] */
  const uint16_t* final_norm;         /* [H] or NULL */
  const uint8_t* lm_head;             /* [vocab][H] e4m3 or NULL */
  float lm_scale;
  const float* cos_tbl;
  const float* sin_tbl;
  int max_pos;
  int kv_bits, kv_group, kv_stride;
} Granite4DecodeModel;

/* Device scratch of the step, caller-owned: hidden [H] (the residual stream,
 * written from the embedding at the start of the step), q_rot [Hq * 128],
 * k_rot and v [Hk * 128], attn_out [Hq * 128], act [I], attn_scratch
 * granite4_attn_split_scratch_bytes(Hq, 1, kv_stride) bytes. */
typedef struct Granite4DecodeBuffers {
  uint16_t* hidden;
  uint16_t* q_rot;
  uint16_t* k_rot;
  uint16_t* v;
  uint16_t* attn_out;
  uint16_t* act;
  void* attn_scratch;
} Granite4DecodeBuffers;

/* Replaces: forward_position (forward_gpu.cu:2066-2285) for the split-KV
 * attention path. One token at position *d_pos (token d_tokens[*d_pos]):
 * embed, then per layer RMSNorm + q|k|v GEMV + RoPE (one launch), KV append
 * at arena row d_pt[*d_pos] (d_pt NULL: row = position) inside the split-KV
 * attention, O GEMV + residual, RMSNorm + gate/up GEMV + SwiGLU, down GEMV +
 * residual; then d_hidden_out = RMSNorm(hidden, final_norm) and d_logits =
 * bf16(lm_scale * lm_head . RMSNorm(hidden)) where given (NULL skips them).
 * 5 launches per layer + 0-2 (the embedding is the prologue of the first
 * layer's q|k|v launch, granite4_gemv_embed_rmsnorm_qkv_rope). Asynchronous
 * on the calling thread's stream,
 * no allocation: capturable once in a HIP graph and replayed per token with
 * *d_pos advanced between replays. Outputs are bit-identical to calling
 * granite4_embed_at_pos, granite4_gemv_rmsnorm_qkv_rope,
 * granite4_attn_decode_append_rotated, granite4_gemv_fp8w_resid,
 * granite4_gemv_rmsnorm_silu_gate_up, granite4_gemv_fp8w_resid,
 * granite4_kernel_rmsnorm and granite4_gemv_rmsnorm_qkv in that order. */
int granite4_decode_step(const Granite4DecodeModel* model, const Granite4DecodeBuffers* buffers,
                         const int32_t* d_tokens, const int* d_pos, const int* d_pt,
                         uint16_t* d_hidden_out, uint16_t* d_logits);

/* ---------------------------------------------------------------------------
 * Batched layer sequences: a prompt chunk (forward_prefill) and one decode
 * position of several sessions (forward_multi_step), over the model of
 * granite4_decode_step.
 * ------------------------------------------------------------------------- */

/* Activation forms of the batched sequences: the reference's bf16
 * activations (GEMMs with a bf16 A), or FP8 e4m3 activations with
 * per-tensor scales on the RMSNorm and SwiGLU outputs (this library's fused
 * RMSNorm -> FP8 and gate|up + SwiGLU -> FP8 ops and its FP8 GEMMs). */
#define GRANITE4_OPS_BF16 0
#define GRANITE4_OPS_FP8 1

/* Caller-owned device buffers for up to max_rows rows (max_rows <= 16 for
 * granite4_decode_step_multi): hidden, normed [max_rows][H]; qkv
 * [max_rows][(Hq + 2 Hk) 128]; q_rot, attn [max_rows][Hq 128]; act
 * [max_rows][I] (bf16). Bf16 form: gu f32 [max_rows][2I]. FP8 form: codes
 * [max_rows][H], act_codes [max_rows][I], scales f32 [2], fp8_work
 * GRANITE4_FP8_WORK_BYTES(max_rows) zero-filled once. The multi step:
 * attn_scratch granite4_attn_split_scratch_bytes(Hq, max_rows, kv_stride),
 * zero-filled once. Unused members may be NULL. */
typedef struct Granite4BatchBuffers {
  int max_rows;
  uint16_t* hidden;
  uint16_t* normed;
  uint16_t* qkv;
  uint16_t* q_rot;
  uint16_t* attn;
  uint16_t* act;
  float* gu;
  uint8_t* codes;
  uint8_t* act_codes;
  float* scales;
  void* fp8_work;
  void* attn_scratch;
} Granite4BatchBuffers;

/* Replaces: forward_prefill (forward_gpu.cu:2751-2863) for one chunk:
 * positions start .. start + rows - 1 of one sequence (tokens
 * d_tokens[start ..], bounds-checked as granite4_embed_rows), every layer's
 * K / V appended to its arena through the row table d_pt (NULL: row =
 * position), causal attention over the pool (granite4_prefill_attn), then
 * d_hidden_out = RMSNorm(hidden, final_norm) [rows][H] and d_logits =
 * bf16(lm_scale * lm_head . that) [rows][vocab] where given. ops: one of
 * GRANITE4_OPS_*. The FP8 form needs the gate and up weights as one
 * [2I][H] block (wu == wg + I * H). Per layer: 9 launches (bf16; 10 when
 * q, k and v are not one [nqkv][H] block) or 8 (FP8). Asynchronous, no
 * allocation; -1 before any launch on invalid arguments. No reference
 * counterpart as one exported call (the reference's is internal). */
int granite4_prefill_layers(const Granite4DecodeModel* model, const Granite4BatchBuffers* buffers,
                            const int32_t* d_tokens, int start, int rows, const int* d_pt,
                            int ops, uint16_t* d_hidden_out, uint16_t* d_logits);

/* Replaces: forward_multi_step (forward_gpu.cu:2486-2623) up to the logits:
 * one decode position for each of `rows` (<= 16) sessions of the device
 * descriptor d_rows (row r: position pos[r], token tok[r][pos[r]], page
 * table pt[r]; draft-tree descriptors, tree != 0, are not supported).
 * Embedding (granite4_multi_embed), then per layer: RMSNorm, q / k / v
 * GEMMs, RoPE + the KV append of every row (granite4_multi_rope_append),
 * the split-KV attention of the rows at their own positions and page tables
 * (granite4_attn_paged with row_pos / row_pt), O + residual, RMSNorm, gate /
 * up + SwiGLU, down + residual; then the optional final norm and logits.
 * ops: one of GRANITE4_OPS_*. The KV format must have per-row scales (group
 * 128) or be bf16. Sampling and advancing the positions are the caller's
 * (the reference's argmax_rows_kernel and multi_scatter_advance_kernel).
 * Asynchronous, no allocation, graph-capturable; -1 before any launch on
 * invalid arguments. */
int granite4_decode_step_multi(const Granite4DecodeModel* model,
                               const Granite4BatchBuffers* buffers, const GpuMultiRows* d_rows,
                               int rows, int ops, uint16_t* d_hidden_out, uint16_t* d_logits);

#ifdef __cplusplus
}  /* extern "C" */

/* The reference's C++ launcher names (prefill_gemm.h:41-105,
 * forward_gpu_api.h:219-229), forwarding to the C entry points above. */
namespace granite4 {
// prefill_gemm.h:12-39: the reference's GemmOut / GemmEpilogue (same fields
// and defaults) and prefill_gemm, over granite4_prefill_gemm.
enum class GemmOut { kBf16 = GRANITE4_GEMM_BF16, kF32 = GRANITE4_GEMM_F32,
                     kResidual = GRANITE4_GEMM_RESIDUAL };
struct GemmEpilogue {
  float scale0 = 1.0f, scale1 = 1.0f, scale2 = 1.0f;
  int seg1 = INT32_MAX, seg2 = INT32_MAX;
  uint16_t* out_bf16 = nullptr;
  float* out_f32 = nullptr;
  const uint16_t* residual = nullptr;
  float resid_scale = 1.0f;
  int ldc = 0;
};
inline int prefill_gemm(GemmOut out, const uint16_t* A, int lda, const uint8_t* W, int M, int N,
                        int K, const GemmEpilogue& ep, float* ws = nullptr,
                        size_t ws_bytes = 0) {
  const Granite4GemmEpilogue e{ep.scale0, ep.scale1, ep.scale2, ep.seg1, ep.seg2, ep.out_bf16,
                               ep.out_f32, ep.residual, ep.resid_scale, ep.ldc};
  return granite4_prefill_gemm(static_cast<int>(out), A, lda, W, M, N, K, &e, ws, ws_bytes);
}
inline size_t prefill_gemm_workspace_bytes(int M, int N) {
  return granite4_prefill_gemm_workspace_bytes(M, N);
}
inline int prefill_embed_rows(const int32_t* d_tokens, int start, int rows, const uint16_t* emb,
                              float mult, uint16_t* out, int H) {
  return granite4_prefill_embed_rows(d_tokens, start, rows, emb, mult, out, H);
}
inline int prefill_rope_split_append(const uint16_t* qkv, const float* c, const float* s,
                                     int base_pos, int rows, int Hq, int Hk, int d, int stride,
                                     uint16_t* q_rot, uint16_t* ck, uint16_t* cv,
                                     const int* d_pt = nullptr) {
  return granite4_prefill_rope_split_append(qkv, c, s, base_pos, rows, Hq, Hk, d, stride, q_rot,
                                            ck, cv, d_pt);
}
inline int prefill_rope_split_append_int8(const uint16_t* qkv, const float* c, const float* s,
                                          int base_pos, int rows, int Hq, int Hk, int d,
                                          int stride, uint16_t* q_rot, int8_t* ck, int8_t* cv,
                                          float* ks, float* vs, const int* d_pt = nullptr) {
  return granite4_prefill_rope_split_append_int8(qkv, c, s, base_pos, rows, Hq, Hk, d, stride,
                                                 q_rot, ck, cv, ks, vs, d_pt);
}
inline int prefill_rope_split_append_int4(const uint16_t* qkv, const float* c, const float* s,
                                          int base_pos, int rows, int Hq, int Hk, int d,
                                          int stride, uint16_t* q_rot, uint8_t* ck, uint8_t* cv,
                                          float* ks, float* vs, const int* d_pt = nullptr) {
  return granite4_prefill_rope_split_append_int4(qkv, c, s, base_pos, rows, Hq, Hk, d, stride,
                                                 q_rot, ck, cv, ks, vs, d_pt);
}
inline int prefill_rope_split_append_k5v4(const uint16_t* qkv, const float* c, const float* s,
                                          int base_pos, int rows, int Hq, int Hk, int d,
                                          int stride, uint16_t* q_rot, uint8_t* ck, uint8_t* cv,
                                          float* ks, float* vs, const int* d_pt = nullptr) {
  return granite4_prefill_rope_split_append_k5v4(qkv, c, s, base_pos, rows, Hq, Hk, d, stride,
                                                 q_rot, ck, cv, ks, vs, d_pt);
}
inline int prefill_silu_mul(const float* gu, int I, int rows, uint16_t* act) {
  return granite4_prefill_silu_mul(gu, I, rows, act);
}
inline int gpu_multi_rope(const uint16_t* x, const float* c, const float* s,
                          const GpuMultiRows* d_rows, int rows, int heads, int d, uint16_t* out) {
  return granite4_multi_rope(x, c, s, d_rows, rows, heads, d, out);
}
inline int gpu_multi_rope_append(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                 const float* c, const float* s, const GpuMultiRows* d_rows,
                                 int rows, int Hq, int Hk, int d, int bits, void* ck, void* cv,
                                 float* ks, float* vs, int stride, uint16_t* q_rot) {
  return granite4_multi_rope_append(q, k, v, c, s, d_rows, rows, Hq, Hk, d, bits, ck, cv, ks, vs,
                                    stride, q_rot);
}
inline int gpu_multi_kv_append(const uint16_t* k, const uint16_t* v, int bits, void* ck,
                               void* cv, float* ks, float* vs, const GpuMultiRows* d_rows,
                               int rows, int stride, int Hk, int d) {
  return granite4_multi_kv_append(k, v, bits, ck, cv, ks, vs, d_rows, rows, stride, Hk, d);
}

// prefill_gemm.h:94-101 (bool flags, default arguments).
inline int prefill_attention(const uint16_t* q_rot, const uint16_t* cache_k,
                             const uint16_t* cache_v, float scale, int Hq, int Hk, int d,
                             int base_pos, int rows, int stride, uint16_t* out,
                             const int8_t* cache_k8, const int8_t* cache_v8, const float* k_scale,
                             const float* v_scale, bool int8, const uint8_t* cache_k4,
                             const uint8_t* cache_v4, bool int4, const int* d_pt = nullptr,
                             bool k5 = false, int window = 0) {
  return granite4_prefill_attention(q_rot, cache_k, cache_v, scale, Hq, Hk, d, base_pos, rows,
                                    stride, out, cache_k8, cache_v8, k_scale, v_scale, int8,
                                    cache_k4, cache_v4, int4, d_pt, k5, window);
}
// attention_gpu.h:17, 53-60 (bool flags, default arguments).
inline size_t attn_split_scratch_bytes(int Hq, int rows, int stride) {
  return granite4_attn_split_scratch_bytes(Hq, rows, stride);
}
inline int attn_split(const uint16_t* q, const uint16_t* cache_k, const uint16_t* cache_v,
                      float scale, int Hq, int Hk, int d, int kv_base, const int* d_pos, int rows,
                      int stride, void* scratch, uint16_t* out, const int8_t* cache_k8 = nullptr,
                      const int8_t* cache_v8 = nullptr, const float* cache_k_scale = nullptr,
                      const float* cache_v_scale = nullptr, bool int8 = false,
                      const uint8_t* cache_k4 = nullptr, const uint8_t* cache_v4 = nullptr,
                      bool int4 = false, const int* d_pt = nullptr, int max_len = 0,
                      const int* row_pos = nullptr, const int* const* row_pt = nullptr,
                      const int* row_grp = nullptr, int ngroups = 0,
                      const int* row_tbase = nullptr, const int* row_tail = nullptr,
                      int kv_hint = 0, bool k5 = false, int window = 0) {
  return granite4_attn_split(q, cache_k, cache_v, scale, Hq, Hk, d, kv_base, d_pos, rows, stride,
                             scratch, out, cache_k8, cache_v8, cache_k_scale, cache_v_scale, int8,
                             cache_k4, cache_v4, int4, d_pt, max_len, row_pos, row_pt, row_grp,
                             ngroups, row_tbase, row_tail, kv_hint, k5, window);
}
}  // namespace granite4
#endif /* __cplusplus */

#endif /* GRANITE4_LAYEROPS_H */
