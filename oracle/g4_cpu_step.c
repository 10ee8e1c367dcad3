/*
 * g4_cpu_step.c - the CPU baseline of bench.py: the T-token one-layer step of
 * BASELINE config 3 (embedding gather from the full [100352][4096] table,
 * add+RMSNorm with FP8 output, SwiGLU with FP8 output, RoPE with the int8
 * paged-KV write) run with the scalar oracle (g4_oracle.c) on host threads.
 *
 * TEST INFRASTRUCTURE ONLY (bench.py's cpu_baseline leg). It times the
 * oracle; it is not the product and the product never calls it.
 *
 * Threads split the step by token rows, as the GPU kernels do: phase A runs
 * embed, add+RMSNorm (bf16 normed), SwiGLU (bf16 act) and RoPE + int8 KV on
 * each thread's rows and takes the slice's max |normed| and max |act|; after a
 * barrier every thread takes the per-tensor FP8 scales (gpu_pack.cc:44-46)
 * from the slice maxima and, in phase B, encodes its rows
 * (gpu_pack.cc:48-51). Every buffer is allocated and filled before the timed
 * loop, so the timing holds only the step's arithmetic and memory traffic.
 */
#define _GNU_SOURCE
#include "g4_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

enum { kH = 4096, kI = 12800, kHq = 32, kHk = 8, kD = 128, kVocab = 100352, kMaxThreads = 256 };

typedef struct {
  int T, threads;
  double seconds;
  int32_t* tok;
  uint16_t *emb, *emb_out, *res, *br, *w, *res_out, *normed, *gu, *act, *qkv, *q_rot;
  uint8_t *codes_h, *codes_i, *cache_k, *cache_v;
  float *k_scale, *v_scale, *cos_t, *sin_t;
  int *pos;
  float amax_n[kMaxThreads], amax_a[kMaxThreads];
  pthread_barrier_t bar;
  volatile int stop;
  int steps;
  double wall;
} Step;

typedef struct {
  Step* s;
  int t;
} Arg;

static double now_s(void) {
  struct timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return ts.tv_sec + ts.tv_nsec * 1e-9;
}

static float amax_bf16(const uint16_t* x, size_t n) {
  float m = 0.0f;
  for (size_t i = 0; i < n; ++i) {
    const float v = fabsf(g4o_bf16_to_f32(x[i]));
    if (v > m) m = v;
  }
  return m;
}

static void* worker(void* p) {
  Arg* a = (Arg*)p;
  Step* s = a->s;
  const int t = a->t, T = s->T;
  const int r0 = (int)((long long)T * t / s->threads), r1 = (int)((long long)T * (t + 1) / s->threads);
  const int n = r1 - r0;
  const int qkv_w = (kHq + 2 * kHk) * kD;
  double t0 = 0.0;
  for (int step = 0;; ++step) {
    pthread_barrier_wait(&s->bar);
    if (t == 0 && step == 0) t0 = now_s();
    if (s->stop) break;
    if (n > 0) {
      g4o_embed_rows(s->tok + r0, n, s->emb, kH, 1.0f, s->emb_out + (size_t)r0 * kH);
      g4o_add_rmsnorm(s->res + (size_t)r0 * kH, s->br + (size_t)r0 * kH, 1.0f, s->w, 1e-5f, n, kH,
                      s->res_out + (size_t)r0 * kH, s->normed + (size_t)r0 * kH);
      s->amax_n[t] = amax_bf16(s->normed + (size_t)r0 * kH, (size_t)n * kH);
      g4o_swiglu_bf16(s->gu + (size_t)r0 * 2 * kI, n, kI, s->act + (size_t)r0 * kI);
      s->amax_a[t] = amax_bf16(s->act + (size_t)r0 * kI, (size_t)n * kI);
      const uint16_t* q = s->qkv + (size_t)r0 * qkv_w;
      g4o_rope_append(q, qkv_w, q + kHq * kD, qkv_w, q + (kHq + kHk) * kD, qkv_w, s->cos_t,
                      s->sin_t, n, kHq, kHk, kD, s->pos + r0, s->pos + r0, 8, kD, 1, 0,
                      s->q_rot + (size_t)r0 * kHq * kD, kHq * kD, s->cache_k, s->cache_v,
                      s->k_scale, s->v_scale, T);
    } else {
      s->amax_n[t] = 0.0f;
      s->amax_a[t] = 0.0f;
    }
    pthread_barrier_wait(&s->bar);
    float mn = 0.0f, ma = 0.0f;
    for (int i = 0; i < s->threads; ++i) {
      if (s->amax_n[i] > mn) mn = s->amax_n[i];
      if (s->amax_a[i] > ma) ma = s->amax_a[i];
    }
    if (n > 0) {
      g4o_fp8_encode_scaled_bf16(s->normed + (size_t)r0 * kH, (size_t)n * kH,
                                 g4o_fp8_scale_for(mn), s->codes_h + (size_t)r0 * kH);
      g4o_fp8_encode_scaled_bf16(s->act + (size_t)r0 * kI, (size_t)n * kI, g4o_fp8_scale_for(ma),
                                 s->codes_i + (size_t)r0 * kI);
    }
    pthread_barrier_wait(&s->bar);
    if (t == 0) {
      s->steps = step + 1;
      s->wall = now_s() - t0;
      if (s->wall >= s->seconds) s->stop = 1;
    }
  }
  return NULL;
}

static void* xmalloc(size_t n) { return n ? malloc(n) : NULL; }

/* Runs the T-token step on `threads` threads until about `seconds` of wall
 * time have passed (at least one step). Returns the steps done (writing the
 * wall seconds of those steps to *wall_s), or -1 on bad arguments or memory. */
int g4o_cpu_step_bench(int T, int threads, double seconds, double* wall_s) {
  if (T <= 0 || threads <= 0 || threads > kMaxThreads || seconds < 0.0 || wall_s == NULL) return -1;
  Step* s = calloc(1, sizeof(Step));
  if (s == NULL) return -1;
  s->T = T;
  s->threads = threads;
  s->seconds = seconds;
  const size_t qkv_w = (kHq + 2 * kHk) * kD;
  s->tok = xmalloc(sizeof(int32_t) * T);
  s->pos = xmalloc(sizeof(int) * T);
  s->emb = xmalloc(sizeof(uint16_t) * (size_t)kVocab * kH);
  s->emb_out = xmalloc(sizeof(uint16_t) * (size_t)T * kH);
  s->res = xmalloc(sizeof(uint16_t) * (size_t)T * kH);
  s->br = xmalloc(sizeof(uint16_t) * (size_t)T * kH);
  s->w = xmalloc(sizeof(uint16_t) * kH);
  s->res_out = xmalloc(sizeof(uint16_t) * (size_t)T * kH);
  s->normed = xmalloc(sizeof(uint16_t) * (size_t)T * kH);
  s->gu = xmalloc(sizeof(uint16_t) * (size_t)T * 2 * kI);
  s->act = xmalloc(sizeof(uint16_t) * (size_t)T * kI);
  s->qkv = xmalloc(sizeof(uint16_t) * (size_t)T * qkv_w);
  s->q_rot = xmalloc(sizeof(uint16_t) * (size_t)T * kHq * kD);
  s->codes_h = xmalloc((size_t)T * kH);
  s->codes_i = xmalloc((size_t)T * kI);
  s->cache_k = xmalloc((size_t)kHk * T * kD);
  s->cache_v = xmalloc((size_t)kHk * T * kD);
  s->k_scale = xmalloc(sizeof(float) * (size_t)kHk * T);
  s->v_scale = xmalloc(sizeof(float) * (size_t)kHk * T);
  s->cos_t = xmalloc(sizeof(float) * (size_t)T * kD / 2);
  s->sin_t = xmalloc(sizeof(float) * (size_t)T * kD / 2);
  int rc = -1;
  if (!s->tok || !s->pos || !s->emb || !s->emb_out || !s->res || !s->br || !s->w || !s->res_out ||
      !s->normed || !s->gu || !s->act || !s->qkv || !s->q_rot || !s->codes_h || !s->codes_i ||
      !s->cache_k || !s->cache_v || !s->k_scale || !s->v_scale || !s->cos_t || !s->sin_t)
    goto done;
  uint32_t* u = (uint32_t*)s->tok;
  g4o_fill_u32(0x5EED, T, u);
  for (int i = 0; i < T; ++i) {
    s->tok[i] = (int32_t)(u[i] % kVocab);
    s->pos[i] = i;
  }
  g4o_fill_uniform_bf16(0x5EED1, 0.04, (size_t)kVocab * kH, s->emb);
  g4o_fill_normal_bf16(0x5EED2, 0.0, 1.0, (size_t)T * kH, s->res);
  g4o_fill_normal_bf16(0x5EED3, 0.0, 1.0, (size_t)T * kH, s->br);
  g4o_fill_normal_bf16(0x5EED4, 1.0, 0.1, kH, s->w);
  g4o_fill_normal_bf16(0x5EED5, 0.0, 1.0, (size_t)T * 2 * kI, s->gu);
  g4o_fill_normal_bf16(0x5EED6, 0.0, 1.0, (size_t)T * qkv_w, s->qkv);
  g4o_rope_tables(1e7, kD, T, s->cos_t, s->sin_t);
  pthread_t th[kMaxThreads];
  Arg args[kMaxThreads];
  pthread_barrier_init(&s->bar, NULL, (unsigned)threads);
  int started = 0;
  for (int t = 0; t < threads; ++t) {
    args[t].s = s;
    args[t].t = t;
    if (pthread_create(&th[t], NULL, worker, &args[t]) != 0) break;
    ++started;
  }
  if (started != threads) {
    /* the barrier can never be passed: abandon without joining */
    goto done;
  }
  for (int t = 0; t < threads; ++t) pthread_join(th[t], NULL);
  pthread_barrier_destroy(&s->bar);
  *wall_s = s->wall;
  rc = s->steps;
done:
  free(s->tok); free(s->pos); free(s->emb); free(s->emb_out); free(s->res); free(s->br);
  free(s->w); free(s->res_out); free(s->normed); free(s->gu); free(s->act); free(s->qkv);
  free(s->q_rot); free(s->codes_h); free(s->codes_i); free(s->cache_k); free(s->cache_v);
  free(s->k_scale); free(s->v_scale); free(s->cos_t); free(s->sin_t);
  if (rc >= 0) free(s);
  return rc;
}
