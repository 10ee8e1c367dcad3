// layer_steps.hip - the engine's batched layer sequences as single C ABI
// calls, built from this library's entry points:
//
//   granite4_prefill_layers     forward_prefill (forward_gpu.cu:2751-2863) for
//                               one chunk of a sequence's prompt;
//   granite4_decode_step_multi  forward_multi_step (forward_gpu.cu:2486-2623):
//                               one decode position of up to 16 independent
//                               sessions (GpuMultiRows).
//
// Per layer (rows = the chunk's tokens or the sessions):
//   normed = RMSNorm(hidden)                          kernel_rmsnorm
//   q|k|v  = GEMM(normed, Wq|Wk|Wv)                   prefill_gemm, bf16 out
//   q_rot, KV append of RoPE(k), v                    rope_append / multi_rope_append
//   attn   = causal attention over the pool           prefill_attn / attn_paged (row_pos)
//   hidden = bf16(hidden + rs * GEMM(attn, Wo))       prefill_gemm, kResidual
//   normed = RMSNorm(hidden)                          kernel_rmsnorm
//   act    = SwiGLU(GEMM(normed, Wg|Wu))              prefill_gemm kF32 + prefill_silu_mul
//   hidden = bf16(hidden + rs * GEMM(act, Wd))        prefill_gemm, kResidual
// which is the reference's order with its bf16 activations (mode
// GRANITE4_OPS_BF16), or, with FP8 activations (GRANITE4_OPS_FP8, BASELINE
// config 2's per-tensor scales on the RMSNorm and SwiGLU outputs):
//   codes, s = RMSNorm -> FP8                         add_rmsnorm_fp8
//   q|k|v  = GEMM_fp8(codes, s, Wq|Wk|Wv)             gemm_fp8, bf16 out
//   ... RoPE + append, attention, O + residual as above ...
//   codes, s = RMSNorm -> FP8                         add_rmsnorm_fp8
//   act codes, s' = SwiGLU(GEMM_fp8(codes, Wg|Wu)) -> FP8   gemm_fp8_swiglu
//   hidden = bf16(hidden + rs * GEMM_fp8(act codes, s', Wd)) gemm_fp8, kResidual
// Every launch is one of the library's entry points on the calling thread's
// stream, so a step equals those calls one by one. Nothing is allocated and
// nothing synchronises: the calls can be captured in a HIP graph. Every
// argument is checked before the first launch, so a call either launches
// nothing (-1) or the whole sequence.
#include "g4_common.h"
#include "granite4_layerops.h"

#include <cmath>
#include <cstddef>
#include <cstdint>
#include <cstdio>

namespace g4 {
// gemm.hip: the skinny GEMM (rows <= 16) with a bf16 output per row segment.
int gemm_rows_split(bool fp8, const void* A, int lda, const float* a_scale, const uint8_t* W,
                    int M, int N, int K, const Granite4GemmEpilogue& ep, uint16_t* const out[3],
                    const int ld[3]);
}  // namespace g4

namespace {

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool fin(float x) { return std::isfinite(x); }

// The GEMM shape rules of both GEMM entry points: K % 128 (FP8) and
// N % 8 for every projection.
bool dims_ok(const Granite4DecodeModel* m) {
  return m != nullptr && m->layers > 0 && m->layer != nullptr && m->Hk > 0 &&
         m->Hq == 4 * m->Hk && m->H > 0 && m->H % 128 == 0 && m->I > 0 && m->I % 128 == 0 &&
         m->emb != nullptr && al16(m->emb) && m->vocab > 0 && m->cos_tbl != nullptr &&
         m->sin_tbl != nullptr && m->max_pos > 0 && m->kv_stride > 0 && fin(m->eps) &&
         fin(m->emb_mult) && fin(m->resid_mult) && fin(m->attn_scale) && fin(m->lm_scale) &&
         (m->kv_bits == 16 || m->kv_bits == 8 || m->kv_bits == 4 || m->kv_bits == 5) &&
         (m->kv_bits == 16 || m->kv_group == 32 || m->kv_group == 64 || m->kv_group == 128) &&
         (m->lm_head == nullptr || (m->final_norm != nullptr && al16(m->lm_head))) &&
         (m->final_norm == nullptr || al16(m->final_norm));
}

bool layers_ok(const Granite4DecodeModel* m, int fp8) {
  for (int l = 0; l < m->layers; ++l) {
    const Granite4DecodeLayer& y = m->layer[l];
    const void* ptrs[] = {y.attn_norm, y.ffn_norm, y.wq, y.wk, y.wv, y.wo, y.wg, y.wu, y.wd};
    for (const void* p : ptrs)
      if (p == nullptr || !al16(p)) return false;
    if (y.cache_k == nullptr || y.cache_v == nullptr ||
        (m->kv_bits != 16 && (y.k_scale == nullptr || y.v_scale == nullptr)))
      return false;
    const float sc[] = {y.sq, y.sk, y.sv, y.so, y.sg, y.su, y.sd};
    for (float x : sc)
      if (!fin(x)) return false;
    // The fused gate|up GEMM of the FP8 form reads one [2I][H] matrix.
    if (fp8 && y.wu != y.wg + static_cast<size_t>(m->I) * m->H) return false;
  }
  return true;
}

bool buffers_ok(const Granite4BatchBuffers* b, const Granite4DecodeModel* m, int rows, int fp8) {
  if (b == nullptr || rows < 1 || rows > b->max_rows) return false;
  const void* ptrs[] = {b->hidden, b->normed, b->qkv, b->q_rot, b->attn, b->act};
  for (const void* p : ptrs)
    if (p == nullptr || !al16(p)) return false;
  if (fp8) {
    if (b->codes == nullptr || b->act_codes == nullptr || b->scales == nullptr ||
        b->fp8_work == nullptr || !al16(b->codes) || !al16(b->act_codes))
      return false;
  } else if (b->gu == nullptr || !al16(b->gu)) {
    return false;
  }
  (void)m;
  return true;
}

Granite4GemmEpilogue epi_bf16(float s0, float s1, float s2, int seg1, int seg2, uint16_t* out,
                              int ldc) {
  Granite4GemmEpilogue e{};
  e.scale0 = s0;
  e.scale1 = s1;
  e.scale2 = s2;
  e.seg1 = seg1;
  e.seg2 = seg2;
  e.out_bf16 = out;
  e.ldc = ldc;
  e.resid_scale = 1.0f;
  return e;
}

Granite4GemmEpilogue epi_resid(float s, uint16_t* hidden, float rs, int ldc) {
  Granite4GemmEpilogue e = epi_bf16(s, s, s, INT32_MAX, INT32_MAX, hidden, ldc);
  e.residual = hidden;
  e.resid_scale = rs;
  return e;
}

constexpr int kSkinnyRows = 16;

// q|k|v of `rows` rows into [rows][ldq] (q at column 0, k at nq, v at
// nq + nk) or into three buffers (q_out / k_out / v_out with their own
// pitches); one GEMM when the three weight matrices are one [nqkv][H] block.
int qkv_gemm(const Granite4DecodeModel* m, const Granite4DecodeLayer& y,
             const Granite4BatchBuffers* b, int rows, int fp8, uint16_t* q_out, int ldq,
             uint16_t* k_out, int ldk, uint16_t* v_out, int ldv) {
  const int H = m->H, nq = m->Hq * 128, nk = m->Hk * 128;
  const bool one = y.wk == y.wq + static_cast<size_t>(nq) * H &&
                   y.wv == y.wk + static_cast<size_t>(nk) * H && k_out == q_out + nq &&
                   v_out == k_out + nk && ldk == ldq && ldv == ldq;
  const auto gemm = [&](const uint8_t* W, int N, const Granite4GemmEpilogue& e) {
    return fp8 ? granite4_gemm_fp8(GRANITE4_GEMM_BF16, b->codes, H, b->scales, W, rows, N, H, &e)
               : granite4_prefill_gemm(GRANITE4_GEMM_BF16, b->normed, H, W, rows, N, H, &e,
                                       nullptr, 0);
  };
  if (one) {
    const Granite4GemmEpilogue e = epi_bf16(y.sq, y.sk, y.sv, nq, nq + nk, q_out, ldq);
    return gemm(y.wq, nq + 2 * nk, e);
  }
  const bool contiguous_w = y.wk == y.wq + static_cast<size_t>(nq) * H &&
                            y.wv == y.wk + static_cast<size_t>(nk) * H;
  if (contiguous_w && rows <= kSkinnyRows) {
    // one launch, three output buffers
    const Granite4GemmEpilogue e = epi_bf16(y.sq, y.sk, y.sv, nq, nq + nk, q_out, ldq);
    uint16_t* const outs[3] = {q_out, k_out, v_out};
    const int lds[3] = {ldq, ldk, ldv};
    return fp8 ? g4::gemm_rows_split(true, b->codes, H, b->scales, y.wq, rows, nq + 2 * nk, H, e, outs, lds)
               : g4::gemm_rows_split(false, b->normed, H, nullptr, y.wq, rows, nq + 2 * nk, H, e, outs,
                                 lds);
  }
  const Granite4GemmEpilogue eq = epi_bf16(y.sq, y.sq, y.sq, INT32_MAX, INT32_MAX, q_out, ldq);
  const Granite4GemmEpilogue ek = epi_bf16(y.sk, y.sk, y.sk, INT32_MAX, INT32_MAX, k_out, ldk);
  const Granite4GemmEpilogue ev = epi_bf16(y.sv, y.sv, y.sv, INT32_MAX, INT32_MAX, v_out, ldv);
  return (gemm(y.wq, nq, eq) != 0 || gemm(y.wk, nk, ek) != 0 || gemm(y.wv, nk, ev) != 0) ? -1 : 0;
}

// The layer's input norm (into b->normed, or FP8 codes + scale 0).
int norm_in(const Granite4DecodeModel* m, const Granite4BatchBuffers* b, const uint16_t* gamma,
            int rows, int fp8) {
  return fp8 ? granite4_add_rmsnorm_fp8(b->hidden, nullptr, 1.0f, gamma, m->eps, rows, m->H,
                                        nullptr, b->codes, b->scales, b->fp8_work)
             : granite4_kernel_rmsnorm(b->hidden, gamma, m->eps, rows, m->H, b->normed);
}

// O + residual, then the MLP: norm, gate|up + SwiGLU, down + residual.
int layer_tail(const Granite4DecodeModel* m, const Granite4DecodeLayer& y,
               const Granite4BatchBuffers* b, int rows, int fp8) {
  const int H = m->H, I = m->I, nq = m->Hq * 128;
  const Granite4GemmEpilogue eo = epi_resid(y.so, b->hidden, m->resid_mult, H);
  if (granite4_prefill_gemm(GRANITE4_GEMM_RESIDUAL, b->attn, nq, y.wo, rows, H, nq, &eo, nullptr,
                            0) != 0 ||
      norm_in(m, b, y.ffn_norm, rows, fp8) != 0)
    return -1;
  const Granite4GemmEpilogue ed = epi_resid(y.sd, b->hidden, m->resid_mult, H);
  if (fp8) {
    return (granite4_gemm_fp8_swiglu(b->codes, H, b->scales, y.wg, rows, I, H, y.sg, y.su, b->act,
                                     b->act_codes, b->scales + 1, b->fp8_work) != 0 ||
            granite4_gemm_fp8(GRANITE4_GEMM_RESIDUAL, b->act_codes, I, b->scales + 1, y.wd, rows,
                              H, I, &ed) != 0)
               ? -1
               : 0;
  }
  Granite4GemmEpilogue eg{};
  eg.scale0 = eg.scale1 = eg.scale2 = y.sg;
  eg.seg1 = eg.seg2 = INT32_MAX;
  eg.out_f32 = b->gu;
  eg.ldc = 2 * I;
  eg.resid_scale = 1.0f;
  Granite4GemmEpilogue eu = eg;
  eu.scale0 = eu.scale1 = eu.scale2 = y.su;
  eu.out_f32 = b->gu + I;
  return (granite4_prefill_gemm(GRANITE4_GEMM_F32, b->normed, H, y.wg, rows, I, H, &eg, nullptr,
                                0) != 0 ||
          granite4_prefill_gemm(GRANITE4_GEMM_F32, b->normed, H, y.wu, rows, I, H, &eu, nullptr,
                                0) != 0 ||
          granite4_prefill_silu_mul(b->gu, I, rows, b->act) != 0 ||
          granite4_prefill_gemm(GRANITE4_GEMM_RESIDUAL, b->act, I, y.wd, rows, H, I, &ed, nullptr,
                                0) != 0)
             ? -1
             : 0;
}

// Final norm into d_hidden_out and / or the LM head's logits [rows][vocab].
int head(const Granite4DecodeModel* m, const Granite4BatchBuffers* b, int rows,
         uint16_t* d_hidden_out, uint16_t* d_logits) {
  if (d_hidden_out == nullptr && d_logits == nullptr) return 0;
  uint16_t* normed = d_hidden_out != nullptr ? d_hidden_out : b->normed;
  if (granite4_kernel_rmsnorm(b->hidden, m->final_norm, m->eps, rows, m->H, normed) != 0)
    return -1;
  if (d_logits == nullptr) return 0;
  const Granite4GemmEpilogue e =
      epi_bf16(m->lm_scale, m->lm_scale, m->lm_scale, INT32_MAX, INT32_MAX, d_logits, m->vocab);
  return granite4_prefill_gemm(GRANITE4_GEMM_BF16, normed, m->H, m->lm_head, rows, m->vocab,
                               m->H, &e, nullptr, 0);
}

}  // namespace

extern "C" {

int granite4_prefill_layers(const Granite4DecodeModel* m, const Granite4BatchBuffers* b,
                            const int32_t* d_tokens, int start, int rows, const int* d_pt, int ops,
                            uint16_t* d_hidden_out, uint16_t* d_logits) {
  const int fp8 = ops == GRANITE4_OPS_FP8;
  if ((ops != GRANITE4_OPS_BF16 && !fp8) || !dims_ok(m) || !layers_ok(m, fp8) ||
      !buffers_ok(b, m, rows, fp8) || d_tokens == nullptr || start < 0 ||
      (d_pt == nullptr && static_cast<long long>(start) + rows > m->kv_stride) ||
      static_cast<long long>(start) + rows > m->max_pos ||
      (d_logits != nullptr && m->lm_head == nullptr) ||
      ((d_hidden_out != nullptr || d_logits != nullptr) && m->final_norm == nullptr)) {
    std::fprintf(stderr, "granite4: granite4_prefill_layers: invalid arguments\n");
    return -1;
  }
  const int Hq = m->Hq, Hk = m->Hk, nq = Hq * 128, nk = Hk * 128, nqkv = nq + 2 * nk;
  const int group = m->kv_bits == 16 ? 128 : m->kv_group;
  if (granite4_embed_rows(d_tokens + start, rows, m->emb, m->vocab, m->H, m->emb_mult,
                          b->hidden) != 0)
    return -1;
  for (int l = 0; l < m->layers; ++l) {
    const Granite4DecodeLayer& y = m->layer[l];
    if (norm_in(m, b, y.attn_norm, rows, fp8) != 0 ||
        qkv_gemm(m, y, b, rows, fp8, b->qkv, nqkv, b->qkv + nq, nqkv, b->qkv + nq + nk, nqkv) != 0 ||
        granite4_rope_append(b->qkv, nqkv, b->qkv + nq, nqkv, b->qkv + nq + nk, nqkv, m->cos_tbl,
                             m->sin_tbl, m->max_pos, rows, Hq, Hk, 128, start, nullptr, d_pt,
                             nullptr, m->kv_bits, group, 0, 1, b->q_rot, nq, y.cache_k,
                             y.cache_v, y.k_scale, y.v_scale, m->kv_stride) != 0 ||
        granite4_prefill_attn(b->q_rot, rows, Hq, Hk, 128, m->attn_scale, y.cache_k, y.cache_v,
                              y.k_scale, y.v_scale, m->kv_bits, group, m->kv_stride, start, d_pt,
                              0, b->attn) != 0 ||
        layer_tail(m, y, b, rows, fp8) != 0) {
      std::fprintf(stderr, "granite4: granite4_prefill_layers: layer %d failed\n", l);
      return -1;
    }
  }
  return head(m, b, rows, d_hidden_out, d_logits);
}

int granite4_decode_step_multi(const Granite4DecodeModel* m, const Granite4BatchBuffers* b,
                               const GpuMultiRows* d_rows, int rows, int ops,
                               uint16_t* d_hidden_out, uint16_t* d_logits) {
  const int fp8 = ops == GRANITE4_OPS_FP8;
  if ((ops != GRANITE4_OPS_BF16 && !fp8) || !dims_ok(m) || !layers_ok(m, fp8) ||
      !buffers_ok(b, m, rows, fp8) || d_rows == nullptr || rows > GRANITE4_MAX_VERIFY_ROWS ||
      b->attn_scratch == nullptr || (m->kv_bits != 16 && m->kv_group != 128) ||
      (d_logits != nullptr && m->lm_head == nullptr) ||
      ((d_hidden_out != nullptr || d_logits != nullptr) && m->final_norm == nullptr)) {
    std::fprintf(stderr, "granite4: granite4_decode_step_multi: invalid arguments\n");
    return -1;
  }
  const int Hq = m->Hq, Hk = m->Hk, nq = Hq * 128, nk = Hk * 128;
  // The attention reads each row's position and page table from the
  // descriptor (device addresses inside it).
  const int* row_pos = reinterpret_cast<const int*>(reinterpret_cast<const char*>(d_rows) +
                                                    offsetof(GpuMultiRows, pos));
  const int* const* row_pt = reinterpret_cast<const int* const*>(
      reinterpret_cast<const char*>(d_rows) + offsetof(GpuMultiRows, pt));
  // The attention's split layout follows the longest sequence the model
  // takes, max_pos (the reference's multi step passes g->max_pos,
  // forward_gpu.cu:2567-2580); a pool shorter than that (which the reference
  // rejects) takes its own length.
  const int split_len = m->max_pos <= m->kv_stride ? m->max_pos : 0;
  // q, k, v as three row blocks of the qkv buffer (the multi append's layout).
  uint16_t* q = b->qkv;
  uint16_t* k = q + static_cast<size_t>(rows) * nq;
  uint16_t* v = k + static_cast<size_t>(rows) * nk;
  if (granite4_multi_embed(d_rows, rows, m->emb, m->vocab, m->H, m->emb_mult, b->hidden) != 0)
    return -1;
  for (int l = 0; l < m->layers; ++l) {
    const Granite4DecodeLayer& y = m->layer[l];
    if (norm_in(m, b, y.attn_norm, rows, fp8) != 0 ||
        qkv_gemm(m, y, b, rows, fp8, q, nq, k, nk, v, nk) != 0 ||
        granite4_multi_rope_append(q, k, v, m->cos_tbl, m->sin_tbl, d_rows, rows, Hq, Hk, 128,
                                   m->kv_bits, y.cache_k, y.cache_v, y.k_scale, y.v_scale,
                                   m->kv_stride, b->q_rot) != 0 ||
        granite4_attn_paged(b->q_rot, rows, Hq, Hk, 128, m->attn_scale, y.cache_k, y.cache_v,
                            y.k_scale, y.v_scale, m->kv_bits, 128, m->kv_stride, 0, nullptr,
                            nullptr, row_pos, row_pt, split_len, 0, b->attn_scratch,
                            b->attn) != 0 ||
        layer_tail(m, y, b, rows, fp8) != 0) {
      std::fprintf(stderr, "granite4: granite4_decode_step_multi: layer %d failed\n", l);
      return -1;
    }
  }
  return head(m, b, rows, d_hidden_out, d_logits);
}

}  // extern "C"
