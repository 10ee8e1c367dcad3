// decode_step.hip - the batch-1 decode step of the whole model as one C ABI
// call: the reference's forward_position (forward_gpu.cu:2066-2285) with the
// layer ops folded into this library's decode GEMVs and attention.
//
// Order per step (position *d_pos, token d_tokens[*d_pos]):
//   hidden = bf16(emb_mult * emb[token])                    } layer 0: one launch,
//   q_rot, k_rot, v = RoPE(GEMV(RMSNorm(hidden)))            } gemv_embed_rmsnorm_qkv_rope
//   per layer (layers > 0 start with):
//     q_rot, k_rot, v = RoPE(GEMV(RMSNorm(hidden)))          gemv_rmsnorm_qkv_rope
//     KV append at d_pt[*d_pos]; attn_out = attention       attn_decode_append_rotated
//     hidden = bf16(hidden + resid_mult * GEMV_o(attn_out))  gemv_fp8w_resid
//     act = SwiGLU(GEMV_g, GEMV_u of RMSNorm(hidden))        gemv_rmsnorm_silu_gate_up
//     hidden = bf16(hidden + resid_mult * GEMV_d(act))       gemv_fp8w_resid
//   hidden_out = RMSNorm(hidden, final_norm)                 (optional)
//   logits = bf16(lm_scale * GEMV_lm(RMSNorm(hidden)))       (optional)
//
// Five launches per layer plus the head, all on the
// calling thread's stream, no allocation and no synchronisation: a caller
// captures the step once in a HIP graph and replays it per token, advancing
// *d_pos between replays (capture_decode_graph, forward_gpu.cu:2934-2964).
// Each launch is one of this library's entry points, so the step's outputs
// are bit-identical to calling them one by one in this order (the first
// launch is bit-identical to granite4_embed_at_pos then
// granite4_gemv_rmsnorm_qkv_rope).
#include "g4_common.h"
#include "granite4_layerops.h"

#include <cmath>
#include <cstdint>
#include <cstdio>

namespace {

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool k_ok(int K) { return K >= 64 && K % 64 == 0 && K <= 16384; }  // the GEMVs' K range
bool fin(float x) { return std::isfinite(x); }

// Every condition the step's entry points check, tested before the first
// launch, so that a call either launches nothing (-1) or launches the whole
// step: a step rejected half-way would already have appended the position's
// K / V rows in the earlier layers.
bool model_ok(const Granite4DecodeModel* m) {
  if (m == nullptr || m->layers <= 0 || m->layer == nullptr || m->Hq <= 0 || m->Hk <= 0 ||
      m->Hq != 4 * m->Hk || !k_ok(m->H) || !k_ok(m->I) || !k_ok(m->Hq * 128) ||
      m->emb == nullptr || !al16(m->emb) || m->vocab <= 0 || m->cos_tbl == nullptr || m->sin_tbl == nullptr ||
      m->max_pos <= 0 || m->kv_stride <= 0 || !fin(m->eps) || !fin(m->emb_mult) ||
      !fin(m->resid_mult) || !fin(m->attn_scale) || !fin(m->lm_scale))
    return false;
  if (m->kv_bits != 16 && m->kv_bits != 8 && m->kv_bits != 4 && m->kv_bits != 5) return false;
  if (m->kv_bits != 16 && m->kv_group != 32 && m->kv_group != 64 && m->kv_group != 128)
    return false;
  if (m->lm_head != nullptr && (m->final_norm == nullptr || !al16(m->lm_head))) return false;
  if (m->final_norm != nullptr && !al16(m->final_norm)) return false;
  const long long qkv_rows = static_cast<long long>(m->Hq + 2 * m->Hk) * 128;
  if (qkv_rows * m->H >= (1LL << 40) || static_cast<long long>(m->I) * m->H >= (1LL << 40) ||
      static_cast<long long>(m->vocab) * m->H >= (1LL << 40))
    return false;
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
  }
  return true;
}

bool buffers_ok(const Granite4DecodeBuffers* b) {
  if (b == nullptr || b->attn_scratch == nullptr) return false;
  const void* ptrs[] = {b->hidden, b->q_rot, b->k_rot, b->v, b->attn_out, b->act};
  for (const void* p : ptrs)
    if (p == nullptr || !al16(p)) return false;
  return true;
}

}  // namespace

extern "C" {

int granite4_decode_step(const Granite4DecodeModel* m, const Granite4DecodeBuffers* b,
                         const int32_t* d_tokens, const int* d_pos, const int* d_pt,
                         uint16_t* d_hidden_out, uint16_t* d_logits) {
  if (!model_ok(m) || !buffers_ok(b) || d_tokens == nullptr || d_pos == nullptr ||
      (d_logits != nullptr && m->lm_head == nullptr) ||
      (d_hidden_out != nullptr && m->final_norm == nullptr)) {
    std::fprintf(stderr, "granite4: granite4_decode_step: invalid arguments\n");
    return -1;
  }
  const int H = m->H, I = m->I, Hq = m->Hq, Hk = m->Hk, nq = Hq * 128;
  for (int l = 0; l < m->layers; ++l) {
    const Granite4DecodeLayer& y = m->layer[l];
    const int qkv =
        l == 0 ? granite4_gemv_embed_rmsnorm_qkv_rope(d_tokens, m->emb, m->vocab, m->emb_mult,
                                                      b->hidden, y.attn_norm, m->eps, y.wq, y.wk,
                                                      y.wv, y.sq, y.sk, y.sv, m->cos_tbl,
                                                      m->sin_tbl, m->max_pos, d_pos, Hq, Hk, H,
                                                      b->q_rot, b->k_rot, b->v)
               : granite4_gemv_rmsnorm_qkv_rope(b->hidden, y.attn_norm, m->eps, y.wq, y.wk, y.wv,
                                                y.sq, y.sk, y.sv, m->cos_tbl, m->sin_tbl,
                                                m->max_pos, d_pos, Hq, Hk, H, b->q_rot, b->k_rot,
                                                b->v);
    if (qkv != 0 ||
        granite4_attn_decode_append_rotated(b->q_rot, b->k_rot, b->v, m->max_pos, d_pos, d_pt,
                                            Hq, Hk, m->attn_scale, y.cache_k, y.cache_v,
                                            y.k_scale, y.v_scale, m->kv_bits, m->kv_group,
                                            m->kv_stride, b->attn_scratch, b->attn_out) != 0 ||
        granite4_gemv_fp8w_resid(b->attn_out, y.wo, y.so, b->hidden, m->resid_mult, H, nq,
                                 b->hidden) != 0 ||
        granite4_gemv_rmsnorm_silu_gate_up(b->hidden, y.ffn_norm, m->eps, y.wg, y.wu, y.sg, y.su,
                                           I, H, b->act) != 0 ||
        granite4_gemv_fp8w_resid(b->act, y.wd, y.sd, b->hidden, m->resid_mult, H, I,
                                 b->hidden) != 0) {
      std::fprintf(stderr, "granite4: granite4_decode_step: layer %d failed\n", l);
      return -1;
    }
  }
  if (d_hidden_out != nullptr &&
      granite4_kernel_rmsnorm(b->hidden, m->final_norm, m->eps, 1, H, d_hidden_out) != 0)
    return -1;
  if (d_logits != nullptr &&
      granite4_gemv_rmsnorm_qkv(b->hidden, m->final_norm, m->eps, m->lm_head, nullptr, nullptr,
                                m->lm_scale, 0.0f, 0.0f, m->vocab, 0, 0, H, d_logits, nullptr,
                                nullptr) != 0)
    return -1;
  return 0;
}

}  // extern "C"
