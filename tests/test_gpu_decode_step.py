"""granite4_decode_step (the reference's forward_position, forward_gpu.cu:
2066-2285): a 2-layer batch-1 decode step of the 8B shapes (H 4096, I 12800,
32 / 8 heads of 128) through the C ABI, against

- the same library entry points called one by one in the step's order
  (bit-identical: hidden, logits, final-normed hidden, every KV arena byte);
- the CPU oracle's composition of the step on the same inputs (the GEMVs as
  exact double sums, then the same roundings). The GPU sums in f32 in its own
  order, and a bf16 rounding that lands on the other side of a tie changes
  later values by an ulp, so the bar here is a tolerance: every element of the
  final hidden and the logits within 2^-5 of the row's rms (32x below the
  values' spread), and at least 95 % of them within 2 bf16 ulps;
- its own HIP graph: captured once, replayed at two consecutive positions
  with *d_pos advanced on the device between replays, every replay equal to
  the eager step at that position from the same starting state.
"""
import sys

import numpy as np
import pytest
import torch

import oracle_lib as ol
from pkg import layerops

pytestmark = pytest.mark.gpu

L = None
H, I_, HQ, HK, D = 4096, 12800, 32, 8, 128
VOCAB = 1000
LAYERS = 2


def setup_module(module):
    global L
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    L = layerops()
    torch.cuda.init()
    L.use_stream()


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def host(t):
    if t.dtype == torch.bfloat16:
        t = t.view(torch.int16)
    a = t.detach().cpu().numpy()
    return a.view(np.uint16) if a.dtype == np.int16 else a


def ulp_diff(a, b):
    ai = a.astype(np.int32)
    bi = b.astype(np.int32)
    ai = np.where(ai & 0x8000, 0x8000 - ai, ai)
    bi = np.where(bi & 0x8000, 0x8000 - bi, bi)
    return np.abs(ai - bi)


class Model:
    """Random 2-layer model (fp8 weights of N(0, 1) values, gammas N(1, 0.1)),
    a paged KV arena per layer with `ctx` positions already filled."""

    def __init__(self, bits, group, ctx, seed):
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        self.bits, self.group, self.ctx = bits, group, ctx
        self.stride = 1024

        def w8(n, k):
            return torch.randn((n, k), generator=g, device="cuda").to(
                torch.float8_e4m3fn).view(torch.uint8)

        def bf(*shape, mean=0.0, std=1.0):
            return (torch.randn(shape, generator=g, device="cuda") * std + mean).to(torch.bfloat16)

        self.emb = bf(VOCAB, H, std=0.05)
        self.final_norm = bf(H, mean=1.0, std=0.1)
        self.lm_head = w8(VOCAB, H)
        self.layers = []
        kb, vb = L.kv_row_bytes(bits)
        ng = 128 // group
        for _ in range(LAYERS):
            ly = {"attn_norm": bf(H, mean=1.0, std=0.1), "ffn_norm": bf(H, mean=1.0, std=0.1),
                  "wq": w8(HQ * D, H), "wk": w8(HK * D, H), "wv": w8(HK * D, H),
                  "wo": w8(H, HQ * D), "wg": w8(I_, H), "wu": w8(I_, H), "wd": w8(H, I_),
                  "sq": 1 / 64, "sk": 1 / 64, "sv": 1 / 64, "so": 1 / 64, "sg": 1 / 64,
                  "su": 1 / 64, "sd": 1 / 112}
            # an arena with every row filled (random codes and scales, or bf16)
            if bits == 16:
                ly["cache_k"] = bf(HK, self.stride, D).view(torch.uint8)
                ly["cache_v"] = bf(HK, self.stride, D).view(torch.uint8)
                ly["k_scale"] = ly["v_scale"] = None
            else:
                ly["cache_k"] = torch.randint(0, 256, (HK, self.stride, kb), generator=g,
                                              device="cuda", dtype=torch.int32).to(torch.uint8)
                ly["cache_v"] = torch.randint(0, 256, (HK, self.stride, vb), generator=g,
                                              device="cuda", dtype=torch.int32).to(torch.uint8)
                ly["k_scale"] = torch.rand((HK, self.stride, ng), generator=g,
                                           device="cuda") * 0.02 + 0.01
                ly["v_scale"] = torch.rand((HK, self.stride, ng), generator=g,
                                           device="cuda") * 0.02 + 0.01
            self.layers.append(ly)
        self.tokens = torch.randint(0, VOCAB, (self.stride,), generator=g, device="cuda",
                                    dtype=torch.int32)
        perm = torch.randperm(self.stride // 16, generator=g, device="cuda").to(torch.int32)
        self.pt = (perm.repeat_interleave(16) * 16 +
                   torch.arange(16, device="cuda", dtype=torch.int32).repeat(self.stride // 16))
        c, s = L.rope_tables(1e7, D, 8192)
        self.cos, self.sin = c, s
        self.step = L.DecodeStep(self.layers, H, I_, HQ, HK, VOCAB, self.emb, c, s, eps=1e-5,
                                 emb_mult=12.0, resid_mult=0.22, attn_scale=1.0 / 128,
                                 final_norm=self.final_norm, lm_head=self.lm_head,
                                 lm_scale=1 / 64, kv_bits=bits, kv_group=group,
                                 kv_stride=self.stride)

    def arenas(self):
        return [(ly["cache_k"].clone(), ly["cache_v"].clone()) for ly in self.layers]

    def restore(self, saved):
        for ly, (k, v) in zip(self.layers, saved):
            ly["cache_k"].copy_(k)
            ly["cache_v"].copy_(v)


def one_by_one(m, pos, hidden_out, logits):
    """The step's launches called individually through the C ABI."""
    st = m.step
    rs = 0.22
    L.call("granite4_embed_at_pos", m.tokens, pos, m.emb, VOCAB, H, 12.0, st.hidden)
    for ly in m.layers:
        L.call("granite4_gemv_rmsnorm_qkv_rope", st.hidden, ly["attn_norm"], 1e-5, ly["wq"],
               ly["wk"], ly["wv"], ly["sq"], ly["sk"], ly["sv"], m.cos, m.sin, m.cos.shape[0],
               pos, HQ, HK, H, st.q_rot, st.k_rot, st.v)
        L.call("granite4_attn_decode_append_rotated", st.q_rot, st.k_rot, st.v, m.cos.shape[0],
               pos, m.pt, HQ, HK, 1.0 / 128, ly["cache_k"], ly["cache_v"], ly["k_scale"],
               ly["v_scale"], m.bits, m.group, m.stride, st.scratch, st.attn_out)
        L.call("granite4_gemv_fp8w_resid", st.attn_out, ly["wo"], ly["so"], st.hidden, rs, H,
               HQ * D, st.hidden)
        L.call("granite4_gemv_rmsnorm_silu_gate_up", st.hidden, ly["ffn_norm"], 1e-5, ly["wg"],
               ly["wu"], ly["sg"], ly["su"], I_, H, st.act)
        L.call("granite4_gemv_fp8w_resid", st.act, ly["wd"], ly["sd"], st.hidden, rs, H, I_,
               st.hidden)
    L.call("granite4_kernel_rmsnorm", st.hidden, m.final_norm, 1e-5, 1, H, hidden_out)
    L.call("granite4_gemv_rmsnorm_qkv", st.hidden, m.final_norm, 1e-5, m.lm_head, None, None,
           1 / 64, 0.0, 0.0, VOCAB, 0, 0, H, logits, None, None)


def oracle_step(m, p, arenas):
    """The step on the CPU: oracle GEMVs (exact products, double sums), the
    oracle's RMSNorm, RoPE, KV append, split-KV attention, SwiGLU formula."""
    bits, group = m.bits, m.group
    c, s = host(m.cos), host(m.sin)
    pt = host(m.pt)
    tok = int(host(m.tokens)[p])
    x = ol.embed_rows(np.array([tok], np.int32), host(m.emb), 12.0)[0]
    rs = np.float32(0.22)

    def gemv(a, w, scale):
        return ol.gemv_fp8w(a, host(w), np.float32(scale))

    def resid(xb, y):
        return ol.f32_to_bf16(ol.bf16_to_f32(xb) + rs * y)

    for li, ly in enumerate(m.layers):
        ck, cv = (host(t).reshape(-1).copy() for t in arenas[li])
        ks = None if ly["k_scale"] is None else host(ly["k_scale"]).reshape(-1).copy()
        vs = None if ly["v_scale"] is None else host(ly["v_scale"]).reshape(-1).copy()
        normed = ol.rmsnorm(x[None], host(ly["attn_norm"]), 1e-5)[0]
        q = ol.f32_to_bf16(gemv(normed, ly["wq"], ly["sq"]))
        k = ol.f32_to_bf16(gemv(normed, ly["wk"], ly["sk"]))
        v = ol.f32_to_bf16(gemv(normed, ly["wv"], ly["sv"]))
        q_rot = ol.rope_rows(q.reshape(1, HQ, D), [p], c, s).reshape(1, -1)
        k_rot = ol.rope_rows(k.reshape(1, HK, D), [p], c, s).reshape(1, -1)
        if ks is None:
            ks = np.zeros(1, np.float32)
            vs = np.zeros(1, np.float32)
        ol.rope_append(None, k_rot, v.reshape(1, -1), None, None, [p], [pt[p]], bits, group,
                       m.stride, HK, rotate_k=False, k_round_bf16=True, cache_k=ck, cache_v=cv,
                       k_scale=ks, v_scale=vs)
        att = ol.attn_split(q_rot, ck, cv, None if bits == 16 else ks, None if bits == 16 else vs,
                            bits, group, m.stride, [p], pts=[pt], scale=1.0 / 128)[0]
        x = resid(x, gemv(att, ly["wo"], ly["so"]))
        normed = ol.rmsnorm(x[None], host(ly["ffn_norm"]), 1e-5)[0]
        gg = gemv(normed, ly["wg"], ly["sg"]).astype(np.float64)
        uu = gemv(normed, ly["wu"], ly["su"]).astype(np.float64)
        act = ol.f32_to_bf16((gg / (1.0 + np.exp(-gg)) * uu).astype(np.float32))
        x = resid(x, gemv(act, ly["wd"], ly["sd"]))
    hid = ol.rmsnorm(x[None], host(m.final_norm), 1e-5)[0]
    logits = ol.f32_to_bf16(gemv(hid, m.lm_head, 1 / 64))
    return hid, logits


def _close(got, want, what):
    g = ol.bf16_to_f32(got).astype(np.float64)
    w = ol.bf16_to_f32(want).astype(np.float64)
    rms = np.sqrt(np.mean(w * w))
    err = np.abs(g - w)
    within = (ulp_diff(got, want) <= 2).mean()
    note(f"  {what}: max |err| / rms {err.max() / rms:.2e}, within 2 ulp {within:.4f}")
    assert err.max() <= rms * 2.0 ** -5, (what, err.max(), rms)
    assert within >= 0.95, (what, within)


@pytest.mark.parametrize("bits,group", [(16, 128), (8, 128), (5, 32), (4, 32), (5, 128)])
def test_decode_step_two_layers(bits, group):
    note(f"decode step bits={bits} group={group}")
    m = Model(bits, group, ctx=300, seed=0xD5 + bits)
    p = 300
    d_pos = torch.tensor([p], dtype=torch.int32, device="cuda")
    start = m.arenas()
    # one by one
    h1 = torch.empty(H, dtype=torch.bfloat16, device="cuda")
    l1 = torch.empty(VOCAB, dtype=torch.bfloat16, device="cuda")
    one_by_one(m, d_pos, h1, l1)
    hid1 = host(m.step.hidden).copy()
    arena1 = [(host(k).copy(), host(v).copy()) for k, v in m.arenas()]
    # the library step from the same starting state
    m.restore(start)
    h2 = torch.empty_like(h1)
    l2 = torch.empty_like(l1)
    m.step(m.tokens, d_pos, m.pt, h2, l2)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(m.step.hidden), hid1)
    np.testing.assert_array_equal(host(h2), host(h1))
    np.testing.assert_array_equal(host(l2), host(l1))
    for (k1, v1), (k2, v2) in zip(arena1, m.arenas()):
        np.testing.assert_array_equal(host(k2), k1)
        np.testing.assert_array_equal(host(v2), v1)
    # the oracle's composition of the same step
    want_h, want_l = oracle_step(m, p, start)
    _close(host(h2), want_h, "final-normed hidden")
    _close(host(l2), want_l, "logits")


def test_decode_step_graph_replays_two_positions():
    """Captured once; replayed at p and p + 1 (*d_pos advanced on the device
    between the replays), each replay equal to the eager step."""
    note("decode step graph")
    m = Model(8, 128, ctx=500, seed=0xD6)
    p = 500
    d_pos = torch.tensor([p], dtype=torch.int32, device="cuda")
    h = torch.empty(H, dtype=torch.bfloat16, device="cuda")
    lg = torch.empty(VOCAB, dtype=torch.bfloat16, device="cuda")
    start = m.arenas()
    want = []
    for i in range(2):
        d_pos.fill_(p + i)
        m.step(m.tokens, d_pos, m.pt, h, lg)
        torch.cuda.synchronize()
        want.append((host(h).copy(), host(lg).copy(),
                     [(host(k).copy(), host(v).copy()) for k, v in m.arenas()]))
    m.restore(start)
    d_pos.fill_(p)
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    L.use_stream(s)
    try:
        with torch.cuda.graph(g, stream=s):
            m.step(m.tokens, d_pos, m.pt, h, lg)
    finally:
        L.call("granite4_set_stream", None)
    torch.cuda.synchronize()
    m.restore(start)  # capture launched nothing, but be explicit
    for i in range(2):
        d_pos.fill_(p + i)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(host(h), want[i][0])
        np.testing.assert_array_equal(host(lg), want[i][1])
        for (k2, v2), (k1, v1) in zip(m.arenas(), want[i][2]):
            np.testing.assert_array_equal(host(k2), k1)
            np.testing.assert_array_equal(host(v2), v1)


def test_decode_step_rejects_bad_arguments():
    note("decode step args")
    m = Model(16, 128, ctx=10, seed=0xD7)
    d_pos = torch.tensor([10], dtype=torch.int32, device="cuda")
    with pytest.raises(L.Granite4Error):
        m.step(None, d_pos, m.pt)
    lg = torch.empty(VOCAB, dtype=torch.bfloat16, device="cuda")
    m.step.model.lm_head = None
    with pytest.raises(L.Granite4Error):
        m.step(m.tokens, d_pos, m.pt, None, lg)


def test_decode_step_rejects_a_bad_later_layer_before_any_launch():
    """A bad argument of the second layer (a NaN weight scale) is rejected
    before anything is launched: no layer's arena is touched, so a caller
    that fixes the argument and calls again appends the position once."""
    note("decode step rejects layer 1 before launching")
    m = Model(8, 128, ctx=40, seed=0xD8)
    d_pos = torch.tensor([40], dtype=torch.int32, device="cuda")
    start = [(host(k).copy(), host(v).copy()) for k, v in m.arenas()]
    hid = host(m.step.hidden).copy()
    m.step._arr[1].sd = float("nan")
    with pytest.raises(L.Granite4Error):
        m.step(m.tokens, d_pos, m.pt)
    torch.cuda.synchronize()
    for (k, v), (k0, v0) in zip(m.arenas(), start):
        np.testing.assert_array_equal(host(k), k0)
        np.testing.assert_array_equal(host(v), v0)
    np.testing.assert_array_equal(host(m.step.hidden), hid)
