"""GPU parity of the batched layer sequences (layer_steps.hip):
granite4_prefill_layers (the reference's forward_prefill for one chunk) and
granite4_decode_step_multi (forward_multi_step: one position of up to 16
sessions through GpuMultiRows), in both activation forms (the reference's
bf16 activations, and FP8 activations with per-tensor scales).

Each sequence is checked three ways: bit-identical to the same entry points
called one by one (hidden, normed hidden, logits and every arena byte),
against the oracle's composition of the same sequence (exact products and
double sums in the GEMMs, so the f32 GPU sums can round across a bf16 tie,
and two layers carry such differences on: within 2^-5 of the rms, and >= 95 %
of the values of magnitude >= rms / 16 within 2 bf16 ulps), and, for the multi step, under graph replay at two
consecutive positions.
"""
import sys

import numpy as np
import pytest
import torch

import oracle_lib as ol
from pkg import layerops

pytestmark = pytest.mark.gpu
L = None


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
    torch.cuda.synchronize()
    a = t.detach().cpu()
    if a.dtype == torch.bfloat16:
        return a.view(torch.int16).numpy().view(np.uint16)
    return a.numpy()


def dev(a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a).cuda()


def ulp_diff(a, b):
    ai = a.astype(np.int32)
    bi = b.astype(np.int32)
    ai = np.where(ai & 0x8000, 0x8000 - ai, ai)
    bi = np.where(bi & 0x8000, 0x8000 - bi, bi)
    return np.abs(ai - bi)


def _close(got, want, what, fp8=False):
    """bf16 activations: max error <= rms 2^-5 and >= 95 % of the values of
    magnitude >= rms / 16 within 2 bf16 ulps (nearer zero a bf16 ulp is far
    below the GEMM sums' rounding, which the rms bound covers).
    FP8 activations: a 1-ulp difference in a bf16 value that a per-tensor
    FP8 quantiser reads can move the tensor's amax, and so every code of it
    by up to half an FP8 step (2^-4 relative), and flip single codes by a
    whole step (2^-3): max error <= rms 2^-3 and mean error <= rms 2^-7."""
    g = ol.bf16_to_f32(got).astype(np.float64)
    w = ol.bf16_to_f32(want).astype(np.float64)
    rms = np.sqrt(np.mean(w * w))
    err = np.abs(g - w)
    big = np.abs(w) >= rms / 16
    within = (ulp_diff(got, want)[big] <= 2).mean()
    note(f"  {what}: max |err| / rms {err.max() / rms:.2e}, mean {err.mean() / rms:.2e}, "
         f"within 2 ulp {within:.4f}")
    if fp8:
        assert err.max() <= rms * 2.0 ** -3, (what, err.max(), rms)
        assert err.mean() <= rms * 2.0 ** -7, (what, err.mean(), rms)
    else:
        assert err.max() <= rms * 2.0 ** -5, (what, err.max(), rms)
        assert within >= 0.95, (what, within)


class Model:
    """Random model (fp8 weights of N(0, 1) values, q|k|v and gate|up each one
    block), `layers` layers, a KV arena per layer with every row filled."""

    def __init__(self, H, I, Hq, Hk, vocab, layers, bits, group, stride, max_rows, seed,
                 max_pos=65536, split_qkv=False):
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        self.H, self.I, self.Hq, self.Hk, self.vocab = H, I, Hq, Hk, vocab
        self.bits, self.group, self.stride = bits, group, stride
        # the multi step's split layout: max_pos when the pool holds that many rows
        self.split_len = max_pos if max_pos <= stride else 0
        self.eps, self.emb_mult, self.rs, self.att, self.lm_scale = 1e-5, 12.0, 0.22, 1 / 128, 1 / 64
        nq, nk = Hq * 128, Hk * 128

        def w8(n, k):
            return torch.randn((n, k), generator=g, device="cuda").to(
                torch.float8_e4m3fn).view(torch.uint8)

        def bf(*shape, mean=0.0, std=1.0):
            return (torch.randn(shape, generator=g, device="cuda") * std + mean).to(torch.bfloat16)

        self.emb = bf(vocab, H, std=0.05)
        self.final_norm = bf(H, mean=1.0, std=0.1)
        self.lm_head = w8(vocab, H)
        self.layers = []
        kb, vb = L.kv_row_bytes(bits)
        ng = 128 // group
        for _ in range(layers):
            if split_qkv:
                wq, wk, wv = w8(nq, H), w8(nk, H), w8(nk, H)
            else:
                wqkv = w8(nq + 2 * nk, H)
                wq, wk, wv = wqkv[:nq], wqkv[nq:nq + nk], wqkv[nq + nk:]
            wgu = w8(2 * I, H)
            ly = {"attn_norm": bf(H, mean=1.0, std=0.1), "ffn_norm": bf(H, mean=1.0, std=0.1),
                  "wq": wq, "wk": wk, "wv": wv, "wo": w8(H, nq), "wg": wgu[:I], "wu": wgu[I:],
                  "wd": w8(H, I), "sq": 1 / 64, "sk": 1 / 64, "sv": 1 / 64, "so": 1 / 64,
                  "sg": 1 / 64, "su": 1 / 64, "sd": 1 / 112}
            if bits == 16:
                ly["cache_k"] = bf(Hk, stride, 128).view(torch.uint8)
                ly["cache_v"] = bf(Hk, stride, 128).view(torch.uint8)
                ly["k_scale"] = ly["v_scale"] = None
            else:
                ly["cache_k"] = torch.randint(0, 256, (Hk, stride, kb), generator=g,
                                              device="cuda", dtype=torch.int32).to(torch.uint8)
                ly["cache_v"] = torch.randint(0, 256, (Hk, stride, vb), generator=g,
                                              device="cuda", dtype=torch.int32).to(torch.uint8)
                if bits == 8:  # int8 codes stay within +-127
                    ly["cache_k"][ly["cache_k"] == 0x80] = 0x81
                    ly["cache_v"][ly["cache_v"] == 0x80] = 0x81
                ly["k_scale"] = torch.rand((Hk, stride, ng), generator=g, device="cuda") * 0.02 + 0.01
                ly["v_scale"] = torch.rand((Hk, stride, ng), generator=g, device="cuda") * 0.02 + 0.01
            self.layers.append(ly)
        c, s = L.rope_tables(1e7, 128, max_pos)
        self.cos, self.sin = c, s
        self.steps = L.LayerSteps(self.layers, H, I, Hq, Hk, vocab, self.emb, c, s, max_rows,
                                  eps=self.eps, emb_mult=self.emb_mult, resid_mult=self.rs,
                                  attn_scale=self.att, final_norm=self.final_norm,
                                  lm_head=self.lm_head, lm_scale=self.lm_scale, kv_bits=bits,
                                  kv_group=group, kv_stride=stride)

    def arenas(self):
        out = []
        for ly in self.layers:
            t = [ly["cache_k"].clone(), ly["cache_v"].clone()]
            if ly["k_scale"] is not None:
                t += [ly["k_scale"].clone(), ly["v_scale"].clone()]
            out.append(t)
        return out

    def restore(self, saved):
        for ly, t in zip(self.layers, saved):
            ly["cache_k"].copy_(t[0])
            ly["cache_v"].copy_(t[1])
            if len(t) > 2:
                ly["k_scale"].copy_(t[2])
                ly["v_scale"].copy_(t[3])

    def host_arenas(self):
        return [[host(x).copy() for x in t] for t in self.arenas()]


def _epi(s0, s1, s2, seg1, seg2, out, ldc, residual=None, rs=1.0, f32=None):
    big = 2 ** 31 - 1
    return L.GemmEpilogue(s0, s1, s2, seg1 if seg1 else big, seg2 if seg2 else big,
                          L._ptr(out), L._ptr(f32), L._ptr(residual), rs, ldc)


def one_by_one(m, rows, fp8, first, attention, tail_q=None):
    """The sequences' launches through the C ABI one at a time: `first`
    embeds into st.hidden, `attention(ly, q_rot_or_qkv)` does RoPE + append +
    attention into st.attn."""
    st = m.steps
    H, I, nq, nk = m.H, m.I, m.Hq * 128, m.Hk * 128
    first()

    def norm(gamma):
        if fp8:
            L.call("granite4_add_rmsnorm_fp8", st.hidden, None, 1.0, gamma, m.eps, rows, H, None,
                   st.codes, st.scales, st.fp8_work)
        else:
            L.call("granite4_kernel_rmsnorm", st.hidden, gamma, m.eps, rows, H, st.normed)

    def gemm(out, W, N, K, ep, A=None, a_scale=None):
        if fp8 and A is None:
            L.call("granite4_gemm_fp8", out, st.codes, K, st.scales, W, rows, N, K, L._c.byref(ep))
        elif A is not None and a_scale is not None:
            L.call("granite4_gemm_fp8", out, A, K, a_scale, W, rows, N, K, L._c.byref(ep))
        else:
            L.call("granite4_prefill_gemm", out, st.normed if A is None else A, K, W, rows, N, K,
                   L._c.byref(ep), None, 0)

    for ly in m.layers:
        norm(ly["attn_norm"])
        attention(ly, gemm)
        gemm(L.GEMM_RESIDUAL, ly["wo"], H, nq, _epi(ly["so"], ly["so"], ly["so"], 0, 0, st.hidden,
                                                     H, st.hidden, m.rs), A=st.attn)
        norm(ly["ffn_norm"])
        if fp8:
            L.call("granite4_gemm_fp8_swiglu", st.codes, H, st.scales, ly["wg"], rows, I, H,
                   ly["sg"], ly["su"], st.act, st.act_codes, st.scales[1:], st.fp8_work)
            gemm(L.GEMM_RESIDUAL, ly["wd"], H, I, _epi(ly["sd"], ly["sd"], ly["sd"], 0, 0,
                                                       st.hidden, H, st.hidden, m.rs),
                 A=st.act_codes, a_scale=st.scales[1:])
        else:
            gemm(L.GEMM_F32, ly["wg"], I, H, _epi(ly["sg"], ly["sg"], ly["sg"], 0, 0, None,
                                                  2 * I, f32=st.gu))
            gemm(L.GEMM_F32, ly["wu"], I, H, _epi(ly["su"], ly["su"], ly["su"], 0, 0, None,
                                                  2 * I, f32=st.gu[:, I:]))
            L.call("granite4_prefill_silu_mul", st.gu, I, rows, st.act)
            gemm(L.GEMM_RESIDUAL, ly["wd"], H, I, _epi(ly["sd"], ly["sd"], ly["sd"], 0, 0,
                                                       st.hidden, H, st.hidden, m.rs), A=st.act)


def oracle_layers(m, x, fp8, arenas, attention):
    """The same sequence on the CPU (oracle GEMMs, norm, FP8 quantiser,
    SwiGLU); attention(li, ly, q, k, v, arena) appends and attends."""
    nq, nk, I = m.Hq * 128, m.Hk * 128, m.I
    rs = np.float32(m.rs)

    def resid(xb, y):
        return ol.f32_to_bf16(ol.bf16_to_f32(xb) + rs * y)

    def gemm_in(normed, W, scales, segs=None):
        if fp8:
            codes, s = ol.fp8_quantize(normed)
            return ol.gemm_fp8(codes, np.float32(s), W, scales, segs)
        return ol.gemm_bf16w(normed, W, scales, segs)

    for li, ly in enumerate(m.layers):
        wqkv = np.concatenate([host(ly["wq"]), host(ly["wk"]), host(ly["wv"])])
        normed = ol.rmsnorm(x, host(ly["attn_norm"]), m.eps)
        qkv = ol.f32_to_bf16(gemm_in(normed, wqkv, (ly["sq"], ly["sk"], ly["sv"]),
                                     (nq, nq + nk)))
        att = attention(li, ly, qkv[:, :nq], qkv[:, nq:nq + nk], qkv[:, nq + nk:], arenas[li])
        x = resid(x, ol.gemm_bf16w(att, host(ly["wo"]), (ly["so"],) * 3))
        normed = ol.rmsnorm(x, host(ly["ffn_norm"]), m.eps)
        wgu = np.concatenate([host(ly["wg"]), host(ly["wu"])])
        gu = gemm_in(normed, wgu, (ly["sg"], ly["su"], ly["su"]), (I, I))
        act = ol.silu_mul_f32(gu)
        if fp8:
            c3, s3 = ol.fp8_quantize(act)
            y = ol.gemm_fp8(c3, np.float32(s3), host(ly["wd"]), (ly["sd"],) * 3)
        else:
            y = ol.gemm_bf16w(act, host(ly["wd"]), (ly["sd"],) * 3)
        x = resid(x, y)
    hid = ol.rmsnorm(x, host(m.final_norm), m.eps)
    logits = ol.f32_to_bf16(ol.gemm_bf16w(hid, host(m.lm_head), (m.lm_scale,) * 3))
    return hid, logits


# ----------------------------------------------------------------------------- multi-session step
def _multi_rows(m, n, max_pos, seed):
    """GpuMultiRows for n sessions at random positions in [0, max_pos), each
    with its own page table over a pool of m.stride rows (the pages holding
    the sessions' positions distinct) and its own token array."""
    rs = np.random.default_rng(seed)
    pos, pts = ol.config2_page_tables(rs, n, m.stride // 16, max_pos)
    pos = np.minimum(pos, max_pos - 2)  # room for the replay at p + 1 (same page)
    toks = [rs.integers(0, m.vocab, max_pos).astype(np.int32) for _ in range(n)]
    keep = [dev(t) for t in pts] + [dev(t) for t in toks]
    M = L.multi_rows_struct()()
    M.n = n
    for i in range(n):
        M.pos[i] = int(pos[i])
        M.pt[i] = keep[i].data_ptr()
        M.tok[i] = keep[n + i].data_ptr()
    d_m = torch.from_numpy(np.frombuffer(bytes(M), np.uint8).copy()).cuda()
    return d_m, pos, pts, toks, keep


def _multi_one_by_one(m, d_m, n, fp8):
    st = m.steps
    nq, nk = m.Hq * 128, m.Hk * 128
    q = st.qkv.view(-1)[:n * nq].view(n, nq)
    k = st.qkv.view(-1)[n * nq:n * (nq + nk)].view(n, nk)
    v = st.qkv.view(-1)[n * (nq + nk):n * (nq + 2 * nk)].view(n, nk)
    off_pos = 4  # offsetof(GpuMultiRows, pos)
    off_pt = 4 + 4 * L.MAX_VERIFY_ROWS + 4  # pointers align to 8
    row_pos = d_m[off_pos:]
    row_pt = d_m[off_pt:]

    def first():
        L.call("granite4_multi_embed", d_m, n, m.emb, m.vocab, m.H, m.emb_mult, st.hidden)

    def attention(ly, gemm):
        gemm(L.GEMM_BF16, ly["wq"], nq, m.H, _epi(ly["sq"], ly["sq"], ly["sq"], 0, 0, q, nq))
        gemm(L.GEMM_BF16, ly["wk"], nk, m.H, _epi(ly["sk"], ly["sk"], ly["sk"], 0, 0, k, nk))
        gemm(L.GEMM_BF16, ly["wv"], nk, m.H, _epi(ly["sv"], ly["sv"], ly["sv"], 0, 0, v, nk))
        L.call("granite4_multi_rope_append", q, k, v, m.cos, m.sin, d_m, n, m.Hq, m.Hk, 128,
               m.bits, ly["cache_k"], ly["cache_v"], ly["k_scale"], ly["v_scale"], m.stride,
               st.q_rot)
        L.call("granite4_attn_paged", st.q_rot, n, m.Hq, m.Hk, 128, m.att, ly["cache_k"],
               ly["cache_v"], ly["k_scale"], ly["v_scale"], m.bits, 128, m.stride, 0, None, None,
               row_pos, row_pt, m.split_len, 0, st.attn_scratch, st.attn)
    one_by_one(m, n, fp8, first, attention)


@pytest.mark.parametrize("ops", ["bf16", "fp8"])
def test_decode_step_multi_matches_one_by_one_and_oracle(ops):
    """BASELINE config 2's step: 8 sessions, int8 KV with per-row scales,
    real 8B shapes (2 layers), positions below 1024 so that the oracle's
    attention stays fast; one by one bit for bit, then the oracle."""
    fp8 = ops == "fp8"
    note(f"decode step multi ops={ops}")
    n, stride = 8, 4096
    m = Model(4096, 12800, 32, 8, 1000, 2, 8, 128, stride, 16, 0x3A1 + fp8, max_pos=1024)
    d_m, pos, pts, toks, keep = _multi_rows(m, n, 1024, 0x3A2)
    start = m.arenas()
    hid1 = torch.empty((n, m.H), dtype=torch.bfloat16, device="cuda")
    log1 = torch.empty((n, m.vocab), dtype=torch.bfloat16, device="cuda")
    _multi_one_by_one(m, d_m, n, fp8)
    L.call("granite4_kernel_rmsnorm", m.steps.hidden, m.final_norm, m.eps, n, m.H, hid1)
    e = _epi(m.lm_scale, m.lm_scale, m.lm_scale, 0, 0, log1, m.vocab)
    L.call("granite4_prefill_gemm", L.GEMM_BF16, hid1, m.H, m.lm_head, n, m.vocab, m.H,
           L._c.byref(e), None, 0)
    want_arena = m.host_arenas()
    want = (host(hid1).copy(), host(log1).copy())
    m.restore(start)
    hid2 = torch.empty_like(hid1)
    log2 = torch.empty_like(log1)
    m.steps.multi(d_m, n, L.OPS_FP8 if fp8 else L.OPS_BF16, hid2, log2)
    np.testing.assert_array_equal(host(hid2), want[0])
    np.testing.assert_array_equal(host(log2), want[1])
    for a, b in zip(m.host_arenas(), want_arena):
        for x, y in zip(a, b):
            np.testing.assert_array_equal(x, y)
    # the oracle's composition, from the starting arenas
    c, s = host(m.cos), host(m.sin)
    tok = np.array([toks[i][pos[i]] for i in range(n)], np.int32)
    x = ol.embed_rows(tok, host(m.emb), m.emb_mult)
    arenas = [[host(t).reshape(-1).copy() for t in a] for a in start]
    arows = np.array([pts[i][pos[i]] for i in range(n)], np.int32)

    def attention(li, ly, q, k, v, ar):
        ck, cv, ks, vs = ar
        q_rot = ol.rope_append(q, k, v, c, s, pos, arows, 8, 128, m.stride, m.Hk,
                               k_round_bf16=True, cache_k=ck, cache_v=cv, k_scale=ks,
                               v_scale=vs)[0]
        return ol.attn_split(q_rot, ck, cv, ks, vs, 8, 128, m.stride, pos, pts=pts,
                             scale=m.att, Hk=m.Hk, max_len=m.split_len)
    hid, logits = oracle_layers(m, x, fp8, arenas, attention)
    _close(host(hid2), hid, "final-normed hidden", fp8)
    _close(host(log2), logits, "logits", fp8)


def test_decode_step_multi_graph_replay_and_high_positions():
    """Config 2's position range: 8 sessions at positions in [0, 65536)
    (FP8 ops, int8 KV). Captured once, replayed at p and p + 1 (the
    descriptor's positions advanced on the device between replays); each
    replay equals the eager step, arenas included."""
    note("decode step multi graph, positions up to 65536")
    n, stride = 8, 4096
    m = Model(4096, 12800, 32, 8, 1000, 2, 8, 128, stride, 8, 0x3B1)
    d_m, pos, pts, toks, keep = _multi_rows(m, n, 65536, 0x3B2)
    assert pos.max() >= 32768
    hid = torch.empty((n, m.H), dtype=torch.bfloat16, device="cuda")
    lg = torch.empty((n, m.vocab), dtype=torch.bfloat16, device="cuda")
    start = m.arenas()
    base = d_m.clone()
    pos_field = d_m[4:4 + 4 * n].view(torch.int32)
    want = []
    for i in range(2):
        d_m.copy_(base)
        pos_field.add_(i)
        m.steps.multi(d_m, n, L.OPS_FP8, hid, lg)
        torch.cuda.synchronize()
        want.append((host(hid).copy(), host(lg).copy(), m.host_arenas()))
    m.restore(start)
    d_m.copy_(base)
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    L.use_stream(s)
    try:
        with torch.cuda.graph(g, stream=s):
            m.steps.multi(d_m, n, L.OPS_FP8, hid, lg)
    finally:
        L.use_stream()
    torch.cuda.synchronize()
    m.restore(start)
    for i in range(2):
        d_m.copy_(base)
        pos_field.add_(i)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(host(hid), want[i][0])
        np.testing.assert_array_equal(host(lg), want[i][1])
        for a, b in zip(m.host_arenas(), want[i][2]):
            for x, y in zip(a, b):
                np.testing.assert_array_equal(x, y)
    assert L.fp8_sync_status(m.steps.fp8_work) == 0


def test_multi_embed_reference_kernel():
    """granite4_multi_embed (embed_multi_v8_kernel): each row the token of
    its session at its position, bit-exact against the oracle; a token
    outside the vocabulary gives a zero row."""
    note("multi embed")
    n, H, vocab = 5, 4096, 777
    emb = ol.normal_bf16(0x3C1, 0.0, 0.05, vocab * H).reshape(vocab, H)
    rs = np.random.default_rng(0x3C2)
    toks = [rs.integers(0, vocab, 300).astype(np.int32) for _ in range(n)]
    pos = rs.integers(0, 300, n).astype(np.int32)
    toks[3][pos[3]] = vocab + 5
    keep = [dev(t) for t in toks]
    M = L.multi_rows_struct()()
    M.n = n
    for i in range(n):
        M.pos[i] = int(pos[i])
        M.tok[i] = keep[i].data_ptr()
    d_m = torch.from_numpy(np.frombuffer(bytes(M), np.uint8).copy()).cuda()
    out = torch.empty((n, H), dtype=torch.int16, device="cuda")
    L.call("granite4_multi_embed", d_m, n, dev(emb), vocab, H, 1.5, out)
    got = host(out).view(np.uint16)
    tok = np.array([toks[i][pos[i]] for i in range(n)], np.int32)
    tok_ok = np.where(tok < vocab, tok, 0)
    want = ol.embed_rows(tok_ok, emb, 1.5)
    want[3] = 0
    np.testing.assert_array_equal(got, want)


# ----------------------------------------------------------------------------- prefill chunk
def _prefill_one_by_one(m, d_tok, start, T, d_pt, fp8):
    st = m.steps
    nq, nk = m.Hq * 128, m.Hk * 128
    nqkv = nq + 2 * nk
    grp = 128 if m.bits == 16 else m.group

    def first():
        L.call("granite4_embed_rows", d_tok[start:], T, m.emb, m.vocab, m.H, m.emb_mult, st.hidden)

    def attention(ly, gemm):
        for W, N, col, sc in ((ly["wq"], nq, 0, ly["sq"]), (ly["wk"], nk, nq, ly["sk"]),
                              (ly["wv"], nk, nq + nk, ly["sv"])):
            gemm(L.GEMM_BF16, W, N, m.H, _epi(sc, sc, sc, 0, 0, st.qkv[:, col:], nqkv))
        L.call("granite4_rope_append", st.qkv, nqkv, st.qkv[:, nq:], nqkv, st.qkv[:, nq + nk:],
               nqkv, m.cos, m.sin, m.cos.shape[0], T, m.Hq, m.Hk, 128, start, None, d_pt, None,
               m.bits, grp, 0, 1, st.q_rot, nq, ly["cache_k"], ly["cache_v"], ly["k_scale"],
               ly["v_scale"], m.stride)
        L.call("granite4_prefill_attn", st.q_rot, T, m.Hq, m.Hk, 128, m.att, ly["cache_k"],
               ly["cache_v"], ly["k_scale"], ly["v_scale"], m.bits, grp, m.stride, start, d_pt, 0,
               st.attn)
    one_by_one(m, T, fp8, first, attention)


@pytest.mark.parametrize("ops,bits,group", [("bf16", 8, 128), ("fp8", 8, 128), ("fp8", 5, 32),
                                            ("bf16", 16, 128), ("fp8", 4, 64)])
def test_prefill_layers_matches_one_by_one_and_oracle(ops, bits, group):
    """A 100-token chunk at position 37 of a sequence paged through a random
    row table (small model: H 1024, I 2048, 8 query and 2 KV heads, 2
    layers): bit for bit the entry points one by one (q|k|v as three GEMMs,
    the weights stored apart), then the oracle's composition."""
    fp8 = ops == "fp8"
    note(f"prefill layers ops={ops} bits={bits} group={group}")
    T, start, stride = 100, 37, 512
    m = Model(1024, 2048, 8, 2, 300, 2, bits, group, stride, 128, 0x3D1 + bits + fp8,
              max_pos=1024, split_qkv=True)
    rs = np.random.default_rng(0x3D2)
    pt = ol.row_table(rs.permutation(stride // 16).astype(np.int32), stride)
    toks = rs.integers(0, m.vocab, 256).astype(np.int32)
    d_tok, d_pt = dev(toks), dev(pt)
    start_arena = m.arenas()
    hid1 = torch.empty((T, m.H), dtype=torch.bfloat16, device="cuda")
    log1 = torch.empty((T, m.vocab), dtype=torch.bfloat16, device="cuda")
    _prefill_one_by_one(m, d_tok, start, T, d_pt, fp8)
    L.call("granite4_kernel_rmsnorm", m.steps.hidden, m.final_norm, m.eps, T, m.H, hid1)
    e = _epi(m.lm_scale, m.lm_scale, m.lm_scale, 0, 0, log1, m.vocab)
    L.call("granite4_prefill_gemm", L.GEMM_BF16, hid1, m.H, m.lm_head, T, m.vocab, m.H,
           L._c.byref(e), None, 0)
    want = (host(hid1).copy(), host(log1).copy(), m.host_arenas())
    m.restore(start_arena)
    hid2 = torch.empty_like(hid1)
    log2 = torch.empty_like(log1)
    m.steps.prefill(d_tok, start, T, d_pt, L.OPS_FP8 if fp8 else L.OPS_BF16, hid2, log2)
    np.testing.assert_array_equal(host(hid2), want[0])
    np.testing.assert_array_equal(host(log2), want[1])
    for a, b in zip(m.host_arenas(), want[2]):
        for x, y in zip(a, b):
            np.testing.assert_array_equal(x, y)
    # the oracle's composition
    c, s = host(m.cos), host(m.sin)
    x = ol.embed_rows(toks[start:start + T], host(m.emb), m.emb_mult)
    arenas = [[host(t).reshape(-1).copy() for t in a] for a in start_arena]
    positions = np.arange(start, start + T)

    def attention(li, ly, q, k, v, ar):
        ck, cv = ar[0], ar[1]
        ks = ar[2] if bits != 16 else np.zeros(1, np.float32)
        vs = ar[3] if bits != 16 else np.zeros(1, np.float32)
        q_rot = ol.rope_append(q, k, v, c, s, positions, pt[positions], bits, group, m.stride,
                               m.Hk, k_round_bf16=False, cache_k=ck, cache_v=cv, k_scale=ks,
                               v_scale=vs)[0]
        return ol.prefill_attn(q_rot, ck, cv, None if bits == 16 else ks,
                               None if bits == 16 else vs, bits, group, m.stride, start, pt=pt,
                               scale=m.att, Hk=m.Hk)
    hid, logits = oracle_layers(m, x, fp8, arenas, attention)
    _close(host(hid2), hid, "final-normed hidden", fp8)
    _close(host(log2), logits, "logits", fp8)


def test_prefill_layers_8b_shape_matches_one_by_one():
    """BASELINE config 3's shape through the whole sequence: 512 tokens of
    the 8B model (2 layers, FP8 ops, int8 KV in fresh pages): bit for bit the
    entry points one by one, with q|k|v and gate|up each one weight block
    (one GEMM each)."""
    note("prefill layers 8B shape T=512")
    T, stride = 512, 1024
    m = Model(4096, 12800, 32, 8, 1000, 2, 8, 128, stride, T, 0x3E1)
    toks = np.random.default_rng(0x3E2).integers(0, m.vocab, T).astype(np.int32)
    d_tok = dev(toks)
    start_arena = m.arenas()
    st = m.steps
    nq, nk = m.Hq * 128, m.Hk * 128
    nqkv = nq + 2 * nk

    def first():
        L.call("granite4_embed_rows", d_tok, T, m.emb, m.vocab, m.H, m.emb_mult, st.hidden)

    def attention(ly, gemm):
        gemm(L.GEMM_BF16, ly["wq"], nqkv, m.H, _epi(ly["sq"], ly["sk"], ly["sv"], nq, nq + nk,
                                                     st.qkv, nqkv))
        L.call("granite4_rope_append", st.qkv, nqkv, st.qkv[:, nq:], nqkv, st.qkv[:, nq + nk:],
               nqkv, m.cos, m.sin, m.cos.shape[0], T, m.Hq, m.Hk, 128, 0, None, None, None, 8,
               128, 0, 1, st.q_rot, nq, ly["cache_k"], ly["cache_v"], ly["k_scale"],
               ly["v_scale"], m.stride)
        L.call("granite4_prefill_attn", st.q_rot, T, m.Hq, m.Hk, 128, m.att, ly["cache_k"],
               ly["cache_v"], ly["k_scale"], ly["v_scale"], 8, 128, m.stride, 0, None, 0,
               st.attn)
    one_by_one(m, T, True, first, attention)
    hid1 = torch.empty((T, m.H), dtype=torch.bfloat16, device="cuda")
    L.call("granite4_kernel_rmsnorm", st.hidden, m.final_norm, m.eps, T, m.H, hid1)
    want = (host(hid1).copy(), m.host_arenas())
    m.restore(start_arena)
    hid2 = torch.empty_like(hid1)
    st.prefill(d_tok, 0, T, None, L.OPS_FP8, hid2)
    np.testing.assert_array_equal(host(hid2), want[0])
    for a, b in zip(m.host_arenas(), want[1]):
        for x, y in zip(a, b):
            np.testing.assert_array_equal(x, y)
    assert L.fp8_sync_status(st.fp8_work) == 0


def test_layer_steps_reject_bad_arguments_before_launching():
    """A bad argument (a NaN scale in the last layer, a missing FP8 buffer, a
    chunk past the table) is rejected before any launch: the arenas are
    untouched."""
    note("layer steps reject")
    m = Model(1024, 2048, 8, 2, 300, 2, 8, 128, 512, 32, 0x3F1, max_pos=1024)
    toks = dev(np.zeros(64, np.int32))
    before = m.host_arenas()
    m.steps._arr[1].sd = float("nan")
    with pytest.raises(L.Granite4Error):
        m.steps.prefill(toks, 0, 16, None, L.OPS_BF16)
    m.steps._arr[1].sd = 1 / 112
    with pytest.raises(L.Granite4Error):
        m.steps.prefill(toks, 1020, 16, None, L.OPS_BF16)
    with pytest.raises(L.Granite4Error):
        m.steps.prefill(toks, 0, 33, None, L.OPS_BF16)  # more rows than the buffers hold
    torch.cuda.synchronize()
    for a, b in zip(m.host_arenas(), before):
        for x, y in zip(a, b):
            np.testing.assert_array_equal(x, y)
