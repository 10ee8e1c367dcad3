"""GPU parity of the batch-1 decode GEMVs (gemv.hip) and their fused
prologue / epilogues.

The plain GEMVs are held to the reference's GEMM bar against g4o_gemv_fp8w
(exact products, double sum): within 2 bf16 ulp of the rounded oracle value,
or within the f32 sum's error bound K * 2^-24 * scale * sum |a w| where the
sum cancels. The fused forms are checked bit for bit against the unfused GPU
composition they replace (granite4_kernel_rmsnorm then the GEMV: the same
sums in the same order), and against the oracle composition within the bar.
"""
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


def dev(a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a).cuda()


def host(t):
    torch.cuda.synchronize()
    a = t.cpu().numpy()
    return a.view(np.uint16) if a.dtype == np.int16 else a


def empty16(n):
    return torch.empty(n, dtype=torch.int16, device="cuda")


def ulp_diff(a, b):
    ai = a.astype(np.int32)
    bi = b.astype(np.int32)
    ai = np.where(ai & 0x8000, 0x8000 - ai, ai)
    bi = np.where(bi & 0x8000, 0x8000 - bi, bi)
    return np.abs(ai - bi)


def bound(a, W, scale):
    """K * 2^-24 * scale * sum |a w| per output row."""
    return ol.gemv_fp8w(a & 0x7FFF, W & 0x7F, abs(scale)).astype(np.float64) * W.shape[1] * 2.0 ** -24


def check_bf16(got, y, bnd):
    want = np.vectorize(ol.lib.g4o_f32_to_bf16, otypes=[np.uint16])(y)
    d = ulp_diff(got, want)
    err = np.abs(ol.bf16_to_f32(got).astype(np.float64) - y)
    bad = (d > 2) & (err > bnd + np.abs(y) * 2.0 ** -7)
    print(f"  exact {(d == 0).mean():.4f}, max ulp {d.max()}", flush=True)
    assert not bad.any(), np.argwhere(bad)[:5]


@pytest.mark.parametrize("N,K", [(100, 4096), (4096, 4096), (4096, 12800), (16, 64), (40, 2112)])
def test_gemv_plain(N, K):
    print(f"gemv N={N} K={K}", flush=True)
    a = ol.normal_bf16(0xA1 + K, 0.0, 1.0, K)
    W = ol.fp8_codes(0xA2 + N, (N, K), std=0.5)
    out = empty16(N)
    L.call("granite4_gemv_fp8w", dev(a), dev(W), 0.0071, N, K, out)
    check_bf16(host(out), ol.gemv_fp8w(a, W, 0.0071), bound(a, W, 0.0071))


def test_gemv_residual_in_place():
    N, K = 4096, 12800
    a = ol.normal_bf16(0xA3, 0.0, 1.0, K)
    W = ol.fp8_codes(0xA4, (N, K), std=0.5)
    res = ol.normal_bf16(0xA5, 0.0, 1.0, N)
    hid = dev(res)
    L.call("granite4_gemv_fp8w_resid", dev(a), dev(W), 0.003, hid, 0.22, N, K, hid)
    y = ol.gemv_fp8w(a, W, 0.003)
    want = (ol.bf16_to_f32(res) + np.float32(0.22) * y).astype(np.float32)
    check_bf16(host(hid), want, bound(a, W, 0.003) * 0.22)


def test_gemv_qkv_and_fused_norm():
    """q|k|v in one launch, then the same with the attention RMSNorm fused in:
    identical to granite4_kernel_rmsnorm followed by the qkv GEMV."""
    K, Nq, Nk, Nv = 4096, 4096, 1024, 1024
    x = ol.normal_bf16(0xA6, 0.0, 1.0, K)
    gamma = ol.normal_bf16(0xA7, 1.0, 0.1, K)
    Ws = [ol.fp8_codes(0xA8 + i, (n, K), std=0.5) for i, n in enumerate((Nq, Nk, Nv))]
    sc = (0.01, 0.02, 0.03)
    dx, dg = dev(x), dev(gamma)
    dW = [dev(w) for w in Ws]
    normed = empty16(K)
    L.call("granite4_kernel_rmsnorm", dx, dg, 1e-5, 1, K, normed)
    outs = [empty16(n) for n in (Nq, Nk, Nv)]
    L.call("granite4_gemv_qkv", normed, *dW, *sc, Nq, Nk, Nv, K, *outs)
    fused = [empty16(n) for n in (Nq, Nk, Nv)]
    L.call("granite4_gemv_rmsnorm_qkv", dx, dg, 1e-5, *dW, *sc, Nq, Nk, Nv, K, *fused)
    nh = host(normed)
    assert ulp_diff(nh, ol.rmsnorm(x.reshape(1, K), gamma, 1e-5)[0]).max() <= 1
    for w, s, o, f in zip(Ws, sc, outs, fused):
        np.testing.assert_array_equal(host(f), host(o))
        check_bf16(host(o), ol.gemv_fp8w(nh, w, s), bound(nh, w, s))


@pytest.mark.parametrize("N,K", [(12800, 4096), (200, 4096)])
def test_silu_gate_up_and_fused_norm(N, K):
    """granite4_kernel_silu_gate_up (the reference's signature) against the
    oracle GEMVs + the reference's f32 SwiGLU, and the norm-fused form
    identical to granite4_kernel_rmsnorm followed by it."""
    print(f"silu_gate_up N={N} K={K}", flush=True)
    x = ol.normal_bf16(0xB1, 0.0, 1.0, K)
    gamma = ol.normal_bf16(0xB2, 1.0, 0.1, K)
    Wg = ol.fp8_codes(0xB3, (N, K), std=0.5)
    Wu = ol.fp8_codes(0xB4, (N, K), std=0.5)
    sg, su = 0.006, 0.009
    dx, dg, dwg, dwu = dev(x), dev(gamma), dev(Wg), dev(Wu)
    normed = empty16(K)
    L.call("granite4_kernel_rmsnorm", dx, dg, 1e-5, 1, K, normed)
    act = empty16(N)
    L.call("granite4_kernel_silu_gate_up", dwg, dwu, normed, sg, su, N, K, act)
    act2 = empty16(N)
    L.call("granite4_gemv_rmsnorm_silu_gate_up", dx, dg, 1e-5, dwg, dwu, sg, su, N, K, act2)
    np.testing.assert_array_equal(host(act2), host(act))
    nh = host(normed)
    g, u = ol.gemv_fp8w(nh, Wg, sg), ol.gemv_fp8w(nh, Wu, su)
    want = ol.silu_mul_f32(np.concatenate([g, u]).reshape(1, 2 * N))[0]
    got = host(act)
    d = ulp_diff(got, want)
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    sig = 1.0 / (1.0 + np.exp(-g64))
    tol = (np.abs(sig * u64) * bound(nh, Wg, sg) * 1.2 + np.abs(g64 * sig) * bound(nh, Wu, su)
           + np.abs(ol.bf16_to_f32(want)) * 2.0 ** -7)
    err = np.abs(ol.bf16_to_f32(got).astype(np.float64) - ol.bf16_to_f32(want))
    print(f"  act exact {(d == 0).mean():.4f}, max ulp {d.max()}", flush=True)
    assert not ((d > 2) & (err > tol)).any()


def test_gemv_invalid_arguments():
    a = torch.zeros(100, dtype=torch.int16, device="cuda")
    W = torch.zeros((4, 100), dtype=torch.uint8, device="cuda")
    with pytest.raises(L.Granite4Error):
        L.call("granite4_gemv_fp8w", a, W, 1.0, 4, 100, empty16(4))  # K % 64 != 0


@pytest.mark.parametrize("bits,group", [(16, 128), (8, 128), (5, 32)])
def test_rmsnorm_qkv_rope_append_fused(bits, group):
    """RMSNorm + q|k|v GEMV + RoPE + KV append in one launch: q_rot, the pool
    row and its scales bit-identical to granite4_gemv_rmsnorm_qkv followed by
    granite4_rope_append_at_pos (same position, same page table)."""
    print(f"qkv rope append fused bits={bits} group={group}", flush=True)
    K, Hq, Hk, D = 4096, 32, 8, 128
    x = dev(ol.normal_bf16(0xC1, 0.0, 1.0, K))
    gamma = dev(ol.normal_bf16(0xC2, 1.0, 0.1, K))
    Wq, Wk, Wv = (dev(ol.fp8_codes(0xC3 + i, (n, K), std=0.5)) for i, n in
                  enumerate((Hq * D, Hk * D, Hk * D)))
    sc = (0.004, 0.005, 0.006)
    cos_t, sin_t = ol.rope_tables(1e7, D, 8192)
    dcos, dsin = dev(cos_t), dev(sin_t)
    stride = 256
    pos = dev(np.array([5000], np.int32))
    pt = dev(np.random.default_rng(3).permutation(8192).astype(np.int32) % stride)
    outs = []
    for fused in (False, True):
        arena = L.KvArena(bits, Hk, stride, group=group)
        q_rot = empty16(Hq * D)
        if fused:
            L.call("granite4_gemv_rmsnorm_qkv_rope_append", x, gamma, 1e-5, Wq, Wk, Wv, *sc, dcos,
                   dsin, 8192, pos, pt, Hq, Hk, bits, group, q_rot, arena.k, arena.v,
                   arena.k_scale, arena.v_scale, stride)
        else:
            q, k, v = empty16(Hq * D), empty16(Hk * D), empty16(Hk * D)
            L.call("granite4_gemv_rmsnorm_qkv", x, gamma, 1e-5, Wq, Wk, Wv, *sc, Hq * D, Hk * D,
                   Hk * D, K, q, k, v)
            L.call("granite4_rope_append_at_pos", q, k, v, dcos, dsin, 8192, pos, pt, Hq, Hk, D,
                   bits, group, q_rot, arena.k, arena.v, arena.k_scale, arena.v_scale, stride)
        outs.append([host(q_rot), host(arena.k), host(arena.v), host(arena.k_scale),
                     host(arena.v_scale)])
    for a, b in zip(*outs):
        np.testing.assert_array_equal(a, b)
    row = int(host(pt)[5000])
    assert np.any(outs[1][1].reshape(Hk, stride, -1)[:, row] != 0)  # the row was written


def _fill_pool(arena, seed):
    """Seeded pool contents in the format's range: bf16 N(0,1) values, or
    random codes with positive scales."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    if arena.bits == 16:
        vals = torch.randn(arena.k.numel() // 2, generator=g, device="cuda").to(torch.bfloat16)
        arena.k.copy_(vals.view(torch.uint8).view(arena.k.shape))
        vals = torch.randn(arena.v.numel() // 2, generator=g, device="cuda").to(torch.bfloat16)
        arena.v.copy_(vals.view(torch.uint8).view(arena.v.shape))
        return
    arena.k.copy_(torch.randint(0, 256, arena.k.shape, generator=g, device="cuda").to(torch.uint8))
    arena.v.copy_(torch.randint(0, 256, arena.v.shape, generator=g, device="cuda").to(torch.uint8))
    if arena.bits == 8:  # int8 codes stay within +-127
        arena.k[arena.k == 0x80] = 0x81
        arena.v[arena.v == 0x80] = 0x81
    arena.k_scale.copy_(torch.rand(arena.k_scale.shape, generator=g, device="cuda") * 0.02)
    arena.v_scale.copy_(torch.rand(arena.v_scale.shape, generator=g, device="cuda") * 0.02)


@pytest.mark.parametrize("pos_v,max_pos", [(5000, 8192), (4095, 8192), (5000, 4096)])
@pytest.mark.parametrize("bits,group", [(16, 128), (8, 128), (5, 32), (4, 64)])
def test_rmsnorm_qkv_rope_then_append_attention(bits, group, pos_v, max_pos):
    """The decode step's q|k|v side in two launches: granite4_gemv_rmsnorm_qkv_rope
    (RoPE in the GEMV epilogue) then granite4_attn_decode_append_rotated (the
    append in the attention). q_rot, the attention output and the whole pool
    bit-identical to granite4_gemv_rmsnorm_qkv + granite4_rope_append_at_pos +
    granite4_attn_paged; also at a position past the RoPE table (q_rot and K
    not written, V appended)."""
    print(f"qkv rope + append attention bits={bits} group={group} pos={pos_v} "
          f"max_pos={max_pos}", flush=True)
    K, Hq, Hk, D = 4096, 32, 8, 128
    x = dev(ol.normal_bf16(0xD1, 0.0, 1.0, K))
    gamma = dev(ol.normal_bf16(0xD2, 1.0, 0.1, K))
    Wq, Wk, Wv = (dev(ol.fp8_codes(0xD3 + i, (n, K), std=0.5)) for i, n in
                  enumerate((Hq * D, Hk * D, Hk * D)))
    sc = (0.004, 0.005, 0.006)
    cos_t, sin_t = ol.rope_tables(1e7, D, max_pos)
    dcos, dsin = dev(cos_t), dev(sin_t)
    stride = 8192
    pos = dev(np.array([pos_v], np.int32))
    pt = dev(np.random.default_rng(7).permutation(stride).astype(np.int32))
    scratch = torch.empty(L.call_size("granite4_attn_split_scratch_bytes", Hq, 1, stride),
                          dtype=torch.uint8, device="cuda")
    outs = []
    for fused in (False, True):
        arena = L.KvArena(bits, Hk, stride, group=group)
        _fill_pool(arena, 0xD9)
        pool = [arena.k, arena.v, arena.k_scale, arena.v_scale]
        q_rot = torch.zeros(Hq * D, dtype=torch.int16, device="cuda")
        out = empty16(Hq * D)
        if fused:
            k_rot, v = empty16(Hk * D), empty16(Hk * D)
            L.call("granite4_gemv_rmsnorm_qkv_rope", x, gamma, 1e-5, Wq, Wk, Wv, *sc, dcos, dsin,
                   max_pos, pos, Hq, Hk, K, q_rot, k_rot, v)
            L.call("granite4_attn_decode_append_rotated", q_rot, k_rot, v, max_pos, pos, pt, Hq,
                   Hk, 1.0 / 16, *pool, bits, group, stride, scratch, out)
        else:
            q, k, v = empty16(Hq * D), empty16(Hk * D), empty16(Hk * D)
            L.call("granite4_gemv_rmsnorm_qkv", x, gamma, 1e-5, Wq, Wk, Wv, *sc, Hq * D, Hk * D,
                   Hk * D, K, q, k, v)
            L.call("granite4_rope_append_at_pos", q, k, v, dcos, dsin, max_pos, pos, pt, Hq, Hk, D,
                   bits, group, q_rot, *pool, stride)
            L.call("granite4_attn_paged", q_rot, 1, Hq, Hk, D, 1.0 / 16, *pool, bits, group,
                   stride, 0, pos, pt, None, None, 0, 0, scratch, out)
        outs.append([host(q_rot), host(out)] + [host(t) for t in pool])
    for a, b in zip(*outs):
        np.testing.assert_array_equal(a, b)
    if pos_v < max_pos:
        assert np.any(outs[1][0] != 0)  # q_rot was written


@pytest.mark.parametrize("mult,tok_kind", [(12.0, "valid"), (1.0, "valid"), (0.37, "invalid"),
                                           (12.0, "negative_pos")])
def test_embed_rmsnorm_qkv_rope_fused(mult, tok_kind):
    """The first layer's q|k|v launch with the embedding as its prologue
    (granite4_gemv_embed_rmsnorm_qkv_rope): hidden, q_rot, k_rot and v
    bit-identical to granite4_embed_at_pos then granite4_gemv_rmsnorm_qkv_rope,
    for embedding multipliers 12 and 1, a token outside the vocabulary (a zero
    row: the norm of zeros gives zero outputs) and a negative position (no
    token read; q_rot / k_rot not written, as the rotation skips positions
    outside the table)."""
    print(f"embed + rmsnorm qkv rope mult={mult} {tok_kind}", flush=True)
    K, Hq, Hk, D, vocab = 4096, 32, 8, 128, 5000
    emb = dev(ol.normal_bf16(0xE1, 0.0, 0.05, vocab * K).reshape(vocab, K))
    gamma = dev(ol.normal_bf16(0xE2, 1.0, 0.1, K))
    Wq, Wk, Wv = (dev(ol.fp8_codes(0xE3 + i, (n, K), std=0.5)) for i, n in
                  enumerate((Hq * D, Hk * D, Hk * D)))
    sc = (0.004, 0.005, 0.006)
    cos_t, sin_t = ol.rope_tables(1e7, D, 8192)
    dcos, dsin = dev(cos_t), dev(sin_t)
    toks = np.random.default_rng(3).integers(0, vocab, 8192).astype(np.int32)
    p = 4321 if tok_kind != "negative_pos" else -3
    if tok_kind == "invalid":
        toks[p] = vocab + 7
    d_tok = dev(toks)
    pos = dev(np.array([p], np.int32))
    outs = []
    for fused in (False, True):
        hid = torch.full((K,), 0x1234, dtype=torch.int16, device="cuda")
        q_rot = torch.zeros(Hq * D, dtype=torch.int16, device="cuda")
        k_rot = torch.zeros(Hk * D, dtype=torch.int16, device="cuda")
        v = empty16(Hk * D)
        if fused:
            L.call("granite4_gemv_embed_rmsnorm_qkv_rope", d_tok, emb, vocab, mult, hid, gamma,
                   1e-5, Wq, Wk, Wv, *sc, dcos, dsin, 8192, pos, Hq, Hk, K, q_rot, k_rot, v)
        else:
            if p >= 0:
                L.call("granite4_embed_at_pos", d_tok, pos, emb, vocab, K, mult, hid)
            else:
                hid.zero_()  # the fused form reads no token at a negative position
            L.call("granite4_gemv_rmsnorm_qkv_rope", hid, gamma, 1e-5, Wq, Wk, Wv, *sc, dcos, dsin,
                   8192, pos, Hq, Hk, K, q_rot, k_rot, v)
        outs.append([host(t) for t in (hid, q_rot, k_rot, v)])
    for a, b in zip(*outs):
        np.testing.assert_array_equal(a, b)
    if tok_kind == "valid":
        want = np.vectorize(ol.lib.g4o_f32_to_bf16, otypes=[np.uint16])(
            np.float32(mult) * ol.bf16_to_f32(host(emb)[toks[p]]))
        np.testing.assert_array_equal(outs[1][0], want)
        assert np.any(outs[1][1] != 0)
