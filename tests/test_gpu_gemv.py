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
