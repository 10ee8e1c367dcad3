"""GPU parity of granite4_prefill_gemm, the reference's own prefill GEMM
(prefill_gemm.h:34-39: bf16 A x fp8 e4m3 W with the kBf16 / kF32 / kResidual
epilogues and per-segment weight scales) against the oracle's g4o_gemm_bf16w
(exact products, double accumulation).

Bar, as the reference's GEMM test (test_kernels.cu:1685-1719): each bf16
output within 2 bf16 ulp of the oracle value rounded to bf16, except where
the sum cancels below the f32 accumulation's reach: there within
K * 2^-24 * s * sum_k |a_k w_k| (the f32 sum's error bound; the matrix cores
add in their own order). f32 outputs are held to that bound everywhere.
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


def dev(a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a).cuda()


def host(t):
    torch.cuda.synchronize()
    if t.dtype == torch.bfloat16:
        t = t.view(torch.int16)
    a = t.cpu().numpy()
    return a.view(np.uint16) if a.dtype == np.int16 else a


def ulp_diff(a, b):
    ai = a.astype(np.int32)
    bi = b.astype(np.int32)
    ai = np.where(ai & 0x8000, 0x8000 - ai, ai)
    bi = np.where(bi & 0x8000, 0x8000 - bi, bi)
    return np.abs(ai - bi)


def bound(A, W, scales, segs):
    """K * 2^-24 * s * sum_k |a_k w_k| per output (the f32 sum's error bound)."""
    K = A.shape[1]
    return ol.gemm_bf16w(A & 0x7FFF, W & 0x7F, scales, segs).astype(np.float64) * K * 2.0 ** -24


def check_bf16(got, y, bnd):
    want = ol.f32_to_bf16(y)
    d = ulp_diff(got, want)
    err = np.abs(ol.bf16_to_f32(got).astype(np.float64) - y.astype(np.float64))
    bad = (d > 2) & (err > bnd + np.abs(y) * 2.0 ** -7)
    assert not bad.any(), (np.argwhere(bad)[:5], d.max())
    return (d == 0).mean()


def inputs(M, N, K, seed):
    A = ol.normal_bf16(seed, 0.0, 1.0, M * K).reshape(M, K)
    W = ol.fp8_codes(seed + 1, (N, K), std=0.5)
    return A, W


@pytest.mark.parametrize("M,N,K", [(1, 8, 32), (37, 40, 96), (130, 264, 256), (300, 520, 512),
                                   (64, 128, 4128), (8, 136, 4096), (16, 40, 96), (3, 520, 12800)])
def test_prefill_gemm_bf16_out(M, N, K):
    note(f"prefill_gemm bf16 M={M} N={N} K={K}")
    A, W = inputs(M, N, K, 0x81 + M)
    sc, segs = (0.02, 0.01, 0.005), (N // 4, N // 2)
    out = L.prefill_gemm(dev(A).view(torch.bfloat16), dev(W), L.GEMM_BF16, scales=sc, segs=segs)
    y = ol.gemm_bf16w(A, W, sc, segs)
    exact = check_bf16(host(out), y, bound(A, W, sc, segs))
    note(f"  bit-exact fraction {exact:.4f}")


@pytest.mark.parametrize("M,N,K", [(33, 72, 160), (256, 384, 1024), (8, 72, 160)])
def test_prefill_gemm_f32_out(M, N, K):
    note(f"prefill_gemm f32 M={M} N={N} K={K}")
    A, W = inputs(M, N, K, 0x91 + M)
    sc = (0.03, 0.03, 0.03)
    out = L.prefill_gemm(dev(A).view(torch.bfloat16), dev(W), L.GEMM_F32, scales=sc)
    y = ol.gemm_bf16w(A, W, sc).astype(np.float64)
    err = np.abs(host(out).astype(np.float64) - y)
    assert np.all(err <= bound(A, W, sc, None) + np.abs(y) * 2.0 ** -23)


# 200 x 256: 4 tiles, the residual prefetched at each tile's start; 2100 x
# 4096: 544 tiles, more than the 512 workgroups resident at two per CU, so the
# form that loads the residual after the K loop runs.
@pytest.mark.parametrize("M,N,K", [(200, 256, 512), (2100, 4096, 128), (8, 4096, 4096)])
def test_prefill_gemm_residual_in_place(M, N, K):
    """kResidual, the O / down projection: hidden = bf16(hidden + rs * y), in place."""
    note(f"prefill_gemm residual M={M} N={N} K={K}")
    A, W = inputs(M, N, K, 0xA1)
    res = ol.normal_bf16(0xA3, 0.0, 1.0, M * N).reshape(M, N)
    sc = (0.02, 0.02, 0.02)
    hid = dev(res).view(torch.bfloat16)
    L.prefill_gemm(dev(A).view(torch.bfloat16), dev(W), L.GEMM_RESIDUAL, scales=sc, out=hid,
                   residual=hid, resid_scale=0.22)
    y = ol.gemm_bf16w(A, W, sc)
    want_f = ol.bf16_to_f32(res).astype(np.float32) + np.float32(0.22) * y
    bnd = 0.22 * bound(A, W, sc, None)
    got = host(hid)
    d = ulp_diff(got, ol.f32_to_bf16(want_f))
    err = np.abs(ol.bf16_to_f32(got).astype(np.float64) - want_f.astype(np.float64))
    assert not ((d > 2) & (err > bnd + np.abs(want_f) * 2.0 ** -7)).any()


@pytest.mark.parametrize("M", [21, 7])
@pytest.mark.parametrize("N,ldc", [(38, 38), (38, 40), (18, 22)])
def test_prefill_gemm_even_widths_and_pitches(N, ldc, M):
    """The reference accepts any even N and ldc: outputs not 16-byte aligned
    per row are written element by element, columns past N untouched."""
    note(f"prefill_gemm N={N} ldc={ldc} M={M}")
    K = 64
    A, W = inputs(M, N, K, 0xB1 + N + ldc)
    full = torch.full((M, ldc), 0x7E7E, dtype=torch.int16, device="cuda")
    ep = L.GemmEpilogue(0.05, 0.05, 0.05, N, N, full.data_ptr(), None, None, 1.0, ldc)
    L.call("granite4_prefill_gemm", L.GEMM_BF16, dev(A), K, dev(W), M, N, K, ep, None, 0)
    got = host(full)
    y = ol.gemm_bf16w(A, W, (0.05, 0.05, 0.05))
    check_bf16(got[:, :N], y, bound(A, W, (0.05, 0.05, 0.05), None))
    assert (got[:, N:] == 0x7E7E).all()


def test_prefill_gemm_qkv_shape_at_T512_sampled_rows():
    """The q|k|v projection of config 3 (512 x 6144 x 4096, three weight
    segments), checked on 24 sampled rows against the oracle."""
    note("prefill_gemm qkv T=512")
    M, N, K = 512, 6144, 4096
    A, W = inputs(M, N, K, 0xC1)
    sc, segs = (1 / 64, 1 / 48, 1 / 32), (4096, 5120)
    out = host(L.prefill_gemm(dev(A).view(torch.bfloat16), dev(W), L.GEMM_BF16, scales=sc,
                              segs=segs))
    rows = np.sort(np.random.default_rng(7).choice(M, 24, replace=False))
    y = ol.gemm_bf16w(A[rows], W, sc, segs)
    exact = check_bf16(out[rows], y, bound(A[rows], W, sc, segs))
    note(f"  bit-exact fraction {exact:.4f}")


def test_prefill_gemm_rejects_reference_invalid_arguments():
    note("prefill_gemm args")
    t = torch.empty(64, dtype=torch.int16, device="cuda")
    ep = L.GemmEpilogue(1.0, 1.0, 1.0, 8, 8, t.data_ptr(), None, None, 1.0, 8)
    lib = L.lib
    assert lib.granite4_prefill_gemm(0, t.data_ptr(), 48, t.data_ptr(), 1, 8, 48, ep, None, 0) == -1  # K % 32
    assert lib.granite4_prefill_gemm(0, t.data_ptr(), 36, t.data_ptr(), 1, 8, 32, ep, None, 0) == -1  # lda % 8
    assert lib.granite4_prefill_gemm(0, t.data_ptr(), 32, t.data_ptr(), 1, 7, 32, ep, None, 0) == -1  # odd N
    assert lib.granite4_prefill_gemm(3, t.data_ptr(), 32, t.data_ptr(), 1, 8, 32, ep, None, 0) == -1
    assert lib.granite4_prefill_gemm_workspace_bytes(512, 4096) == 0
