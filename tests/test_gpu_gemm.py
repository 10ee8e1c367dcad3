"""GPU parity of the FP8 x FP8 GEMM and its fused epilogues
(granite4_gemm_fp8, granite4_gemm_fp8_swiglu) against the oracle's
g4o_gemm_fp8 (exact products, double accumulation).

Bar, as the reference's own GEMM test (test_kernels.cu:1685-1719): each bf16
output within 2 bf16 ulp of the oracle value rounded to bf16, except where
the sum cancels below the f32 accumulation's reach: there within
K * 2^-22 * s * sum_k |a_k w_k|. That is four times the error bound of K
sequential round-to-nearest f32 additions: each 16x16x128 fp8 matrix-core
instruction forms its 128-product dot internally, aligning the products
before one rounding into the f32 accumulator, and does not round like a
chain of IEEE adds. At 1100x4096x128, three outputs that cancel to 1e-4 of
sum |a w| came out 0.9e-5 .. 1.5e-5 of sum |a w| off, against 0.76e-5 for
the sequential bound and 3.05e-5 for this one. f32 outputs are held to this
bound everywhere. FP8
codes of the fused SwiGLU are bit-exact against the oracle's quantiser
applied to the GPU's own bf16 act (the same scale).
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


def note(msg):
    print(msg, flush=True)


def dev(a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a).cuda()


def host(t):
    torch.cuda.synchronize()
    a = t.cpu().numpy()
    return a.view(np.uint16) if a.dtype == np.int16 else a


def ulp_diff(a, b):
    ai = a.astype(np.int32)
    bi = b.astype(np.int32)
    ai = np.where(ai & 0x8000, 0x8000 - ai, ai)
    bi = np.where(bi & 0x8000, 0x8000 - bi, bi)
    return np.abs(ai - bi)


def abs_bound(A, W, s):
    """K * 2^-22 * s * sum_k |a_k w_k| per output (the fp8 matrix-core sum's error bound)."""
    K = A.shape[1]
    return ol.gemm_fp8(A & 0x7F, abs(s), W & 0x7F).astype(np.float64) * K * 2.0 ** -22


def bf16_ok(got, y_want, bound):
    """got (bf16 bits) vs the f32 oracle value: 2 ulp of bf16(y) or the sum's bound."""
    want = np.vectorize(ol.lib.g4o_f32_to_bf16, otypes=[np.uint16])(y_want)
    d = ulp_diff(got, want)
    err = np.abs(ol.bf16_to_f32(got).astype(np.float64) - y_want.astype(np.float64))
    bad = (d > 2) & (err > bound + np.abs(y_want) * 2.0 ** -7)
    return bad, d


def run_gemm(kind, A, a_scale, W, scales=(1.0, 1.0, 1.0), segs=None, residual=None, rs=1.0):
    M, N = A.shape[0], W.shape[0]
    dA, dW = dev(A), dev(W)
    if kind == L.GEMM_F32:
        out = torch.empty((M, N), dtype=torch.float32, device="cuda")
    elif residual is not None:
        out = dev(residual)
    else:
        out = torch.empty((M, N), dtype=torch.int16, device="cuda")
    L.gemm_fp8(dA, a_scale, dW, out_kind=kind, scales=scales, segs=segs, out=out,
               residual=out if residual is not None else None, resid_scale=rs)
    return host(out)


# Fewer than 256 output tiles of 128 x 128 take the 128 x 64 tile form, and
# where those give each CU at most one tile, K split between the two halves of
# a 512-thread workgroup (K = 128 and 384: an odd count of 128-wide K tiles,
# half 1 idle in the last step); the 1100-row shape (9 x 32 = 288 tiles) the
# 128 x 128 form.
# M <= 16 takes the skinny kernel (16-column workgroups, K in quarters: 384 gives
# quarters of 0, 1, 1 and 1 steps), M = 17 the tiled one.
SHAPES = [(1, 128, 128), (70, 136, 256), (128, 256, 512), (300, 520, 1024), (257, 1024, 4096),
          (1100, 4096, 128), (96, 192, 384), (8, 136, 4096), (16, 520, 384), (17, 520, 384),
          (5, 4096, 12800)]


@pytest.mark.parametrize("M,N,K", SHAPES)
def test_gemm_fp8_bf16(M, N, K):
    note(f"gemm_fp8 bf16 M={M} N={N} K={K}")
    A = ol.fp8_codes(0x71 + M, (M, K))
    W = ol.fp8_codes(0x72 + N, (N, K), std=0.5)
    a_s, w_s = 0.0213, 0.0071
    got = run_gemm(L.GEMM_BF16, A, a_s, W, scales=(w_s, w_s, w_s))
    y = ol.gemm_fp8(A, a_s, W, scales=(w_s, w_s, w_s))
    bad, d = bf16_ok(got, y, abs_bound(A, W, a_s * w_s))
    note(f"  exact fraction {(d == 0).mean():.4f}, max ulp {d.max()}")
    assert not bad.any(), (np.argwhere(bad)[:5], d.max())


@pytest.mark.parametrize("M,N,K", SHAPES[:4])
def test_gemm_fp8_f32(M, N, K):
    note(f"gemm_fp8 f32 M={M} N={N} K={K}")
    A = ol.fp8_codes(0x73 + M, (M, K))
    W = ol.fp8_codes(0x74 + N, (N, K), std=0.5)
    got = run_gemm(L.GEMM_F32, A, 0.5, W, scales=(0.25, 0.25, 0.25))
    y = ol.gemm_fp8(A, 0.5, W, scales=(0.25, 0.25, 0.25))
    err = np.abs(got.astype(np.float64) - y)
    bound = abs_bound(A, W, 0.125) + np.abs(y) * 2.0 ** -23
    note(f"  exact fraction {(got == y).mean():.4f}")
    assert np.all(err <= bound), float((err / (bound + 1e-30)).max())


def test_gemm_fp8_segment_scales():
    """q|k|v-style segments: three weight tensors back to back, three scales."""
    M, K = 96, 512
    N = 384
    A = ol.fp8_codes(0x75, (M, K))
    W = ol.fp8_codes(0x76, (N, K), std=0.5)
    sc, segs = (0.01, 0.02, 0.04), (128, 256)
    got = run_gemm(L.GEMM_BF16, A, 0.3, W, scales=sc, segs=segs)
    y = ol.gemm_fp8(A, 0.3, W, scales=sc, segs=segs)
    bad, d = bf16_ok(got, y, abs_bound(A, W, 0.3 * 0.04))
    assert not bad.any()


@pytest.mark.parametrize("M,N,K", [(64, 256, 512), (200, 4096, 4096), (2100, 2048, 256),
                                   (130, 512, 1408), (8, 4096, 12800), (1, 256, 512)])
def test_gemm_fp8_residual_in_place(M, N, K):
    """The O / down projection: hidden = bf16(hidden + rs * y), in place."""
    note(f"gemm_fp8 residual M={M} N={N} K={K}")
    A = ol.fp8_codes(0x77 + M, (M, K))
    W = ol.fp8_codes(0x78 + N, (N, K), std=0.5)
    res = ol.normal_bf16(0x79, 0.0, 1.0, M * N).reshape(M, N)
    rs, a_s, w_s = 0.22, 0.05, 0.003
    got = run_gemm(L.GEMM_RESIDUAL, A, a_s, W, scales=(w_s, w_s, w_s), residual=res, rs=rs)
    y = ol.gemm_fp8(A, a_s, W, scales=(w_s, w_s, w_s))
    want_f32 = (ol.bf16_to_f32(res) + np.float32(rs) * y).astype(np.float32)
    bad, d = bf16_ok(got, want_f32, abs_bound(A, W, a_s * w_s) * rs)
    note(f"  exact fraction {(d == 0).mean():.4f}, max ulp {d.max()}")
    assert not bad.any()


@pytest.mark.parametrize("M,I,K", [(1, 64, 128), (100, 328, 512), (257, 1280, 4096),
                                   (8, 1280, 4096), (16, 328, 512)])
def test_gemm_fp8_swiglu_fused(M, I, K):
    """gate|up GEMM + SwiGLU (+ FP8) in one GEMM epilogue vs the oracle GEMM
    followed by the reference's f32 SwiGLU (g4o_silu_mul_f32)."""
    note(f"gemm_fp8_swiglu M={M} I={I} K={K}")
    A = ol.fp8_codes(0x7A + M, (M, K))
    W = ol.fp8_codes(0x7B + I, (2 * I, K), std=0.5)
    a_s, gs, us = 0.04, 0.006, 0.009
    dA, dW = dev(A), dev(W)
    work = L.fp8_workspace(rows=16)
    act, codes, scale = L.gemm_fp8_swiglu(dA, a_s, dW, gs, us, work,
                                          act=torch.empty((M, I), dtype=torch.int16, device="cuda"))
    y = ol.gemm_fp8(A, a_s, W, scales=(gs, us, us), segs=(I, I))
    want = ol.silu_mul_f32(y)
    got = host(act)
    d = ulp_diff(got, want)
    # where gate or up nearly cancel, bound the act error by the sums' bounds
    bg = abs_bound(A, W[:I], a_s * gs)
    bu = abs_bound(A, W[I:], a_s * us)
    g, u = y[:, :I].astype(np.float64), y[:, I:].astype(np.float64)
    sig = 1.0 / (1.0 + np.exp(-g))
    tol = np.abs(sig * u) * bg * 1.2 + np.abs(g * sig) * bu + np.abs(ol.bf16_to_f32(want)) * 2.0 ** -7
    err = np.abs(ol.bf16_to_f32(got).astype(np.float64) - ol.bf16_to_f32(want))
    bad = (d > 2) & (err > tol)
    note(f"  act exact fraction {(d == 0).mean():.4f}, max ulp {d.max()}")
    assert not bad.any(), (np.argwhere(bad)[:5], d.max())
    want_codes, want_scale = ol.fp8_quantize(got)
    assert host(scale)[0] == np.float32(want_scale)
    np.testing.assert_array_equal(host(codes), want_codes)
    # act only (no codes)
    act2 = L.gemm_fp8_swiglu(dA, a_s, dW, gs, us, work, fp8=False,
                             act=torch.empty((M, I), dtype=torch.int16, device="cuda"))
    np.testing.assert_array_equal(host(act2), got)


def test_gemm_fp8_invalid_arguments():
    A = torch.zeros((4, 100), dtype=torch.uint8, device="cuda")
    W = torch.zeros((8, 100), dtype=torch.uint8, device="cuda")
    with pytest.raises(L.Granite4Error):
        L.gemm_fp8(A, 1.0, W)  # K % 128 != 0
    A = torch.zeros((4, 128), dtype=torch.uint8, device="cuda")
    W = torch.zeros((12, 128), dtype=torch.uint8, device="cuda")
    with pytest.raises(L.Granite4Error):
        L.gemm_fp8(A, 1.0, W)  # N % 8 != 0 (the vector epilogue)


@pytest.mark.parametrize("M", [64, 512])
def test_gemm_fp8_residual_rmsnorm_fp8(M):
    """O / down GEMM + residual, then the next RMSNorm to FP8: the updated
    hidden against the oracle (as the residual test), and the codes / scale
    identical to granite4_add_rmsnorm_fp8 run alone on that hidden."""
    H, K = 4096, 4096
    note(f"gemm_fp8_residual_rmsnorm_fp8 M={M}")
    A = ol.fp8_codes(0x7C + M, (M, K))
    W = ol.fp8_codes(0x7D, (H, K), std=0.5)
    res = ol.normal_bf16(0x7E, 0.0, 1.0, M * H).reshape(M, H)
    gamma = ol.normal_bf16(0x7F, 1.0, 0.1, H)
    rs, a_s, w_s = 0.22, 0.05, 0.003
    dA, dW, hid, dg = dev(A), dev(W), dev(res), dev(gamma)
    codes = torch.empty((M, H), dtype=torch.uint8, device="cuda")
    scale = torch.empty(1, dtype=torch.float32, device="cuda")
    work = L.fp8_workspace(rows=M)
    d_as = torch.tensor([a_s], dtype=torch.float32, device="cuda")
    L.call("granite4_gemm_fp8_residual_rmsnorm_fp8", dA, K, d_as, dW, M, H, K, w_s, hid, rs, dg,
           1e-5, codes, scale, work)
    got = host(hid)
    y = ol.gemm_fp8(A, a_s, W, scales=(w_s, w_s, w_s))
    want_f32 = (ol.bf16_to_f32(res) + np.float32(rs) * y).astype(np.float32)
    bad, d = bf16_ok(got, want_f32, abs_bound(A, W, a_s * w_s) * rs)
    assert not bad.any()
    codes2 = torch.empty_like(codes)
    scale2 = torch.empty_like(scale)
    L.call("granite4_add_rmsnorm_fp8", hid, None, 1.0, dg, 1e-5, M, H, None, codes2, scale2, work)
    np.testing.assert_array_equal(host(codes), host(codes2))
    assert host(scale)[0] == host(scale2)[0]
    # and the norm itself against the oracle (<= 1 ulp) through the bf16 form
    normed = torch.empty_like(hid)
    L.call("granite4_kernel_rmsnorm", hid, dg, 1e-5, M, H, normed)
    assert ulp_diff(host(normed), ol.rmsnorm(got, gamma, 1e-5)).max() <= 1
    want_codes, want_scale = ol.fp8_quantize(host(normed))
    assert host(scale)[0] == np.float32(want_scale)
    np.testing.assert_array_equal(host(codes), want_codes)


def test_norm_fp8_feeds_gemm_through_device_scale_graph_replay():
    """add+RMSNorm -> FP8 chained into the GEMM through the device scale the
    norm writes (no host round trip), captured once as a HIP graph and
    replayed with new inputs written between replays: every replay matches
    the oracle GEMM of that replay's codes and scale."""
    M, H, N = 96, 4096, 256
    gamma = dev(ol.normal_bf16(0x90, 1.0, 0.1, H))
    W = ol.fp8_codes(0x91, (N, H), std=0.5)
    dW = dev(W)
    res = torch.empty((M, H), dtype=torch.int16, device="cuda")
    br = torch.empty_like(res)
    ro = torch.empty_like(res)
    codes = torch.empty((M, H), dtype=torch.uint8, device="cuda")
    scale = torch.empty(1, dtype=torch.float32, device="cuda")
    out = torch.empty((M, N), dtype=torch.int16, device="cuda")
    work = L.fp8_workspace(rows=M)
    w_s = 0.004

    def step():
        L.call("granite4_add_rmsnorm_fp8", res, br, 1.0, gamma, 1e-5, M, H, ro, codes, scale, work)
        L.gemm_fp8(codes, scale, dW, out=out, scales=(w_s, w_s, w_s))

    def fill(seed):
        res.copy_(dev(ol.normal_bf16(seed, 0.0, 1.0, M * H).reshape(M, H)))
        br.copy_(dev(ol.normal_bf16(seed + 1, 0.0, 2.0, M * H).reshape(M, H)))

    fill(0x92)
    step()
    torch.cuda.synchronize()
    cap = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(cap):
        L.use_stream(cap)
        with torch.cuda.graph(g, stream=cap):
            step()
    L.use_stream()
    torch.cuda.synchronize()
    for rep, seed in enumerate((0x93, 0x95, 0x97)):
        fill(seed)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        c, s = host(codes), host(scale)[0]
        y = ol.gemm_fp8(c, s, W, scales=(w_s, w_s, w_s))
        bad, d = bf16_ok(host(out), y, abs_bound(c, W, s * w_s))
        note(f"  replay {rep}: scale {s:.6g}, max ulp {d.max()}")
        assert not bad.any()


@pytest.mark.parametrize("M", [512, 8192])
def test_gemm_fp8_swiglu_fp8_8b_shape(M):
    """The gate|up + SwiGLU -> FP8 GEMM at the 8B shape (I 12800, K 4096):
    codes and scale of the reference quantiser on the act the GEMM stored,
    the same in every FP8 launch mode."""
    note(f"gemm_fp8_swiglu 8B shape M={M}")
    I, K = 12800, 4096
    dA = dev(ol.fp8_codes(0x7C, (M, K)))
    dW = dev(ol.fp8_codes(0x7D, (2 * I, K), std=0.5))
    a_s, gs, us = 0.04, 0.006, 0.009
    work = L.fp8_workspace(rows=16)
    res = []
    for mode in (0, 1):
        prev = L.set_fp8_launch_mode(mode)
        try:
            act, codes, scale = L.gemm_fp8_swiglu(
                dA, a_s, dW, gs, us, work, act=torch.empty((M, I), dtype=torch.int16, device="cuda"))
            res.append((host(act).copy(), host(codes).copy(), host(scale)[0]))
        finally:
            L.set_fp8_launch_mode(prev)
    np.testing.assert_array_equal(res[0][0], res[1][0])
    np.testing.assert_array_equal(res[0][1], res[1][1])
    assert res[0][2] == res[1][2]
    want_codes, want_scale = ol.fp8_quantize(res[0][0])
    assert res[0][2] == np.float32(want_scale)
    np.testing.assert_array_equal(res[0][1], want_codes)
    assert L.fp8_sync_status(work) == 0
