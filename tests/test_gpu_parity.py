"""GPU parity: the gfx950 kernels, called through the C ABI, against the CPU
oracle on the same seeded inputs.

Bars: bit-exact for the embedding gather, FP8 / int8 /
int4 / K5 codes and scales, and page indexing; RMSNorm, SwiGLU and RoPE within
1 bf16 ulp of the oracle's f32 evaluation (RMSNorm and RoPE are expected, and
reported, bit-exact; SwiGLU uses hardware exp / rcp and may differ by 1 ulp).
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
    print("device arch:", L.device_arch(), flush=True)


def dev(a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    elif a.dtype == np.uint32:
        a = a.view(np.int32)
    return torch.from_numpy(a).cuda()


def host(t, dtype=None):
    a = t.detach().cpu().numpy()
    if a.dtype == np.int16:
        a = a.view(np.uint16)
    return a if dtype is None else a.view(dtype)


def ulp_diff(a, b):
    """bf16 ulp distance of two uint16 arrays (same-sign ordering)."""
    ai = a.astype(np.int32)
    bi = b.astype(np.int32)
    ai = np.where(ai & 0x8000, 0x8000 - ai, ai)
    bi = np.where(bi & 0x8000, 0x8000 - bi, bi)
    return np.abs(ai - bi)


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


# ----------------------------------------------------------------------------- hardware conversions
def test_selftest_bf16_hw_conversion_all_f32():
    note("selftest bf16 (2^32 patterns)")
    res = torch.zeros(2, dtype=torch.int64, device="cuda")
    L.call("granite4_selftest_bf16", res)
    r = host(res)
    assert r[0] == 0, f"{r[0]} mismatches, first input bits {int(r[1]):#010x}"


@pytest.mark.parametrize("scale", [1.0, 3.0 / 448, 4.0 / 448, 7.0 / 448, 0.1, 1e-20, 7.7e5, 2.0 ** -90])
def test_selftest_fp8_hw_encoder_exhaustive(scale):
    note(f"selftest fp8 scale={scale}")
    res = torch.zeros(2, dtype=torch.int64, device="cuda")
    L.call("granite4_selftest_fp8", float(np.float32(scale)), res)
    r = host(res)
    assert r[0] == 0, f"{r[0]} mismatches, first input bits {int(r[1]):#010x}"


# ----------------------------------------------------------------------------- embed
@pytest.mark.parametrize("rows,mult", [(1, 1.0), (8, 1.0), (512, 1.0), (37, 0.7071), (4100, 0.5)])
def test_embed_rows_bit_exact(rows, mult):
    note(f"embed rows={rows} mult={mult}")
    vocab, H = 1000, 4096
    emb = ol.normal_bf16(0xE1, 0.0, 0.02, vocab * H).reshape(vocab, H)
    tok = (ol.u32(0xE2 + rows, rows) % vocab).astype(np.int32)
    d_emb, d_tok = dev(emb), dev(tok)
    out = torch.empty((rows, H), dtype=torch.int16, device="cuda")
    L.call("granite4_embed_rows", d_tok, rows, d_emb, vocab, H, mult, out)
    np.testing.assert_array_equal(host(out), ol.embed_rows(tok, emb, mult))
    # the reference-named prefill form with a start offset
    out2 = torch.empty_like(out)
    big = np.concatenate([np.zeros(5, np.int32), tok])
    L.prefill_embed_rows(dev(big), 5, rows, d_emb, mult, out2, H)
    np.testing.assert_array_equal(host(out2), host(out))


def test_embed_invalid_token_zero_row_and_decode_pos():
    note("embed invalid/decode")
    vocab, H = 64, 4096
    emb = ol.normal_bf16(0xE3, 0.0, 0.02, vocab * H).reshape(vocab, H)
    tok = np.array([3, -1, 64, 63], np.int32)
    out = torch.full((4, H), 77, dtype=torch.int16, device="cuda")
    L.call("granite4_embed_rows", dev(tok), 4, dev(emb), vocab, H, 1.0, out)
    o = host(out)
    np.testing.assert_array_equal(o[0], emb[3])
    assert not o[1].any() and not o[2].any()
    np.testing.assert_array_equal(o[3], emb[63])
    one = torch.empty((1, H), dtype=torch.int16, device="cuda")
    pos = dev(np.array([3], np.int32))
    L.call("granite4_embed_at_pos", dev(tok), pos, dev(emb), vocab, H, 1.0, one)
    np.testing.assert_array_equal(host(one)[0], emb[63])


@pytest.mark.parametrize("rows", [4095, 4096, 8193])
def test_embed_whole_row_workgroups_invalid_tokens(rows):
    """The whole-row workgroup forms (two rows each below 4096 rows, one from
    4096): tokens outside [0, vocab) give zero rows at every position,
    including the odd last row, and the rest match the oracle."""
    note(f"embed whole rows invalid rows={rows}")
    vocab, H = 300, 4096
    emb = ol.normal_bf16(0xE4, 0.0, 0.02, vocab * H).reshape(vocab, H)
    tok = (ol.u32(0xE5 + rows, rows) % vocab).astype(np.int32)
    bad = np.array([0, 1, rows // 2, rows - 2, rows - 1])
    tok[bad[::2]] = -7
    tok[bad[1::2]] = vocab
    out = torch.full((rows, H), 77, dtype=torch.int16, device="cuda")
    L.call("granite4_embed_rows", dev(tok), rows, dev(emb), vocab, H, 0.75, out)
    o = host(out)
    assert not o[bad].any()
    good = np.setdiff1d(np.arange(rows), bad)
    np.testing.assert_array_equal(o[good], ol.embed_rows(tok[good], emb, 0.75))


# ----------------------------------------------------------------------------- rmsnorm
def _hidden(rows, cols, seed, outliers=True):
    x = ol.normal_bf16(seed, 0.0, 1.0, rows * cols).reshape(rows, cols)
    if outliers:
        ch = np.random.default_rng(seed).choice(cols, max(1, cols // 100), replace=False)
        xf = ol.bf16_to_f32(x)
        xf[:, ch] *= 20.0
        x = ol.f32_to_bf16(xf)
    return x


@pytest.mark.parametrize("rows,cols", [(64, 256), (5, 4096), (16, 4096), (512, 4096),
                                       (3, 4000), (2, 12800)])
def test_rmsnorm_reference_api(rows, cols):
    note(f"rmsnorm rows={rows} cols={cols}")
    if cols == 256:
        x = ol.uniform_bf16(0x4242, 4.0, rows * cols).reshape(rows, cols)
        w = ol.uniform_bf16(0x4243, 1.5, cols)
    else:
        x = _hidden(rows, cols, 0x4244 + rows)
        w = ol.normal_bf16(0x4245, 1.0, 0.1, cols)
    out = torch.empty((rows, cols), dtype=torch.int16, device="cuda")
    fn = "granite4_kernel_rmsnorm_batched" if rows <= 16 else "granite4_kernel_rmsnorm"
    L.call(fn, dev(x), dev(w), 1e-5, rows, cols, out)
    d = ulp_diff(host(out), ol.rmsnorm(x, w, 1e-5))
    assert d.max() <= 1
    assert (d == 0).mean() >= 0.9999, (d != 0).sum()


@pytest.mark.parametrize("rows", [1, 8, 512, 2500])
@pytest.mark.parametrize("mult", [1.0, 0.25])
def test_add_rmsnorm_bf16(rows, mult):
    note(f"add_rmsnorm rows={rows} mult={mult}")
    cols = 4096
    res = _hidden(rows, cols, 0xA1 + rows)
    br = ol.normal_bf16(0xA2 + rows, 0.0, 1.0, rows * cols).reshape(rows, cols)
    w = ol.normal_bf16(0xA3, 1.0, 0.1, cols)
    ro_want, no_want = ol.add_rmsnorm(res, br, mult, w, 1e-5)
    d_res = dev(res)
    ro = torch.empty_like(d_res)
    no = torch.empty_like(d_res)
    L.call("granite4_add_rmsnorm", d_res, dev(br), mult, dev(w), 1e-5, rows, cols, ro, no)
    np.testing.assert_array_equal(host(ro), ro_want)
    d = ulp_diff(host(no), no_want)
    assert d.max() <= 1 and (d == 0).mean() >= 0.9999
    # in place: res_out aliases res
    L.call("granite4_add_rmsnorm", d_res, dev(br), mult, dev(w), 1e-5, rows, cols, d_res, no)
    np.testing.assert_array_equal(host(d_res), ro_want)


def _fp8_check(codes, scale, normed_bf16):
    """codes / scale must be the reference quantiser applied to the bf16 tensor."""
    want_codes, want_scale = ol.fp8_quantize(normed_bf16)
    assert scale == np.float32(want_scale), (scale, want_scale)
    np.testing.assert_array_equal(codes, want_codes)


# Up to 4096 rows of 4096 take the single-launch form on 256 CUs (1024
# workgroups x 4 rows held in VGPRs); up to 12288 the deep single-launch form
# (x 8 rows in VGPRs + 4 in LDS); 12289 takes two launches.
@pytest.mark.parametrize("rows", [1, 8, 512, 2048, 3000, 4096, 4097, 8192, 12289])
def test_add_rmsnorm_fp8(rows):
    note(f"add_rmsnorm_fp8 rows={rows}")
    cols = 4096
    res = _hidden(rows, cols, 0xB1 + rows)
    br = ol.normal_bf16(0xB2, 0.0, 1.0, rows * cols).reshape(rows, cols)
    w = ol.normal_bf16(0xB3, 1.0, 0.1, cols)
    d_res, d_br, d_w = dev(res), dev(br), dev(w)
    work = L.fp8_workspace()
    ro = torch.empty_like(d_res)
    codes = torch.empty((rows, cols), dtype=torch.uint8, device="cuda")
    scale = torch.empty(1, dtype=torch.float32, device="cuda")
    L.call("granite4_add_rmsnorm_fp8", d_res, d_br, 1.0, d_w, 1e-5, rows, cols, ro, codes, scale,
           work)
    # the bf16 normed tensor of the same inputs (the GPU's own)
    no = torch.empty_like(d_res)
    L.call("granite4_add_rmsnorm", d_res, d_br, 1.0, d_w, 1e-5, rows, cols, torch.empty_like(d_res),
           no)
    ro_want, no_want = ol.add_rmsnorm(res, br, 1.0, w, 1e-5)
    np.testing.assert_array_equal(host(ro), ro_want)
    _fp8_check(host(codes), host(scale)[0], host(no))
    assert ulp_diff(host(no), no_want).max() <= 1
    # the two-launch form: same residual, codes and scale
    prev = L.set_fp8_launch_mode(1)
    try:
        ro3 = torch.empty_like(d_res)
        codes3 = torch.empty_like(codes)
        scale3 = torch.empty_like(scale)
        L.call("granite4_add_rmsnorm_fp8", d_res, d_br, 1.0, d_w, 1e-5, rows, cols, ro3, codes3,
               scale3, work)
    finally:
        L.set_fp8_launch_mode(prev)
    np.testing.assert_array_equal(host(ro3), ro_want)
    np.testing.assert_array_equal(host(codes3), host(codes))
    assert host(scale3)[0] == host(scale)[0]
    # a second, smaller call on the same workspace
    r2 = max(1, rows // 3)
    L.call("granite4_add_rmsnorm_fp8", d_res, d_br, 1.0, d_w, 1e-5, r2, cols, ro, codes, scale,
           work)
    _fp8_check(host(codes)[:r2], host(scale)[0], host(no)[:r2])


def test_add_rmsnorm_fp8_graph_replay():
    """A captured single-launch add+RMSNorm->FP8 replayed with new inputs
    between replays (the synchronisation slots advance through the
    workspace's generation word): every replay equals an eager call."""
    note("add_rmsnorm_fp8 graph")
    rows, cols = 200, 4096
    w = dev(ol.normal_bf16(0xB6, 1.0, 0.1, cols))
    work = L.fp8_workspace(rows)
    xs = [dev(_hidden(rows, cols, 0xB7 + i)) for i in range(3)]
    br = dev(ol.normal_bf16(0xBA, 0.0, 0.5, rows * cols).reshape(rows, cols))
    ro = torch.empty_like(xs[0])
    codes = torch.empty((rows, cols), dtype=torch.uint8, device="cuda")
    scale = torch.empty(1, dtype=torch.float32, device="cuda")
    want = []
    for x in xs:
        L.call("granite4_add_rmsnorm_fp8", x, br, 0.5, w, 1e-5, rows, cols, ro, codes, scale, work)
        want.append((host(ro).copy(), host(codes).copy(), host(scale)[0]))
    src = torch.empty_like(xs[0])
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    L.use_stream(s)
    try:
        with torch.cuda.graph(g, stream=s):
            L.call("granite4_add_rmsnorm_fp8", src, br, 0.5, w, 1e-5, rows, cols, ro, codes, scale,
                   work)
    finally:
        L.call("granite4_set_stream", None)
    for i in (1, 2, 0, 1):
        src.copy_(xs[i])
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(host(ro), want[i][0])
        np.testing.assert_array_equal(host(codes), want[i][1])
        assert host(scale)[0] == want[i][2]


def test_add_rmsnorm_fp8_zero_tensor_and_no_residual():
    note("add_rmsnorm_fp8 zero")
    rows, cols = 4, 4096
    z = np.zeros((rows, cols), np.uint16)
    w = ol.normal_bf16(0xB4, 1.0, 0.1, cols)
    work = L.fp8_workspace(rows)
    codes = torch.full((rows, cols), 0x55, dtype=torch.uint8, device="cuda")
    scale = torch.full((1,), 7.0, dtype=torch.float32, device="cuda")
    L.call("granite4_add_rmsnorm_fp8", dev(z), None, 1.0, dev(w), 1e-5, rows, cols, None, codes,
           scale, work)
    assert host(scale)[0] == 0.0 and not host(codes).any()
    # plain RMSNorm -> FP8 (no residual): codes of the quantised rmsnorm
    x = _hidden(rows, cols, 0xB5)
    L.call("granite4_add_rmsnorm_fp8", dev(x), None, 1.0, dev(w), 1e-5, rows, cols, None, codes,
           scale, work)
    _fp8_check(host(codes), host(scale)[0], ol.rmsnorm(x, w, 1e-5))


# ----------------------------------------------------------------------------- swiglu
# 655 rows of I = 12800 are the largest the register-only single-launch form
# holds (1024 workgroups x 256 lanes x 4 vectors); 656 and up take the held
# form, which keeps 21 vectors per lane (12 in VGPRs, 9 in LDS: ~3440 rows
# on a full grid) and streams the rest twice; 5000 rows stream.
@pytest.mark.parametrize("rows", [1, 8, 64, 655, 656, 2048, 2700, 5000])
def test_swiglu_bf16_and_fp8(rows):
    note(f"swiglu rows={rows}")
    I_ = 12800
    gu = ol.normal_bf16(0xC1 + rows, 0.0, 1.0, rows * 2 * I_).reshape(rows, 2 * I_)
    d_gu = dev(gu)
    act = torch.empty((rows, I_), dtype=torch.int16, device="cuda")
    L.call("granite4_swiglu", d_gu, rows, I_, act)
    want = ol.swiglu(gu)
    d = ulp_diff(host(act), want)
    assert d.max() <= 1, d.max()
    note(f"  swiglu bf16 exact fraction {(d == 0).mean():.6f}")
    work = L.fp8_workspace()
    codes = torch.empty((rows, I_), dtype=torch.uint8, device="cuda")
    scale = torch.empty(1, dtype=torch.float32, device="cuda")
    act2 = torch.empty_like(act)
    L.call("granite4_swiglu_fp8", d_gu, rows, I_, codes, scale, work, act2)
    np.testing.assert_array_equal(host(act2), host(act))
    _fp8_check(host(codes), host(scale)[0], host(act))
    # without the act buffer the encode launch recomputes the SiLU: same codes
    codes2 = torch.empty_like(codes)
    scale2 = torch.empty_like(scale)
    L.call("granite4_swiglu_fp8", d_gu, rows, I_, codes2, scale2, work, None)
    np.testing.assert_array_equal(host(codes2), host(codes))
    assert host(scale2)[0] == host(scale)[0]
    # the two-launch form gives the same codes and scale
    prev = L.set_fp8_launch_mode(1)
    try:
        codes3 = torch.empty_like(codes)
        scale3 = torch.empty_like(scale)
        L.call("granite4_swiglu_fp8", d_gu, rows, I_, codes3, scale3, work, None)
    finally:
        L.set_fp8_launch_mode(prev)
    np.testing.assert_array_equal(host(codes3), host(codes))
    assert host(scale3)[0] == host(scale)[0]


def test_swiglu_fp8_single_launch_repeated_and_graph_replay():
    """Back-to-back single-launch calls on one workspace (the synchronisation
    slots are reused through the generation word), then a captured graph
    replayed several times with new inputs written between replays: every
    result equals an eager call on the same inputs."""
    note("swiglu_fp8 repeated + graph")
    rows, I_ = 96, 12800
    work = L.fp8_workspace()
    gus = [dev(ol.normal_bf16(0xC7 + i, 0.0, 1.0 + i, rows * 2 * I_).reshape(rows, 2 * I_))
           for i in range(4)]
    codes = torch.empty((rows, I_), dtype=torch.uint8, device="cuda")
    scale = torch.empty(1, dtype=torch.float32, device="cuda")
    want = []
    for g in gus:
        L.call("granite4_swiglu_fp8", g, rows, I_, codes, scale, work, None)
        want.append((host(codes).copy(), host(scale)[0]))
        act = torch.empty((rows, I_), dtype=torch.int16, device="cuda")
        L.call("granite4_swiglu", g, rows, I_, act)
        _fp8_check(want[-1][0], want[-1][1], host(act))
    # repeated calls alternate inputs of different scales on one workspace
    for i in (1, 0, 3, 2):
        L.call("granite4_swiglu_fp8", gus[i], rows, I_, codes, scale, work, None)
        np.testing.assert_array_equal(host(codes), want[i][0])
        assert host(scale)[0] == want[i][1]
    src = torch.empty_like(gus[0])
    src.copy_(gus[0])
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    L.use_stream(s)
    try:
        with torch.cuda.graph(g, stream=s):
            L.call("granite4_swiglu_fp8", src, rows, I_, codes, scale, work, None)
    finally:
        L.call("granite4_set_stream", None)  # back to the per-thread default stream
    for i in (2, 1, 3, 0, 2):
        src.copy_(gus[i])
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(host(codes), want[i][0])
        assert host(scale)[0] == want[i][1]


def test_prefill_silu_mul_f32():
    note("prefill_silu_mul")
    rows, I_ = 4, 12800
    gu = np.random.default_rng(3).normal(0, 2, (rows, 2 * I_)).astype(np.float32)
    act = torch.empty((rows, I_), dtype=torch.int16, device="cuda")
    L.call("granite4_prefill_silu_mul", torch.from_numpy(gu).cuda(), I_, rows, act)
    want = np.empty((rows, I_), np.uint16)
    ol.lib.g4o_silu_mul_f32(gu.ctypes.data_as(ol.f32p), I_, rows, want.ctypes.data_as(ol.u16p))
    assert ulp_diff(host(act), want).max() <= 1


# ----------------------------------------------------------------------------- rope
@pytest.fixture(scope="module")
def tables():
    c, s = ol.rope_tables(1e7, 128, 65536)
    return c, s, dev(c), dev(s)


def test_rope_tables_fill_and_build(tables):
    note("rope tables")
    c, s, dc, ds = tables
    gc, gs = L.rope_tables(1e7, 128, 65536)
    np.testing.assert_array_equal(host(gc), c)
    np.testing.assert_array_equal(host(gs), s)


def test_rope_reference_apis(tables):
    note("rope ref apis")
    c, s, dc, ds = tables
    rows = 128  # test_kernels.cu:1057: 128 positions x d 128, seed 0x1337
    x = ol.uniform_bf16(0x1337, 4.0, rows * 128).reshape(rows, 1, 128)
    out = torch.empty((rows, 128), dtype=torch.int16, device="cuda")
    L.call("granite4_kernel_rope", dev(x), dc, ds, rows, 128, out)
    np.testing.assert_array_equal(host(out), ol.rope_rows(x, np.arange(rows), c, s).reshape(rows, 128))
    # one position, many heads
    xh = ol.uniform_bf16(0x1338, 4.0, 40 * 128).reshape(1, 40, 128)
    p = 60001
    out = torch.empty((40, 128), dtype=torch.int16, device="cuda")
    L.call("granite4_kernel_rope_at_pos", dev(xh), dc[p], ds[p], 40, 128, out)
    np.testing.assert_array_equal(host(out), ol.rope_rows(xh, [p], c, s).reshape(40, 128))
    # batched verify rows with per-row table rows
    xb = ol.uniform_bf16(0x1339, 4.0, 7 * 32 * 128).reshape(7, 32, 128)
    base = 5000
    out = torch.empty((7, 32 * 128), dtype=torch.int16, device="cuda")
    L.call("granite4_kernel_rope_at_pos_batched", dev(xb), dc[base:], ds[base:], 7, 32, 128, out)
    np.testing.assert_array_equal(host(out).reshape(7, 32, 128),
                                  ol.rope_rows(xb, np.arange(base, base + 7), c, s))
    # a head dim other than 128 takes the generic kernel
    x64 = ol.uniform_bf16(0x133A, 4.0, 9 * 64).reshape(9, 1, 64)
    c64, s64 = ol.rope_tables(1e7, 64, 16)
    out = torch.empty((9, 64), dtype=torch.int16, device="cuda")
    L.call("granite4_kernel_rope", dev(x64), dev(c64), dev(s64), 9, 64, out)
    np.testing.assert_array_equal(host(out), ol.rope_rows(x64, np.arange(9), c64, s64).reshape(9, 64))


def _qkv(rows, seed, Hq=32, Hk=8):
    return ol.normal_bf16(seed, 0.0, 1.0, rows * (Hq + 2 * Hk) * 128).reshape(rows, -1)


def _arena_compare(arena, want, bits, group, Hk, stride):
    _, ck, cv, ks, vs = want
    kb, vb = L.kv_row_bytes(bits)
    np.testing.assert_array_equal(host(arena.k).reshape(-1), ck.reshape(-1))
    np.testing.assert_array_equal(host(arena.v).reshape(-1), cv.reshape(-1))
    if bits != 16:
        np.testing.assert_array_equal(host(arena.k_scale).reshape(-1), ks.reshape(-1))
        np.testing.assert_array_equal(host(arena.v_scale).reshape(-1), vs.reshape(-1))


def _oracle_arena(bits, group, Hk, stride, fill=0xEE):
    kb, vb = L.kv_row_bytes(bits)
    ng = 128 // group
    return (np.full(Hk * stride * kb, fill, np.uint8), np.full(Hk * stride * vb, fill, np.uint8),
            np.zeros(Hk * stride * ng, np.float32), np.zeros(Hk * stride * ng, np.float32))


@pytest.mark.parametrize("rows", [40, 300, 800])
@pytest.mark.parametrize("bits", [16, 8, 4, 5])
def test_prefill_rope_split_append_paged(tables, bits, rows):
    """The reference's prefill launchers: f32-rotated K quantised, random page table,
    untouched rows keep their 0xEE fill (test_kernels.cu:730-801). 40 and 300 rows take
    the one-unit-per-lane-group kernel, 800 the per-token one (from 704 rows)."""
    note(f"prefill split append bits={bits} rows={rows}")
    c, s, dc, ds = tables
    Hq, Hk, base = 32, 8, 100
    pages = (base + rows + 15) // 16 + 2
    stride = pages * 16
    bt = np.random.default_rng(bits).permutation(pages).astype(np.int32)
    pt = ol.row_table(bt, stride)
    qkv = _qkv(rows, 0x5A5A + bits)
    arena = L.KvArena(bits, Hk, stride, fill=0xEE)
    q_rot = torch.empty((rows, Hq * 128), dtype=torch.int16, device="cuda")
    L.prefill_rope_split_append(bits, dev(qkv), dc, ds, base, rows, Hq, Hk, 128, stride, q_rot,
                                arena.k, arena.v, arena.k_scale, arena.v_scale, dev(pt))
    q, k, v = qkv[:, :Hq * 128], qkv[:, Hq * 128:(Hq + Hk) * 128], qkv[:, (Hq + Hk) * 128:]
    ck, cv, ks, vs = _oracle_arena(bits, 128, Hk, stride)
    pos = np.arange(base, base + rows)
    want = ol.rope_append(q, k, v, c, s, pos, pt[pos], bits, 128, stride, Hk, k_round_bf16=False,
                          cache_k=ck, cache_v=cv, k_scale=ks, v_scale=vs)
    np.testing.assert_array_equal(host(q_rot), want[0])
    _arena_compare(arena, want, bits, 128, Hk, stride)


@pytest.mark.parametrize("rows", [64, 800])
@pytest.mark.parametrize("bits,group", [(8, 128), (8, 32), (4, 32), (5, 32), (5, 64), (16, 128)])
def test_rope_append_fused_entry(tables, bits, group, rows):
    """granite4_rope_append at config-4 positions (57344..), group scales, per-row arena rows
    (64 rows: one unit per lane group; 800: one workgroup per token)."""
    note(f"rope_append bits={bits} group={group} rows={rows}")
    c, s, dc, ds = tables
    Hq, Hk = 32, 8
    stride = 1024  # arena rows: a permutation of [0, stride), one per token row (rows <= stride)
    assert rows <= stride
    qkv = _qkv(rows, 0x77 + bits + group)
    d_qkv = dev(qkv)
    q, k, v = d_qkv[:, :Hq * 128], d_qkv[:, Hq * 128:(Hq + Hk) * 128], d_qkv[:, (Hq + Hk) * 128:]
    arena = L.KvArena(bits, Hk, stride, group=group, fill=0xEE)
    base = min(57344 + 8000, 65536 - rows)
    arows = np.random.default_rng(group).permutation(stride)[:rows].astype(np.int32)
    for k_round in (False, True):
        q_rot = L.rope_append(arena, q, k, v, dc, ds, base_pos=base, arena_rows=dev(arows),
                              k_round_bf16=k_round)
        ck, cv, ks, vs = _oracle_arena(bits, group, Hk, stride)
        hq, hk, hv = qkv[:, :Hq * 128], qkv[:, Hq * 128:(Hq + Hk) * 128], qkv[:, (Hq + Hk) * 128:]
        want = ol.rope_append(hq, hk, hv, c, s, np.arange(base, base + rows), arows, bits, group,
                              stride, Hk, k_round_bf16=k_round, cache_k=ck, cache_v=cv,
                              k_scale=ks, v_scale=vs)
        np.testing.assert_array_equal(host(q_rot), want[0])
        _arena_compare(arena, want, bits, group, Hk, stride)


@pytest.mark.parametrize("bits", [16, 8, 4, 5])
def test_kv_append_batched_reference_api(bits):
    note(f"kv_append_batched bits={bits}")
    rows, Hk, base, stride = 11, 8, 30, 64
    kx = ol.uniform_bf16(0x8ABC + bits, 4.0, rows * Hk * 128).reshape(rows, Hk * 128)
    vx = ol.uniform_bf16(0x8ABD + bits, 3.0, rows * Hk * 128).reshape(rows, Hk * 128)
    kx[0, :128] = 0  # an all-zero row: scale 0, zero codes
    pt = np.random.default_rng(9).permutation(stride).astype(np.int32)
    arena = L.KvArena(bits, Hk, stride, fill=0xEE)
    name = {16: "granite4_kernel_kv_append_batched", 8: "granite4_kernel_kv_append_int8_batched",
            4: "granite4_kernel_kv_append_int4_batched",
            5: "granite4_kernel_kv_append_k5v4_batched"}[bits]
    if bits == 16:
        L.call(name, dev(kx), dev(vx), arena.k, arena.v, base, rows, stride, Hk, 128, dev(pt))
    else:
        L.call(name, dev(kx), dev(vx), arena.k, arena.v, arena.k_scale, arena.v_scale, base, rows,
               stride, Hk, 128, dev(pt))
    ck, cv, ks, vs = _oracle_arena(bits, 128, Hk, stride)
    pos = np.arange(base, base + rows)
    want = ol.rope_append(None, kx, vx, None, None, pos, pt[pos], bits, 128, stride, Hk,
                          rotate_k=False, cache_k=ck, cache_v=cv, k_scale=ks, v_scale=vs)
    _arena_compare(arena, want, bits, 128, Hk, stride)


def test_kv_append_int8_generic_head_dim():
    note("kv_append int8 d=64")
    rows, Hk, d, stride = 5, 2, 64, 8
    kx = ol.uniform_bf16(0x101, 4.0, rows * Hk * d).reshape(rows, Hk * d)
    vx = ol.uniform_bf16(0x102, 4.0, rows * Hk * d).reshape(rows, Hk * d)
    ck = torch.zeros((Hk, stride, d), dtype=torch.int8, device="cuda")
    cv = torch.zeros_like(ck)
    ks = torch.zeros((Hk, stride), dtype=torch.float32, device="cuda")
    vs = torch.zeros_like(ks)
    L.call("granite4_kernel_kv_append_int8_batched", dev(kx), dev(vx), ck, cv, ks, vs, 2, rows,
           stride, Hk, d, None)
    want = ol.rope_append(None, kx, vx, None, None, np.arange(2, 2 + rows), np.arange(2, 2 + rows),
                          8, d, stride, Hk, d=d, rotate_k=False)
    np.testing.assert_array_equal(host(ck).view(np.uint8).reshape(-1), want[1])
    np.testing.assert_array_equal(host(ks).reshape(-1), want[3])


def test_verify_qkv_stage(tables):
    note("verify_qkv_stage")
    c, s, dc, ds = tables
    rows, Hq, Hk, base, stride = 6, 32, 8, 900, 1024
    q = ol.uniform_bf16(0x21, 4.0, rows * Hq * 128).reshape(rows, Hq * 128)
    k = ol.uniform_bf16(0x22, 4.0, rows * Hk * 128).reshape(rows, Hk * 128)
    v = ol.uniform_bf16(0x23, 4.0, rows * Hk * 128).reshape(rows, Hk * 128)
    q_rot = torch.empty((rows, Hq * 128), dtype=torch.int16, device="cuda")
    k_rot = torch.empty((rows, Hk * 128), dtype=torch.int16, device="cuda")
    arena = L.KvArena(16, Hk, stride, fill=0xEE)
    L.call("granite4_kernel_verify_qkv_stage", dev(q), dev(k), dev(v), dc[base:], ds[base:], base,
           rows, Hq, Hk, 128, stride, q_rot, k_rot, arena.k, arena.v, None)
    pos = np.arange(base, base + rows)
    np.testing.assert_array_equal(host(q_rot).reshape(rows, Hq, 128),
                                  ol.rope_rows(q.reshape(rows, Hq, 128), pos, c, s))
    kr = ol.rope_rows(k.reshape(rows, Hk, 128), pos, c, s)
    np.testing.assert_array_equal(host(k_rot).reshape(rows, Hk, 128), kr)
    ck, cv, _, _ = _oracle_arena(16, 128, Hk, stride)
    want = ol.rope_append(None, kr.reshape(rows, -1), v, None, None, pos, pos, 16, 128, stride, Hk,
                          rotate_k=False, cache_k=ck, cache_v=cv, k_scale=np.zeros(1, np.float32),
                          v_scale=np.zeros(1, np.float32))
    _arena_compare(arena, want, 16, 128, Hk, stride)


@pytest.mark.parametrize("bits", [16, 8, 4, 5])
def test_multi_rope_append(tables, bits):
    """8 sessions at random positions in [0, 65536) with their own page tables
    (BASELINE config 2 shape); K quantised from its bf16 rounding."""
    note(f"multi rope append bits={bits}")
    c, s, dc, ds = tables
    n, Hq, Hk = 8, 32, 8
    pool_pages = 64
    stride = pool_pages * 16
    rs = np.random.default_rng(40 + bits)
    pos, tables_pt = ol.config2_page_tables(rs, n, pool_pages)
    assert pos.max() >= 32768, "the draw should reach the upper half of [0, 65536)"
    d_pts = [dev(t) for t in tables_pt]
    M = L.multi_rows_struct()
    m = M()
    m.n = n
    for i in range(n):
        m.pos[i] = int(pos[i])
        m.pt[i] = d_pts[i].data_ptr()
    d_m = torch.from_numpy(np.frombuffer(bytes(m), np.uint8).copy()).cuda()
    q = ol.uniform_bf16(0x31 + bits, 4.0, n * Hq * 128).reshape(n, Hq * 128)
    k = ol.uniform_bf16(0x32 + bits, 4.0, n * Hk * 128).reshape(n, Hk * 128)
    v = ol.uniform_bf16(0x33 + bits, 4.0, n * Hk * 128).reshape(n, Hk * 128)
    arena = L.KvArena(bits, Hk, stride, fill=0xEE)
    q_rot = torch.empty((n, Hq * 128), dtype=torch.int16, device="cuda")
    L.call("granite4_multi_rope_append", dev(q), dev(k), dev(v), dc, ds, d_m, n, Hq, Hk, 128, bits,
           arena.k, arena.v, arena.k_scale, arena.v_scale, stride, q_rot)
    arows = np.array([tables_pt[i][pos[i]] for i in range(n)], np.int32)
    ck, cv, ks, vs = _oracle_arena(bits, 128, Hk, stride)
    want = ol.rope_append(q, k, v, c, s, pos, arows, bits, 128, stride, Hk, k_round_bf16=True,
                          cache_k=ck, cache_v=cv, k_scale=ks, v_scale=vs)
    np.testing.assert_array_equal(host(q_rot), want[0])
    _arena_compare(arena, want, bits, 128, Hk, stride)
    # rope-only multi form on q
    out = torch.empty_like(q_rot)
    L.call("granite4_multi_rope", dev(q), dc, ds, d_m, n, Hq, 128, out)
    np.testing.assert_array_equal(host(out), want[0])


@pytest.mark.parametrize("bits", [8, 5])
def test_decode_rope_append_at_pos(tables, bits):
    note(f"decode rope_append_at_pos bits={bits}")
    c, s, dc, ds = tables
    Hq, Hk, stride = 32, 8, 8192
    q = ol.uniform_bf16(0x41, 4.0, Hq * 128).reshape(1, -1)
    k = ol.uniform_bf16(0x42, 4.0, Hk * 128).reshape(1, -1)
    v = ol.uniform_bf16(0x43, 4.0, Hk * 128).reshape(1, -1)
    p = 4321
    pt = np.random.default_rng(1).permutation(stride).astype(np.int32)
    arena = L.KvArena(bits, Hk, stride, fill=0xEE)
    q_rot = torch.empty((1, Hq * 128), dtype=torch.int16, device="cuda")
    L.call("granite4_rope_append_at_pos", dev(q), dev(k), dev(v), dc, ds, 65536,
           dev(np.array([p], np.int32)), dev(pt), Hq, Hk, 128, bits, 128, q_rot, arena.k, arena.v,
           arena.k_scale, arena.v_scale, stride)
    ck, cv, ks, vs = _oracle_arena(bits, 128, Hk, stride)
    want = ol.rope_append(q, k, v, c, s, [p], [pt[p]], bits, 128, stride, Hk, k_round_bf16=True,
                          cache_k=ck, cache_v=cv, k_scale=ks, v_scale=vs)
    np.testing.assert_array_equal(host(q_rot), want[0])
    _arena_compare(arena, want, bits, 128, Hk, stride)


def test_out_of_range_rows_are_skipped(tables):
    note("out of range rows")
    c, s, dc, ds = tables
    rows, Hk, stride = 4, 8, 16
    kx = ol.uniform_bf16(0x51, 4.0, rows * Hk * 128).reshape(rows, Hk * 128)
    arena = L.KvArena(8, Hk, stride, fill=0xEE)
    arows = np.array([0, -1, 16, 5], np.int32)
    d_k = dev(kx)
    L.rope_append(arena, None, d_k, d_k, dc, ds, base_pos=0, arena_rows=dev(arows), rotate_k=False)
    k = host(arena.k)
    assert (k[:, 1:5] == 0xEE).all() and (k[:, 6:] == 0xEE).all()
    assert not (k[:, 0] == 0xEE).all() and not (k[:, 5] == 0xEE).all()


# ----------------------------------------------------------------------------- grid-sync failure
@pytest.mark.parametrize("clear", [True, False])
@pytest.mark.parametrize("op,rows", [("norm", 8), ("norm", 512), ("norm", 8192), ("swiglu", 8),
                                     ("swiglu", 512), ("swiglu", 2048)])
def test_fp8_single_launch_wait_give_up_is_reported(op, rows, clear):
    """The single-launch FP8 forms' bounded wait, forced by the host to give
    up at once (spin limit 0: workgroup 0 publishes a NaN maximum without
    polling, so every kernel exits normally): the scale is NaN and the sticky
    error word reads 1 until cleared. The next call on the same workspace is
    correct whether or not the caller cleared it first, also on other inputs
    than the failed call's (8 rows is the one-hop synchronisation, whose
    slots would otherwise still carry the next tag)."""
    note(f"fp8 sync give-up {op} rows={rows} clear={clear}")
    work = L.fp8_workspace()
    assert L.fp8_sync_status(work) == 0
    if op == "norm":
        cols = 4096
        xs = [dev(_hidden(rows, cols, 0xD1)), dev(_hidden(rows, cols, 0xD4))]
        w_h = ol.normal_bf16(0xD2, 1.0, 0.1, cols)
        w = dev(w_h)
        codes = torch.empty((rows, cols), dtype=torch.uint8, device="cuda")

        def run(i, scale, wk):
            L.call("granite4_add_rmsnorm_fp8", xs[i], None, 1.0, w, 1e-5, rows, cols, None, codes,
                   scale, wk)
    else:
        I_ = 12800
        gus = [dev(ol.normal_bf16(0xD3, 0.0, 1.0, rows * 2 * I_).reshape(rows, 2 * I_)),
               dev(ol.normal_bf16(0xD5, 0.0, 3.0, rows * 2 * I_).reshape(rows, 2 * I_))]
        codes = torch.empty((rows, I_), dtype=torch.uint8, device="cuda")

        def run(i, scale, wk):
            L.call("granite4_swiglu_fp8", gus[i], rows, I_, codes, scale, wk, None)
    fresh = L.fp8_workspace()
    want_scale, want_codes = [], []
    for i in range(2):
        sc = torch.empty(1, dtype=torch.float32, device="cuda")
        run(i, sc, fresh)
        want_scale.append(host(sc)[0])
        want_codes.append(host(codes).copy())
    assert want_scale[0] != want_scale[1]
    good = torch.empty(1, dtype=torch.float32, device="cuda")
    run(0, good, work)
    assert host(good)[0] == want_scale[0]
    assert L.fp8_sync_status(work) == 0
    prev = L.set_sync_spin_limit(0)
    try:
        bad = torch.empty(1, dtype=torch.float32, device="cuda")
        run(1, bad, work)
        torch.cuda.synchronize()
    finally:
        L.set_sync_spin_limit(prev)
    assert np.isnan(host(bad)[0])
    assert L.fp8_sync_status(work) == 1
    if clear:
        assert L.fp8_sync_status(work, clear=True) == 1
        assert L.fp8_sync_status(work) == 0
    for i in (1, 0):
        again = torch.empty(1, dtype=torch.float32, device="cuda")
        run(i, again, work)
        assert host(again)[0] == want_scale[i]
        np.testing.assert_array_equal(host(codes), want_codes[i])
    assert L.fp8_sync_status(work) == (0 if clear else 1)


@pytest.mark.parametrize("rows", [8, 512, 2048])
def test_swiglu_fp8_nan_inputs_are_ignored_by_the_scale(rows):
    """A NaN act (from a NaN gate) is skipped by the per-tensor maximum, as
    the reference quantiser's `a > amax` skips it (gpu_pack.cc:44-46); the
    single-launch forms take that maximum on bf16 bit patterns, where a NaN
    pattern would otherwise win."""
    note(f"swiglu_fp8 NaN rows={rows}")
    I_ = 12800
    gu = ol.normal_bf16(0xE5 + rows, 0.0, 1.0, rows * 2 * I_).reshape(rows, 2 * I_)
    gu[rows // 2, 17] = 0x7FC1   # NaN gate
    gu[0, I_ + 3] = 0xFFC0       # NaN up (negative sign bit)
    d_gu = dev(gu)
    act = torch.empty((rows, I_), dtype=torch.int16, device="cuda")
    L.call("granite4_swiglu", d_gu, rows, I_, act)
    work = L.fp8_workspace()
    for mode in (0, 1):
        prev = L.set_fp8_launch_mode(mode)
        try:
            codes = torch.empty((rows, I_), dtype=torch.uint8, device="cuda")
            scale = torch.empty(1, dtype=torch.float32, device="cuda")
            L.call("granite4_swiglu_fp8", d_gu, rows, I_, codes, scale, work, None)
        finally:
            L.set_fp8_launch_mode(prev)
        a = host(act)
        assert np.isnan(ol.bf16_to_f32(a[rows // 2, 17]))
        _fp8_check(host(codes), host(scale)[0], a)
        assert np.isfinite(host(scale)[0]) and host(scale)[0] > 0


@pytest.mark.parametrize("rows", [8, 512, 8192])
def test_add_rmsnorm_fp8_nan_row_is_ignored_by_the_scale(rows):
    """A NaN in one residual row makes that row's normed values NaN; the
    per-tensor maximum skips them (the reference quantiser's `a > amax`), in
    the single-launch forms as in the two-launch form."""
    note(f"add_rmsnorm_fp8 NaN rows={rows}")
    cols = 4096
    res = _hidden(rows, cols, 0xE9 + rows)
    res[rows // 2, 100] = 0x7FC0  # NaN
    w = ol.normal_bf16(0xEA, 1.0, 0.1, cols)
    d_res, d_w = dev(res), dev(w)
    no = torch.empty_like(d_res)
    L.call("granite4_add_rmsnorm", d_res, None, 1.0, d_w, 1e-5, rows, cols, None, no)
    work = L.fp8_workspace()
    for mode in (0, 1):
        prev = L.set_fp8_launch_mode(mode)
        try:
            codes = torch.empty((rows, cols), dtype=torch.uint8, device="cuda")
            scale = torch.empty(1, dtype=torch.float32, device="cuda")
            L.call("granite4_add_rmsnorm_fp8", d_res, None, 1.0, d_w, 1e-5, rows, cols, None,
                   codes, scale, work)
        finally:
            L.set_fp8_launch_mode(prev)
        _fp8_check(host(codes), host(scale)[0], host(no))
        assert np.isfinite(host(scale)[0]) and host(scale)[0] > 0


@pytest.mark.parametrize("op,rows", [("norm", 8), ("norm", 512), ("norm", 8192), ("swiglu", 8),
                                     ("swiglu", 512), ("swiglu", 8192)])
def test_fp8_cooperative_launch_mode(op, rows):
    """FP8 launch mode 2 (the single-launch forms through
    hipLaunchCooperativeKernel): codes and scale identical to mode 0, eagerly
    and as a captured graph replayed twice on other inputs."""
    note(f"fp8 cooperative launch {op} rows={rows}")
    work = L.fp8_workspace()
    if op == "norm":
        cols = 4096
        xs = [dev(_hidden(rows, cols, 0xC1 + i)) for i in range(2)]
        w = dev(ol.normal_bf16(0xC3, 1.0, 0.1, cols))
        src = torch.empty_like(xs[0])
        codes = torch.empty((rows, cols), dtype=torch.uint8, device="cuda")

        def run(x, scale):
            L.call("granite4_add_rmsnorm_fp8", x, None, 1.0, w, 1e-5, rows, cols, None, codes,
                   scale, work)
    else:
        I_ = 12800
        xs = [dev(ol.normal_bf16(0xC4 + i, 0.0, 1.0 + i, rows * 2 * I_).reshape(rows, 2 * I_))
              for i in range(2)]
        src = torch.empty_like(xs[0])
        codes = torch.empty((rows, I_), dtype=torch.uint8, device="cuda")

        def run(x, scale):
            L.call("granite4_swiglu_fp8", x, rows, I_, codes, scale, work, None)
    want = []
    for x in xs:
        sc = torch.empty(1, dtype=torch.float32, device="cuda")
        run(x, sc)
        want.append((host(codes).copy(), host(sc)[0]))
    prev = L.set_fp8_launch_mode(2)
    try:
        for x, (c, s) in zip(xs, want):
            sc = torch.empty(1, dtype=torch.float32, device="cuda")
            run(x, sc)
            np.testing.assert_array_equal(host(codes), c)
            assert host(sc)[0] == s
        sc = torch.empty(1, dtype=torch.float32, device="cuda")
        stream = torch.cuda.Stream()
        g = torch.cuda.CUDAGraph()
        torch.cuda.synchronize()
        L.use_stream(stream)
        try:
            with torch.cuda.graph(g, stream=stream):
                run(src, sc)
        finally:
            L.use_stream()
        for i in (1, 0):
            src.copy_(xs[i])
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            np.testing.assert_array_equal(host(codes), want[i][0])
            assert host(sc)[0] == want[i][1]
    finally:
        L.set_fp8_launch_mode(prev)
    assert L.fp8_sync_status(work) == 0
