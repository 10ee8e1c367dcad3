"""GPU parity at the BASELINE configs' full sizes, through the C ABI.

- config 5: the 40-layer x T=32768 bf16 sequence (add+RMSNorm, RoPE + bf16
  paged-KV write, add+RMSNorm, SwiGLU per layer, GEMM outputs replaced by
  seeded bf16 tensors). Every layer's outputs are checked finite on the
  device, sampled rows of every op are checked against the oracle on the same
  inputs (residual and RoPE / KV bit-exact, normed and act within 1 bf16 ulp),
  and layer 0 is checked against the oracle on every row;
- config 4: SwiGLU -> FP8 at 8192 x 12800 (the held-and-streamed kernel),
  RoPE + K5V4 group-32 append at 8192 rows from position 57344 through a
  random page table;
- config 3: SwiGLU -> FP8 and RoPE + int8 append at exactly 512 rows;
- the reference entry points granite4_rope_tables_build (allocating) and
  granite4_multi_kv_append (forward_gpu.cu:3915) in all four KV formats;
- the embedding multiplier against a closed form (power-of-two multipliers
  scale exactly, so bf16(m * x) is x with its exponent moved).
"""
import ctypes
import sys

import numpy as np
import pytest
import torch

import oracle_lib as ol
from pkg import layerops

pytestmark = pytest.mark.gpu

L = None
H, I_, HQ, HK, D = 4096, 12800, 32, 8, 128


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


@pytest.fixture(scope="module")
def tables():
    c, s = ol.rope_tables(1e7, 128, 65536)
    return c, s, dev(c), dev(s)


# ----------------------------------------------------------------------------- config 5
def test_stress_sequence_40_layers_T32768(tables):
    """BASELINE config 5 as a correctness run: 40 layers of the bf16 sequence
    over the full [32768, 4096] residual stream and [32768, 12800] MLP
    activations, GEMM outputs replaced by seeded bf16 tensors."""
    c, s, dc, ds = tables
    T, layers = 32768, 40
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0x5757)

    def randn(shape, std=1.0, mean=0.0):
        return torch.empty(shape, dtype=torch.float32, device="cuda").normal_(
            mean, std, generator=gen).to(torch.bfloat16)

    res = randn((T, H))
    ch = torch.randperm(H, generator=gen, device="cuda")[: H // 100]
    res[:, ch] = (res[:, ch].float() * 20).to(torch.bfloat16)
    gamma_a = randn((H,), 0.1, 1.0)
    gamma_m = randn((H,), 0.1, 1.0)
    w_a, w_m = host(gamma_a), host(gamma_m)
    branch = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
    normed = torch.empty_like(branch)
    qkv = torch.empty((T, (HQ + 2 * HK) * D), dtype=torch.bfloat16, device="cuda")
    q_rot = torch.empty((T, HQ * D), dtype=torch.bfloat16, device="cuda")
    gu = torch.empty((T, 2 * I_), dtype=torch.bfloat16, device="cuda")
    act = torch.empty((T, I_), dtype=torch.bfloat16, device="cuda")
    arena = L.KvArena(16, HK, T, fill=0xEE)
    # positions 0..T-1 through a random page table of 16-row pages
    bt = np.random.default_rng(0x5758).permutation(T // 16).astype(np.int32)
    pt = ol.row_table(bt, T)
    d_pt = dev(pt)
    rs = np.random.default_rng(0x5759)
    mult_a, mult_m = 0.5, 0.22  # Granite's residual multiplier is < 1

    def finite(t):
        return bool(torch.isfinite(t).all().item())

    for layer in range(layers):
        full = layer == 0
        rows = np.arange(T) if full else np.sort(np.concatenate(
            [[0, T - 1], rs.choice(np.arange(1, T - 1), 14, replace=False)]))
        d_rows = torch.from_numpy(rows).cuda()
        note(f"config 5 layer {layer} ({'all' if full else len(rows)} rows checked)")
        # attention half: residual += 0.5 * branch, RMSNorm
        branch.normal_(0.0, 1.0, generator=gen)
        res_in, br_in = host(res[d_rows]), host(branch[d_rows])
        L.call("granite4_add_rmsnorm", res, branch, mult_a, gamma_a, 1e-5, T, H, res, normed)
        ro_w, no_w = ol.add_rmsnorm(res_in, br_in, mult_a, w_a, 1e-5)
        np.testing.assert_array_equal(host(res[d_rows]), ro_w)
        d = ulp_diff(host(normed[d_rows]), no_w)
        assert d.max() <= 1 and (d == 0).mean() >= 0.9999, (layer, d.max())
        assert finite(res) and finite(normed), layer
        # RoPE on q / k and the bf16 KV write through the page table
        qkv.normal_(0.0, 1.0, generator=gen)
        L.rope_append(arena, qkv[:, :HQ * D], qkv[:, HQ * D:(HQ + HK) * D],
                      qkv[:, (HQ + HK) * D:], dc, ds, base_pos=0, d_pt=d_pt, q_rot=q_rot)
        x = host(qkv[d_rows])
        n = len(rows)
        want = ol.rope_append(x[:, :HQ * D], x[:, HQ * D:(HQ + HK) * D], x[:, (HQ + HK) * D:],
                              c, s, rows, np.arange(n), 16, 128, n, HK)
        np.testing.assert_array_equal(host(q_rot[d_rows]), want[0])
        d_arows = torch.from_numpy(pt[rows].astype(np.int64)).cuda()
        np.testing.assert_array_equal(host(arena.k[:, d_arows]).reshape(-1), want[1])
        np.testing.assert_array_equal(host(arena.v[:, d_arows]).reshape(-1), want[2])
        assert finite(q_rot), layer
        # MLP half: residual += 0.22 * branch, RMSNorm, then SwiGLU of gate|up
        branch.normal_(0.0, 1.0, generator=gen)
        res_in, br_in = host(res[d_rows]), host(branch[d_rows])
        L.call("granite4_add_rmsnorm", res, branch, mult_m, gamma_m, 1e-5, T, H, res, normed)
        ro_w, no_w = ol.add_rmsnorm(res_in, br_in, mult_m, w_m, 1e-5)
        np.testing.assert_array_equal(host(res[d_rows]), ro_w)
        assert ulp_diff(host(normed[d_rows]), no_w).max() <= 1, layer
        gu.normal_(0.0, 1.0, generator=gen)
        L.call("granite4_swiglu", gu, T, I_, act)
        d = ulp_diff(host(act[d_rows]), ol.swiglu(host(gu[d_rows])))
        assert d.max() <= 1, (layer, d.max())
        assert finite(res) and finite(normed) and finite(act), layer
        del d_rows
    torch.cuda.synchronize()


# ----------------------------------------------------------------------------- config 4
def _fp8_vs_oracle(codes, scale, act_gpu, gu):
    """FP8 codes / scale of SwiGLU: bit-exact against the reference quantiser of
    the GPU's own act, and against the oracle's act wherever the two acts agree
    (the SwiGLU itself is allowed 1 bf16 ulp)."""
    want_c, want_s = ol.fp8_quantize(act_gpu)
    assert scale == np.float32(want_s)
    np.testing.assert_array_equal(codes, want_c)
    act_o = ol.swiglu(gu)
    d = ulp_diff(act_gpu, act_o)
    assert d.max() <= 1
    oc, os_ = ol.fp8_quantize(act_o)
    if os_ == want_s:
        same = d == 0
        np.testing.assert_array_equal(codes[same], oc[same])
    return (d == 0).mean()


@pytest.mark.parametrize("rows", [512, 8192])
def test_swiglu_fp8_config_sizes(rows):
    """512 rows: the single-launch register-held kernel (config 3). 8192 rows:
    the persistent kernel that holds part of act on chip across the grid
    synchronisation and streams the rest twice (config 4)."""
    note(f"swiglu_fp8 rows={rows}")
    gu = ol.normal_bf16(0x5F1 + rows, 0.0, 1.0, rows * 2 * I_).reshape(rows, 2 * I_)
    d_gu = dev(gu)
    work = L.fp8_workspace()
    act = torch.empty((rows, I_), dtype=torch.int16, device="cuda")
    L.call("granite4_swiglu", d_gu, rows, I_, act)
    codes = torch.empty((rows, I_), dtype=torch.uint8, device="cuda")
    scale = torch.empty(1, dtype=torch.float32, device="cuda")
    L.call("granite4_swiglu_fp8", d_gu, rows, I_, codes, scale, work, None)
    exact = _fp8_vs_oracle(host(codes), host(scale)[0], host(act), gu)
    note(f"  act exact fraction {exact:.6f}")
    prev = L.set_fp8_launch_mode(1)
    try:
        codes2 = torch.empty_like(codes)
        scale2 = torch.empty_like(scale)
        L.call("granite4_swiglu_fp8", d_gu, rows, I_, codes2, scale2, work, None)
    finally:
        L.set_fp8_launch_mode(prev)
    np.testing.assert_array_equal(host(codes2), host(codes))
    assert host(scale2)[0] == host(scale)[0]


def test_rope_append_k5v4_g32_T8192_at_57344(tables):
    """Config 4's RoPE + K5 / V4 group-32 append: 8192 rows at positions
    57344..65535 through a random page table (the per-token kernel)."""
    note("rope_append k5v4 g32 T=8192 @57344")
    c, s, dc, ds = tables
    T, pos0 = 8192, 57344
    stride = T + 64
    bt = np.random.default_rng(0x4B5).permutation(stride // 16).astype(np.int32)
    pt_full = np.full(pos0 + T, -1, np.int32)
    pt_full[pos0:] = ol.row_table(bt, T + 16)[16:T + 16]  # skip the first page
    qkv = ol.normal_bf16(0x4B6, 0.0, 1.0, T * (HQ + 2 * HK) * D).reshape(T, -1)
    d_qkv = dev(qkv)
    arena = L.KvArena(5, HK, stride, group=32, fill=0xEE)
    q_rot = L.rope_append(arena, d_qkv[:, :HQ * D], d_qkv[:, HQ * D:(HQ + HK) * D],
                          d_qkv[:, (HQ + HK) * D:], dc, ds, base_pos=pos0, d_pt=dev(pt_full))
    kb, vb = L.kv_row_bytes(5)
    ck = np.full(HK * stride * kb, 0xEE, np.uint8)
    cv = np.full(HK * stride * vb, 0xEE, np.uint8)
    ks = np.zeros(HK * stride * 4, np.float32)
    vs = np.zeros(HK * stride * 4, np.float32)
    pos = np.arange(pos0, pos0 + T)
    want = ol.rope_append(qkv[:, :HQ * D], qkv[:, HQ * D:(HQ + HK) * D], qkv[:, (HQ + HK) * D:],
                          c, s, pos, pt_full[pos], 5, 32, stride, HK, cache_k=ck, cache_v=cv,
                          k_scale=ks, v_scale=vs)
    np.testing.assert_array_equal(host(q_rot), want[0])
    np.testing.assert_array_equal(host(arena.k).reshape(-1), want[1])
    np.testing.assert_array_equal(host(arena.v).reshape(-1), want[2])
    np.testing.assert_array_equal(host(arena.k_scale).reshape(-1), want[3])
    np.testing.assert_array_equal(host(arena.v_scale).reshape(-1), want[4])


def test_rope_append_int8_T512_fresh_pages(tables):
    """Config 3's RoPE + int8 append: 512 rows at positions 0..511 into a
    contiguous run of fresh pages (the per-token kernel, exactly 512 rows)."""
    note("rope_append int8 T=512")
    c, s, dc, ds = tables
    T, first = 512, 7 * 16
    stride = first + T + 16
    pt = (np.arange(T) + first).astype(np.int32)
    qkv = ol.normal_bf16(0x4B7, 0.0, 1.0, T * (HQ + 2 * HK) * D).reshape(T, -1)
    d_qkv = dev(qkv)
    arena = L.KvArena(8, HK, stride, fill=0xEE)
    q_rot = L.rope_append(arena, d_qkv[:, :HQ * D], d_qkv[:, HQ * D:(HQ + HK) * D],
                          d_qkv[:, (HQ + HK) * D:], dc, ds, base_pos=0, d_pt=dev(pt))
    ck = np.full(HK * stride * 128, 0xEE, np.uint8)
    cv = np.full(HK * stride * 128, 0xEE, np.uint8)
    ks = np.zeros(HK * stride, np.float32)
    vs = np.zeros(HK * stride, np.float32)
    want = ol.rope_append(qkv[:, :HQ * D], qkv[:, HQ * D:(HQ + HK) * D], qkv[:, (HQ + HK) * D:],
                          c, s, np.arange(T), pt, 8, 128, stride, HK, cache_k=ck, cache_v=cv,
                          k_scale=ks, v_scale=vs)
    np.testing.assert_array_equal(host(q_rot), want[0])
    np.testing.assert_array_equal(host(arena.k).reshape(-1), want[1])
    np.testing.assert_array_equal(host(arena.v).reshape(-1), want[2])
    np.testing.assert_array_equal(host(arena.k_scale).reshape(-1), want[3])
    np.testing.assert_array_equal(host(arena.v_scale).reshape(-1), want[4])


# ----------------------------------------------------------------------------- boundary gaps
def _hip():
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    hip.hipMemcpy.restype = ctypes.c_int
    return hip


@pytest.mark.parametrize("max_pos", [8192, 65536])
def test_rope_tables_build_allocating_reference_api(tables, max_pos):
    """granite4_rope_tables_build (kernels_phase2.cu:868) allocates the tables
    and hands them to the caller: bit-exact against the oracle, usable by the
    reference-signature RoPE launcher, then freed."""
    note(f"rope_tables_build max_pos={max_pos}")
    c, s = ol.rope_tables(1e7, 128, max_pos)
    pc, ps = ctypes.c_void_p(), ctypes.c_void_p()
    rc = L.lib.granite4_rope_tables_build(1e7, 128, max_pos, ctypes.byref(pc), ctypes.byref(ps))
    assert rc == 0 and pc.value and ps.value
    try:
        hip = _hip()
        gc = np.empty_like(c)
        gs = np.empty_like(s)
        assert hip.hipMemcpy(gc.ctypes.data, pc.value, gc.nbytes, 2) == 0
        assert hip.hipMemcpy(gs.ctypes.data, ps.value, gs.nbytes, 2) == 0
        np.testing.assert_array_equal(gc, c)
        np.testing.assert_array_equal(gs, s)
        rows = 96
        x = ol.uniform_bf16(0x1340, 4.0, rows * 128).reshape(rows, 1, 128)
        out = torch.empty((rows, 128), dtype=torch.int16, device="cuda")
        L.call("granite4_kernel_rope", dev(x), pc.value, ps.value, rows, 128, out)
        np.testing.assert_array_equal(host(out),
                                      ol.rope_rows(x, np.arange(rows), c, s).reshape(rows, 128))
        torch.cuda.synchronize()
    finally:
        assert L.lib.granite4_rope_tables_free(pc.value, ps.value) == 0
    # invalid arguments: -1, nothing allocated
    assert L.lib.granite4_rope_tables_build(1e7, 127, 16, ctypes.byref(pc), ctypes.byref(ps)) == -1
    assert L.lib.granite4_rope_tables_build(1e7, 128, 0, ctypes.byref(pc), ctypes.byref(ps)) == -1


def test_rope_table_registry_bounds_many_tables():
    """The length registry behind the reference-signature RoPE launchers,
    which carry no table length: 70 tables from granite4_rope_tables_build
    (past the registry's 64 lock-free slots, so the overflow map is used
    too), max_pos 8 + i. A 80-row granite4_kernel_rope over table i rotates
    rows < max_pos exactly as the oracle and leaves the rest unwritten; after
    every table is freed, a freed slot is reused by a new table with its own
    bound."""
    note("rope table registry")
    rows = 80
    x = ol.uniform_bf16(0x1341, 4.0, rows * 128).reshape(rows, 1, 128)
    dx = dev(x)
    built = []
    try:
        for i in range(70):
            pc, ps = ctypes.c_void_p(), ctypes.c_void_p()
            assert L.lib.granite4_rope_tables_build(1e7, 128, 8 + i, ctypes.byref(pc),
                                                   ctypes.byref(ps)) == 0
            built.append((pc.value, ps.value, 8 + i))
        full_c, full_s = ol.rope_tables(1e7, 128, 80)
        want_all = ol.rope_rows(x, np.arange(rows), full_c, full_s).reshape(rows, 128)
        for i in (0, 1, 40, 63, 64, 65, 69):
            pc, ps, mp = built[i]
            out = torch.full((rows, 128), 0x7E7E, dtype=torch.int16, device="cuda")
            L.call("granite4_kernel_rope", dx, pc, ps, rows, 128, out)
            got = host(out)
            np.testing.assert_array_equal(got[:mp], want_all[:mp])
            assert (got[mp:] == 0x7E7E).all(), i
    finally:
        for pc, ps, _ in built:
            assert L.lib.granite4_rope_tables_free(pc, ps) == 0
    pc, ps = ctypes.c_void_p(), ctypes.c_void_p()
    assert L.lib.granite4_rope_tables_build(1e7, 128, 20, ctypes.byref(pc), ctypes.byref(ps)) == 0
    try:
        out = torch.full((rows, 128), 0x7E7E, dtype=torch.int16, device="cuda")
        L.call("granite4_kernel_rope", dx, pc.value, ps.value, rows, 128, out)
        got = host(out)
        c20, s20 = ol.rope_tables(1e7, 128, 20)
        np.testing.assert_array_equal(got[:20], ol.rope_rows(x[:20], np.arange(20), c20, s20).reshape(20, 128))
        assert (got[20:] == 0x7E7E).all()
    finally:
        assert L.lib.granite4_rope_tables_free(pc.value, ps.value) == 0


@pytest.mark.parametrize("bits", [16, 8, 4, 5])
def test_multi_kv_append_reference_api(bits):
    """granite4_multi_kv_append (forward_gpu.cu:3915): 8 sessions at random
    positions, each through its own random page table; K is written as given
    (no rotation). Untouched arena rows keep their fill."""
    note(f"multi_kv_append bits={bits}")
    n, pool_pages = 8, 64
    stride = pool_pages * 16
    rs = np.random.default_rng(0x3915 + bits)
    pos, pts = ol.config2_page_tables(rs, n, pool_pages)
    d_pts = [dev(t) for t in pts]
    m = L.multi_rows_struct()()
    m.n = n
    for i in range(n):
        m.pos[i] = int(pos[i])
        m.pt[i] = d_pts[i].data_ptr()
    d_m = torch.from_numpy(np.frombuffer(bytes(m), np.uint8).copy()).cuda()
    k = ol.uniform_bf16(0x61 + bits, 4.0, n * HK * D).reshape(n, HK * D)
    v = ol.uniform_bf16(0x62 + bits, 3.0, n * HK * D).reshape(n, HK * D)
    k[2, :D] = 0  # a zero head row: scale 0, zero codes
    arena = L.KvArena(bits, HK, stride, fill=0xEE)
    L.call("granite4_multi_kv_append", dev(k), dev(v), bits, arena.k, arena.v,
           arena.k_scale if bits != 16 else None, arena.v_scale if bits != 16 else None, d_m, n,
           stride, HK, D)
    kb, vb = L.kv_row_bytes(bits)
    ck = np.full(HK * stride * kb, 0xEE, np.uint8)
    cv = np.full(HK * stride * vb, 0xEE, np.uint8)
    ks = np.zeros(HK * stride, np.float32)
    vs = np.zeros(HK * stride, np.float32)
    arows = np.array([pts[i][pos[i]] for i in range(n)], np.int32)
    want = ol.rope_append(None, k, v, None, None, pos, arows, bits, 128, stride, HK,
                          rotate_k=False, cache_k=ck, cache_v=cv, k_scale=ks, v_scale=vs)
    np.testing.assert_array_equal(host(arena.k).reshape(-1), want[1])
    np.testing.assert_array_equal(host(arena.v).reshape(-1), want[2])
    if bits != 16:
        np.testing.assert_array_equal(host(arena.k_scale).reshape(-1), want[3])
        np.testing.assert_array_equal(host(arena.v_scale).reshape(-1), want[4])


@pytest.mark.parametrize("mult", [0.5, 2.0, 0.125])
def test_embed_power_of_two_multiplier_closed_form(mult):
    """bf16(m * x) for a power-of-two m and normal x is x with its exponent
    moved, exactly: the gather must return that, independent of the oracle."""
    note(f"embed closed form mult={mult}")
    vocab, rows = 512, 300
    emb = ol.normal_bf16(0xE7, 0.0, 0.02, vocab * H).reshape(vocab, H)
    emb[5, :64] = 0
    emb[5, 64:128] = 0x8000  # -0.0
    tok = (ol.u32(0xE8, rows) % vocab).astype(np.int32)
    tok[:3] = 5
    out = torch.empty((rows, H), dtype=torch.int16, device="cuda")
    L.call("granite4_embed_rows", dev(tok), rows, dev(emb), vocab, H, mult, out)
    x = ol.bf16_to_f32(emb[tok])
    want = (x * np.float32(mult)).astype(np.float32)
    assert np.all(np.abs(want[want != 0]) >= 2.0 ** -126)  # no subnormal results
    want_bits = (want.view(np.uint32) >> 16).astype(np.uint16)
    assert np.all((want.view(np.uint32) & 0xFFFF) == 0)  # exactly representable: no rounding
    np.testing.assert_array_equal(host(out), want_bits)
