"""GPU parity of the split-KV decode attention (granite4_attn_paged /
granite4_attn_split) against the oracle's g4o_attn_split on the same caches.

The kernel follows the oracle's structure exactly (64-position tiles, the same
splits, bf16 logits, bf16(p * v_scale) in the value product for one scale
per row, the dequantised bf16 path for scale groups of 32 / 64, the same
combine); what differs is the order of the f32 sums inside the MFMA and the
hardware exponential. Bar, per output element: within 2 bf16 steps of the
oracle's value, or within 2^-8 of max |V| where the output nearly cancels
(a logit whose f32 dot product lands on a bf16 rounding boundary can round
the other way and move one probability by 2^-8 of itself). The tests print
the fraction of bit-identical outputs.
"""
import numpy as np
import pytest
import torch

import oracle_lib as ol
from pkg import layerops

pytestmark = pytest.mark.gpu

HK, HQ, D = 8, 32, 128
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
    return t.cpu().numpy()


def make_cache(bits, group, stride, seed, kstd=0.5):
    """Random pool contents: bf16 values, or random codes with scales in
    [0.01, 0.11)."""
    rng = np.random.default_rng(seed)
    kb, vb = ol.KV_ROW_BYTES[bits]
    if bits == 16:
        ck = ol.normal_bf16(seed, 0.0, kstd, HK * stride * D).view(np.uint8)
        cv = ol.normal_bf16(seed + 1, 0.0, 1.0, HK * stride * D).view(np.uint8)
        return ck, cv, None, None
    ck = rng.integers(0, 256, HK * stride * kb, dtype=np.uint8)
    cv = rng.integers(0, 256, HK * stride * vb, dtype=np.uint8)
    ng = D // group
    ks = (rng.random(HK * stride * ng, dtype=np.float32) * 0.1 + 0.01).astype(np.float32)
    vs = (rng.random(HK * stride * ng, dtype=np.float32) * 0.1 + 0.01).astype(np.float32)
    if bits == 8:
        ks *= np.float32(0.05)  # int8 codes are 16x larger than int4 ones
    return ck, cv, ks, vs


def vmax(cv, vs, bits):
    if bits == 16:
        return float(np.abs(ol.bf16_to_f32(cv.view(np.uint16))).max())
    qmax = 127 if bits == 8 else 8
    return float(qmax * vs.max())


def check(got, want, vm, what):
    fa = ol.bf16_to_f32(got).astype(np.float64)
    fb = ol.bf16_to_f32(want).astype(np.float64)
    mag = np.maximum(np.abs(fa), np.abs(fb))
    step = np.where(mag > 0, 2.0 ** (np.floor(np.log2(np.maximum(mag, 1e-30))) - 7), 1e-30)
    ulps = np.abs(fa - fb) / step
    ok = (ulps <= 2) | (np.abs(fa - fb) <= 2.0 ** -8 * vm)
    note(f"  {what}: exact {np.mean(got == want):.4f}, max ulps {ulps.max():.1f}, "
         f"max |diff| / max|v| {np.abs(fa - fb).max() / vm:.2e}")
    assert ok.all(), f"{what}: {np.count_nonzero(~ok)} elements out of tolerance"


def run_paged(q, ck, cv, ks, vs, bits, group, stride, *, kv_base=0, d_pos=None, d_pt=None,
              row_pos=None, row_pts=None, max_len=0, window=0, scale=1.0 / 16):
    rows = q.shape[0]
    scratch = torch.zeros(L.call_size("granite4_attn_split_scratch_bytes", HQ, rows,
                                      max_len if max_len else stride),
                          dtype=torch.uint8, device="cuda")
    out = torch.empty((rows, HQ * D), dtype=torch.int16, device="cuda")
    keep = []
    rp_dev = rpt_dev = None
    if row_pos is not None:
        rp_dev = dev(np.asarray(row_pos, np.int32))
        keep = [dev(np.asarray(t, np.int32)) for t in row_pts]
        rpt_dev = torch.tensor([t.data_ptr() for t in keep], dtype=torch.int64, device="cuda")
    dks = None if ks is None else dev(ks)
    dvs = None if vs is None else dev(vs)
    L.call("granite4_attn_paged", dev(q), rows, HQ, HK, D, scale, dev(ck), dev(cv), dks, dvs,
           bits, group, stride, kv_base, d_pos, d_pt, rp_dev, rpt_dev, max_len, window, scratch,
           out)
    return host(out).view(np.uint16)


@pytest.mark.parametrize("bits", [16, 8, 4, 5])
@pytest.mark.parametrize("rows", [1, 4, 9])
def test_attn_contiguous(bits, rows):
    note(f"attn contiguous bits={bits} rows={rows}")
    stride = 400
    ck, cv, ks, vs = make_cache(bits, D, stride, 0xD0 + bits)
    q = ol.normal_bf16(0xD1 + rows, 0.0, 1.0, rows * HQ * D).reshape(rows, HQ * D)
    kv_base = 300 - rows
    got = run_paged(q, ck, cv, ks, vs, bits, D, stride, kv_base=kv_base)
    pos = [kv_base + r for r in range(rows)]
    want = ol.attn_split(q, ck, cv, ks, vs, bits, D, stride, pos, scale=1.0 / 16, Hk=HK)
    check(got, want, vmax(cv, vs, bits), f"bits {bits} rows {rows}")


@pytest.mark.parametrize("bits", [8, 16])
def test_attn_combine_give_up_is_reported(bits):
    """The fused combine's bounded wait, forced by the host to give up before
    polling (spin limit 0, so every kernel still exits normally): the outputs
    are NaN and the scratch's sticky error word reads 1. After the zero fill
    the error word asks for, the same scratch gives the oracle's result."""
    note(f"attn combine give-up bits={bits}")
    pages = 80
    stride = 16 * pages
    ck, cv, ks, vs = make_cache(bits, D, stride, 0xE5 + bits)
    pt = ol.row_table(np.random.default_rng(7 + bits).permutation(pages).astype(np.int32), stride)
    q = ol.normal_bf16(0xE6, 0.0, 1.0, HQ * D).reshape(1, HQ * D)
    pos = dev(np.array([1100], np.int32))
    scratch = torch.zeros(L.call_size("granite4_attn_split_scratch_bytes", HQ, 1, stride),
                          dtype=torch.uint8, device="cuda")
    dks = None if ks is None else dev(ks)
    dvs = None if vs is None else dev(vs)
    d_q, d_ck, d_cv, d_pt = dev(q), dev(ck), dev(cv), dev(pt)

    def run():
        out = torch.empty((1, HQ * D), dtype=torch.int16, device="cuda")
        L.call("granite4_attn_paged", d_q, 1, HQ, HK, D, 1.0 / 16, d_ck, d_cv, dks, dvs, bits, D,
               stride, 0, pos, d_pt, None, None, 0, 0, scratch, out)
        return host(out).view(np.uint16)

    prev_mode = L.set_attn_combine_mode(0)
    try:
        assert L.attn_sync_status(scratch) == 0
        prev = L.set_sync_spin_limit(0)
        try:
            bad = run()
            torch.cuda.synchronize()
        finally:
            L.set_sync_spin_limit(prev)
        assert ((bad & 0x7FFF) > 0x7F80).all(), "every output should be NaN after a give-up"
        assert L.attn_sync_status(scratch) == 1
        scratch.zero_()
        assert L.attn_sync_status(scratch) == 0
        got = run()
        assert L.attn_sync_status(scratch) == 0
    finally:
        L.set_attn_combine_mode(prev_mode)
    want = ol.attn_split(q, ck, cv, ks, vs, bits, D, stride, [1100], pts=[pt], scale=1.0 / 16,
                         Hk=HK)
    check(got, want, vmax(cv, vs, bits), f"bits {bits} after give-up")


@pytest.mark.parametrize("bits", [8, 16])
def test_attn_unmapped_split_block(bits):
    """A whole split block of positions without an arena row (page-table
    entries -1 for positions 256..511: one block of 4 splits at this stride)
    contributes nothing: the block publishes an empty partial rather than
    leaving the previous call's in its scratch slot (the first call, with
    every position mapped, fills that slot)."""
    note(f"attn unmapped split block bits={bits}")
    pages = 80
    stride = 16 * pages
    ck, cv, ks, vs = make_cache(bits, D, stride, 0xE1 + bits)
    pt = ol.row_table(np.random.default_rng(bits).permutation(pages).astype(np.int32), stride)
    pt_hole = pt.copy()
    pt_hole[256:512] = -1
    q = ol.normal_bf16(0xE2, 0.0, 1.0, HQ * D).reshape(1, HQ * D)
    pos = dev(np.array([1000], np.int32))
    scratch = torch.empty(L.call_size("granite4_attn_split_scratch_bytes", HQ, 1, stride),
                          dtype=torch.uint8, device="cuda")
    dks = None if ks is None else dev(ks)
    dvs = None if vs is None else dev(vs)
    outs = []
    for table in (pt, pt_hole):
        out = torch.empty((1, HQ * D), dtype=torch.int16, device="cuda")
        L.call("granite4_attn_paged", dev(q), 1, HQ, HK, D, 1.0 / 16, dev(ck), dev(cv), dks, dvs,
               bits, D, stride, 0, pos, dev(table), None, None, 0, 0, scratch, out)
        outs.append(host(out).view(np.uint16))
    for got, table in zip(outs, (pt, pt_hole)):
        want = ol.attn_split(q, ck, cv, ks, vs, bits, D, stride, [1000], pts=[table],
                             scale=1.0 / 16, Hk=HK)
        check(got, want, vmax(cv, vs, bits), f"bits {bits} hole={table is pt_hole}")
    assert not np.array_equal(outs[0], outs[1])


@pytest.mark.parametrize("bits,group", [(8, 128), (5, 128), (16, 128), (5, 32), (4, 32), (8, 64)])
def test_attn_paged_device_pos(bits, group):
    note(f"attn paged bits={bits} group={group}")
    pages = 80
    stride = 16 * pages
    ck, cv, ks, vs = make_cache(bits, group, stride, 0xD2 + bits + group)
    rng = np.random.default_rng(group + bits)
    perm = rng.permutation(pages).astype(np.int32)
    pt = ol.row_table(perm, stride)
    pos0 = 1000
    rows = 3
    q = ol.normal_bf16(0xD3, 0.0, 1.0, rows * HQ * D).reshape(rows, HQ * D)
    got = run_paged(q, ck, cv, ks, vs, bits, group, stride, d_pos=dev(np.array([pos0], np.int32)),
                    d_pt=dev(pt))
    want = ol.attn_split(q, ck, cv, ks, vs, bits, group, stride, [pos0, pos0 + 1, pos0 + 2],
                         pts=[pt] * rows, scale=1.0 / 16, Hk=HK)
    check(got, want, vmax(cv, vs, bits), f"paged bits {bits} group {group}")


def test_attn_long_context_multi_tile_splits():
    """20000 positions: 313 tiles, 2 tiles per split (157 splits)."""
    note("attn long context")
    bits, stride, pos0 = 8, 20480, 19999
    ck, cv, ks, vs = make_cache(bits, D, stride, 0xD4)
    q = ol.normal_bf16(0xD5, 0.0, 1.0, HQ * D).reshape(1, HQ * D)
    got = run_paged(q, ck, cv, ks, vs, bits, D, stride, d_pos=dev(np.array([pos0], np.int32)))
    want = ol.attn_split(q, ck, cv, ks, vs, bits, D, stride, [pos0], scale=1.0 / 16, Hk=HK)
    check(got, want, vmax(cv, vs, bits), "long context int8")
    # the Granite multiplier (1/128): flat softmax over 20000 keys
    got = run_paged(q, ck, cv, ks, vs, bits, D, stride, d_pos=dev(np.array([pos0], np.int32)),
                    scale=1.0 / 128)
    want = ol.attn_split(q, ck, cv, ks, vs, bits, D, stride, [pos0], scale=1.0 / 128, Hk=HK)
    check(got, want, vmax(cv, vs, bits), "long context int8, scale 1/128")


def test_attn_multi_sequence_rows():
    """Rows of different sessions: own positions and own page tables
    (row_pos / row_pt), as the multi-session decode step."""
    note("attn multi-sequence")
    bits, pages = 8, 64
    stride = 16 * pages
    ck, cv, ks, vs = make_cache(bits, D, stride, 0xD6)
    rng = np.random.default_rng(6)
    pos = [5, 700, 63, 64, 1000]
    pts = [ol.row_table(rng.permutation(pages).astype(np.int32), stride) for _ in pos]
    q = ol.normal_bf16(0xD7, 0.0, 1.0, len(pos) * HQ * D).reshape(len(pos), HQ * D)
    got = run_paged(q, ck, cv, ks, vs, bits, D, stride, row_pos=pos, row_pts=pts)
    want = ol.attn_split(q, ck, cv, ks, vs, bits, D, stride, pos, pts=pts, scale=1.0 / 16, Hk=HK)
    check(got, want, vmax(cv, vs, bits), "multi-sequence")


@pytest.mark.parametrize("bits,group", [(8, 128), (5, 32), (4, 64)])
def test_attn_multi_sequence_layout_from_max_len(bits, group):
    """The multi-session step's form over a pool longer than the sequences:
    stride 20480 (320 tiles: 2 tiles per split) with the layout taken from
    max_len 8192 (1 tile per split), 6 sessions with their own page tables at
    positions up to 8191 (a tile's first and last key, a split's last key).
    Against the oracle with the same layout, and each row bit for bit the
    single-sequence call (device position and page table) with the same
    max_len."""
    note(f"attn multi-sequence max_len bits={bits} group={group}")
    pages, max_len = 1280, 8192
    stride = 16 * pages
    ck, cv, ks, vs = make_cache(bits, group, stride, 0xDA + bits)
    rng = np.random.default_rng(0xDB)
    pos = [8191, 64, 4095, 127, 0, 6000]
    pts = [ol.row_table(rng.permutation(pages).astype(np.int32), stride) for _ in pos]
    q = ol.normal_bf16(0xDC, 0.0, 1.0, len(pos) * HQ * D).reshape(len(pos), HQ * D)
    got = run_paged(q, ck, cv, ks, vs, bits, group, stride, row_pos=pos, row_pts=pts,
                    max_len=max_len)
    want = ol.attn_split(q, ck, cv, ks, vs, bits, group, stride, pos, pts=pts, scale=1.0 / 16,
                         Hk=HK, max_len=max_len)
    check(got, want, vmax(cv, vs, bits), "multi-sequence, layout from max_len")
    for r, p in enumerate(pos):
        one = run_paged(q[r:r + 1], ck, cv, ks, vs, bits, group, stride,
                        d_pos=dev(np.array([p], np.int32)), d_pt=dev(pts[r]), max_len=max_len)
        np.testing.assert_array_equal(one[0], got[r], err_msg=f"row {r} at {p}")


@pytest.mark.parametrize("window", [1, 100, 5000])
def test_attn_window(window):
    note(f"attn window={window}")
    bits, stride = 16, 1200
    ck, cv, ks, vs = make_cache(bits, D, stride, 0xD8)
    q = ol.normal_bf16(0xD9, 0.0, 1.0, 2 * HQ * D).reshape(2, HQ * D)
    got = run_paged(q, ck, cv, ks, vs, bits, D, stride, kv_base=1000, window=window)
    want = ol.attn_split(q, ck, cv, ks, vs, bits, D, stride, [1000, 1001], window=window,
                         scale=1.0 / 16, Hk=HK)
    check(got, want, vmax(cv, vs, bits), f"window {window}")
    if window == 1:  # exact: each query head returns its KV head's value row
        vv = cv.view(np.uint16).reshape(HK, stride, D)
        for r, p in enumerate((1000, 1001)):
            for h in range(HQ):
                np.testing.assert_array_equal(got[r, h * D:(h + 1) * D], vv[h // 4, p])


def test_attn_reference_entry_point_int8_and_k5():
    """granite4_attn_split (the reference's signature) selects the same
    kernels as granite4_attn_paged."""
    note("attn_split reference entry point")
    stride, rows, kv_base = 256, 2, 200
    q = ol.normal_bf16(0xDA, 0.0, 1.0, rows * HQ * D).reshape(rows, HQ * D)
    for bits in (8, 5):
        ck, cv, ks, vs = make_cache(bits, D, stride, 0xDB + bits)
        want = run_paged(q, ck, cv, ks, vs, bits, D, stride, kv_base=kv_base)
        scratch = torch.empty(L.call_size("granite4_attn_split_scratch_bytes", HQ, rows, stride),
                              dtype=torch.uint8, device="cuda")
        out = torch.empty((rows, HQ * D), dtype=torch.int16, device="cuda")
        dk, dv, dks, dvs = dev(ck), dev(cv), dev(ks), dev(vs)
        int8 = bits == 8
        L.call("granite4_attn_split", dev(q), None, None, 1.0 / 16, HQ, HK, D, kv_base, None, rows,
               stride, scratch, out, dk if int8 else None, dv if int8 else None, dks, dvs,
               int(int8), None if int8 else dk, None if int8 else dv, int(not int8), None, 0,
               None, None, None, 0, None, None, 0, int(bits == 5), 0)
        np.testing.assert_array_equal(host(out).view(np.uint16), want)


# ----------------------------------------------------------------- causal prefill attention
def run_prefill(q, ck, cv, ks, vs, bits, group, stride, base, d_pt=None, window=0, scale=1.0 / 16):
    rows = q.shape[0]
    out = torch.empty((rows, HQ * D), dtype=torch.int16, device="cuda")
    dks = None if ks is None else dev(ks)
    dvs = None if vs is None else dev(vs)
    L.call("granite4_prefill_attn", dev(q), rows, HQ, HK, D, scale, dev(ck), dev(cv), dks, dvs, bits,
           group, stride, base, d_pt, window, out)
    return host(out).view(np.uint16)


@pytest.mark.parametrize("bits", [16, 8, 4, 5])
def test_prefill_attn_contiguous(bits):
    note(f"prefill attn bits={bits}")
    stride, base, rows = 256, 30, 50
    ck, cv, ks, vs = make_cache(bits, D, stride, 0xE0 + bits)
    q = ol.normal_bf16(0xE1 + bits, 0.0, 1.0, rows * HQ * D).reshape(rows, HQ * D)
    got = run_prefill(q, ck, cv, ks, vs, bits, D, stride, base)
    want = ol.prefill_attn(q, ck, cv, ks, vs, bits, D, stride, base, scale=1.0 / 16, Hk=HK)
    check(got, want, vmax(cv, vs, bits), f"prefill bits {bits}")


@pytest.mark.parametrize("bits,group,window", [(5, 32, 0), (8, 64, 0), (16, 128, 64), (4, 128, 100)])
def test_prefill_attn_paged(bits, group, window):
    note(f"prefill attn paged bits={bits} group={group} window={window}")
    pages = 24
    stride = 16 * pages
    base, rows = 200, 150
    ck, cv, ks, vs = make_cache(bits, group, stride, 0xE2 + bits + group)
    rng = np.random.default_rng(bits * 7 + group)
    pt = ol.row_table(rng.permutation(pages).astype(np.int32), stride)
    q = ol.normal_bf16(0xE3, 0.0, 1.0, rows * HQ * D).reshape(rows, HQ * D)
    got = run_prefill(q, ck, cv, ks, vs, bits, group, stride, base, d_pt=dev(pt), window=window)
    want = ol.prefill_attn(q, ck, cv, ks, vs, bits, group, stride, base, pt=pt, window=window,
                           scale=1.0 / 16, Hk=HK)
    check(got, want, vmax(cv, vs, bits), f"prefill paged bits {bits} group {group} w {window}")


@pytest.mark.parametrize("rows", [1100, 2100])
@pytest.mark.parametrize("bits,group,window", [(5, 32, 0), (8, 128, 300), (16, 128, 0)])
def test_prefill_attn_long_prompt_eight_wave_form(bits, group, window, rows):
    """1100 rows (8-wave workgroups of 32 positions, one column block per
    wave: enough of them for every CU, where shorter prompts take the
    key-split form) and 2100 rows (64 positions, two column blocks per wave,
    the last workgroup partly past the end), paged, at base 60. Three 32-row
    ranges checked against the oracle run on those rows alone (a row's output
    depends only on its position and the pool)."""
    note(f"prefill attn long prompt rows={rows} bits={bits} group={group} window={window}")
    base = 60
    pages = (base + rows + 15) // 16 + 4
    stride = 16 * pages
    ck, cv, ks, vs = make_cache(bits, group, stride, 0xF4 + bits)
    rng = np.random.default_rng(bits + 99)
    pt = ol.row_table(rng.permutation(pages).astype(np.int32), stride)
    q = ol.normal_bf16(0xF5, 0.0, 1.0, rows * HQ * D).reshape(rows, HQ * D)
    got = run_prefill(q, ck, cv, ks, vs, bits, group, stride, base, d_pt=dev(pt), window=window)
    for r0 in (0, 530, rows - 32):
        want = ol.prefill_attn(q[r0:r0 + 32], ck, cv, ks, vs, bits, group, stride, base + r0,
                               pt=pt, window=window, scale=1.0 / 16, Hk=HK)
        check(got[r0:r0 + 32], want, vmax(cv, vs, bits), f"prefill rows {r0}.. bits {bits}")


def test_prefill_attn_t512_from_zero_and_reference_entry_point():
    """T = 512 from position 0 (BASELINE config 3's prefill shape), int8, and
    the reference-named granite4_prefill_attention on the same inputs."""
    note("prefill attn T=512")
    stride, rows = 512, 512
    ck, cv, ks, vs = make_cache(8, D, stride, 0xE4)
    q = ol.normal_bf16(0xE5, 0.0, 1.0, rows * HQ * D).reshape(rows, HQ * D)
    got = run_prefill(q, ck, cv, ks, vs, 8, D, stride, 0, scale=1.0 / 128)
    want = ol.prefill_attn(q, ck, cv, ks, vs, 8, D, stride, 0, scale=1.0 / 128, Hk=HK)
    check(got, want, vmax(cv, vs, 8), "prefill T=512 int8")
    out = torch.empty((rows, HQ * D), dtype=torch.int16, device="cuda")
    dk, dv = dev(ck), dev(cv)
    L.call("granite4_prefill_attention", dev(q), None, None, 1.0 / 128, HQ, HK, D, 0, rows, stride,
           out, dk, dv, dev(ks), dev(vs), 1, None, None, 0, None, 0, 0)
    np.testing.assert_array_equal(host(out).view(np.uint16), got)


@pytest.mark.parametrize("pos_v,max_pos", [(1000, 4096), (0, 4096), (1023, 4096), (1279, 4096),
                                           (1000, 512)])
@pytest.mark.parametrize("bits,group", [(16, 128), (8, 128), (5, 32), (4, 64)])
def test_attn_decode_append_fused(bits, group, pos_v, max_pos):
    """RoPE + KV append folded into the attention launch: the output and the
    whole pool bit-identical to granite4_rope_append_at_pos followed by
    granite4_attn_paged at the same position and page table. Positions at the
    first / a middle / the last key of a tile and the arena's last row (the
    appended key is read from the wave's LDS copy), and one past the RoPE
    table (K not written, V read back from the pool)."""
    note(f"attn decode append bits={bits} group={group} pos={pos_v} max_pos={max_pos}")
    pages = 80
    stride = 16 * pages
    ck, cv, ks, vs = make_cache(bits, group, stride, 0xF1 + bits)
    rng = np.random.default_rng(bits + group)
    pt = dev(ol.row_table(rng.permutation(pages).astype(np.int32), stride))
    pos = dev(np.array([pos_v], np.int32))
    q = dev(ol.normal_bf16(0xF2, 0.0, 1.0, HQ * D))
    k = dev(ol.normal_bf16(0xF3, 0.0, 1.0, HK * D))
    v = dev(ol.normal_bf16(0xF4, 0.0, 1.0, HK * D))
    cos_t, sin_t = ol.rope_tables(1e7, D, max_pos)
    dcos, dsin = dev(cos_t), dev(sin_t)
    scratch = torch.empty(L.call_size("granite4_attn_split_scratch_bytes", HQ, 1, stride),
                          dtype=torch.uint8, device="cuda")
    res = []
    for fused in (False, True):
        pool = [dev(ck), dev(cv), None if ks is None else dev(ks), None if vs is None else dev(vs)]
        out = torch.empty(HQ * D, dtype=torch.int16, device="cuda")
        if fused:
            L.call("granite4_attn_decode_append", q, k, v, dcos, dsin, max_pos, pos, pt, HQ, HK,
                   1.0 / 16, *pool, bits, group, stride, scratch, out)
        else:
            # zeros: a position past the table leaves q_rot unwritten, and the
            # fused form then attends with a zero query
            q_rot = torch.zeros(HQ * D, dtype=torch.int16, device="cuda")
            L.call("granite4_rope_append_at_pos", q, k, v, dcos, dsin, max_pos, pos, pt, HQ, HK, D,
                   bits, group, q_rot, *pool, stride)
            L.call("granite4_attn_paged", q_rot, 1, HQ, HK, D, 1.0 / 16, *pool, bits, group, stride,
                   0, pos, pt, None, None, 0, 0, scratch, out)
        res.append([host(out)] + [host(t) for t in pool if t is not None])
    for a_, b_ in zip(*res):
        np.testing.assert_array_equal(a_, b_)



@pytest.mark.parametrize("bits,group", [(8, 128), (16, 128), (5, 32)])
def test_attn_decode_append_long_context_repeated(bits, group):
    """The fused decode attention over many split blocks: stride 16384 (256
    splits, 64 split blocks), positions whose combine covers 1, 17, 64 and 32
    blocks, called repeatedly on one scratch. Output and pool bit-identical
    to rope_append_at_pos + granite4_attn_paged every time."""
    pages = 1024
    stride = 16 * pages
    ck, cv, ks, vs = make_cache(bits, group, stride, 0xA1 + bits)
    rng = np.random.default_rng(bits)
    pt = dev(ol.row_table(rng.permutation(pages).astype(np.int32), stride))
    cos_t, sin_t = ol.rope_tables(1e7, D, stride)
    dcos, dsin = dev(cos_t), dev(sin_t)
    scratch = torch.empty(L.call_size("granite4_attn_split_scratch_bytes", HQ, 1, stride),
                          dtype=torch.uint8, device="cuda")
    for it, pos_v in enumerate((100, 4321, 16383, 255, 8191)):
        note(f"attn decode long context bits={bits} group={group} pos={pos_v} call={it}")
        pos = dev(np.array([pos_v], np.int32))
        q = dev(ol.normal_bf16(0xA2 + it, 0.0, 1.0, HQ * D))
        k = dev(ol.normal_bf16(0xA3 + it, 0.0, 1.0, HK * D))
        v = dev(ol.normal_bf16(0xA4 + it, 0.0, 1.0, HK * D))
        res = []
        for fused in (False, True):
            pool = [dev(ck), dev(cv), None if ks is None else dev(ks),
                    None if vs is None else dev(vs)]
            out = torch.empty(HQ * D, dtype=torch.int16, device="cuda")
            if fused:
                L.call("granite4_attn_decode_append", q, k, v, dcos, dsin, stride, pos, pt, HQ,
                       HK, 1.0 / 16, *pool, bits, group, stride, scratch, out)
            else:
                q_rot = torch.zeros(HQ * D, dtype=torch.int16, device="cuda")
                L.call("granite4_rope_append_at_pos", q, k, v, dcos, dsin, stride, pos, pt, HQ,
                       HK, D, bits, group, q_rot, *pool, stride)
                L.call("granite4_attn_paged", q_rot, 1, HQ, HK, D, 1.0 / 16, *pool, bits, group,
                       stride, 0, pos, pt, None, None, 0, 0, scratch, out)
            res.append([host(out)] + [host(t) for t in pool if t is not None])
        got = (res[1][0].view(np.uint16).astype(np.uint32) << 16).view(np.float32)
        assert np.isfinite(got).all()
        for a_, b_ in zip(*res):
            np.testing.assert_array_equal(a_, b_)


# ------------------------------------------------- combine inside the split launch
COMBINE_CASES = [
    dict(name="rows1_int8", bits=8, stride=2000, rows=1, kv_base=1999),
    dict(name="rows4_k5", bits=5, stride=2000, rows=4, kv_base=1300),
    dict(name="rows9_bf16", bits=16, stride=3000, rows=9, kv_base=2900),
    dict(name="window100", bits=16, stride=5000, rows=2, kv_base=4000, window=100),
    dict(name="window700_int4", bits=4, stride=5000, rows=3, kv_base=4000, window=700),
    dict(name="long64blocks", bits=8, stride=16384, rows=1, kv_base=16383),
    dict(name="multi_seq_with_empty", bits=8, stride=1024, rows=5, multi=[-1, 700, 63, 64, 1000]),
]


@pytest.mark.parametrize("case", COMBINE_CASES, ids=[c["name"] for c in COMBINE_CASES])
def test_attn_combine_in_split_launch_matches_second_launch(case):
    """The split blocks' partials combined by the last block of each (row
    group, KV head) inside the split launch (the default) give the same
    output bits as the combine's own launch (mode 1), including windows
    (blocks from the window's first), 64 split blocks (four 16-block chunks)
    and a multi-sequence row with no keys (position -1: its group has no
    block with work, and block 0 combines nothing in both forms). Each form
    runs twice on one scratch, the second call finding the first's tags and
    partials there."""
    note(f"attn combine forms {case['name']}")
    bits, stride, rows = case["bits"], case["stride"], case["rows"]
    ck, cv, ks, vs = make_cache(bits, D, stride, 0xC0 + bits)
    q = ol.normal_bf16(0xC1 + rows, 0.0, 1.0, rows * HQ * D).reshape(rows, HQ * D)
    kw = dict(window=case.get("window", 0))
    if "multi" in case:
        pages = stride // 16
        rng = np.random.default_rng(11)
        kw["row_pos"] = case["multi"]
        kw["row_pts"] = [ol.row_table(rng.permutation(pages).astype(np.int32), stride)
                         for _ in case["multi"]]
    else:
        kw["kv_base"] = case["kv_base"]
    outs = {}
    prev = L.set_attn_combine_mode(0)
    try:
        for mode in (1, 0, 1, 0):
            L.set_attn_combine_mode(mode)
            outs.setdefault(mode, []).append(run_paged(q, ck, cv, ks, vs, bits, D, stride, **kw))
    finally:
        L.set_attn_combine_mode(prev)
    for o in outs[1][1:] + outs[0]:
        np.testing.assert_array_equal(o, outs[1][0])
    if "multi" not in case:  # and both against the oracle
        pos = [case["kv_base"] + r for r in range(rows)]
        want = ol.attn_split(q, ck, cv, ks, vs, bits, D, stride, pos, window=kw["window"],
                             scale=1.0 / 16, Hk=HK)
        check(outs[0][0], want, vmax(cv, vs, bits), case["name"])


def test_attn_combine_in_split_launch_graph_replays():
    """A captured granite4_attn_paged (device position, paged, int8) replays
    with one tag baked in: every replay must find the tag slots re-zeroed by
    the previous call's combining block. Four replays at positions covering
    2, 20, 32 and 1 split blocks, each followed by an eager call on the same
    scratch (a fresh tag) and checked against the second-launch form."""
    note("attn combine graph replays")
    bits, pages = 8, 512
    stride = 16 * pages
    ck, cv, ks, vs = make_cache(bits, D, stride, 0xC7)
    rng = np.random.default_rng(12)
    pt = dev(ol.row_table(rng.permutation(pages).astype(np.int32), stride))
    dk, dv, dks, dvs = dev(ck), dev(cv), dev(ks), dev(vs)
    q = dev(ol.normal_bf16(0xC8, 0.0, 1.0, HQ * D))
    pos = torch.zeros(1, dtype=torch.int32, device="cuda")
    scratch = torch.empty(L.call_size("granite4_attn_split_scratch_bytes", HQ, 1, stride),
                          dtype=torch.uint8, device="cuda")
    out = torch.empty(HQ * D, dtype=torch.int16, device="cuda")
    out_e = torch.empty(HQ * D, dtype=torch.int16, device="cuda")

    def call(o):
        L.call("granite4_attn_paged", q, 1, HQ, HK, D, 1.0 / 16, dk, dv, dks, dvs, bits, D, stride,
               0, pos, pt, None, None, 0, 0, scratch, o)

    prev = L.set_attn_combine_mode(0)
    try:
        pos.fill_(300)
        call(out)  # warm-up outside the capture
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        L.use_stream(s)
        try:
            with torch.cuda.graph(g, stream=s):
                call(out)
        finally:
            L.use_stream()
        for p in (300, 5000, 8191, 63):
            pos.fill_(p)
            g.replay()
            torch.cuda.synchronize()
            got = host(out).copy()
            call(out_e)  # eager fused call in between (another tag)
            fused_eager = host(out_e).copy()
            L.set_attn_combine_mode(1)
            call(out_e)
            two = host(out_e).copy()
            L.set_attn_combine_mode(0)
            np.testing.assert_array_equal(got, two, err_msg=f"replay at {p}")
            np.testing.assert_array_equal(fused_eager, two, err_msg=f"eager at {p}")
    finally:
        L.set_attn_combine_mode(prev)
        L.use_stream()
