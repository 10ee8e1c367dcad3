"""Pins the oracle's split-KV attention (g4o_attn_split) before it checks the GPU.

- Against the reference's own host attention (kernel_math.h:312-331, built into
  oracle/_ref from the reference sources) on contiguous bf16 caches. The two
  round differently (the reference normalises p before its bf16 rounding, the
  split kernels round the unnormalised p and keep l in f32), so the bar is a
  tolerance, stated below.
- Exact properties: one key returns its value row; a window of one returns the
  last key's row; a paged pool equals the contiguous cache it permutes;
  quantised caches with power-of-two scales equal the bf16 path on the
  dequantised values bit for bit (this pins the int8 / int4 / K5 code layouts
  and offsets); a window covering everything changes nothing.
- Closeness to an f64 softmax attention without roundings.
"""
import numpy as np
import pytest

import oracle_lib as ol

D = 128


def _rand_q(seed, rows, Hq, std=1.0):
    return ol.normal_bf16(seed, 0.0, std, rows * Hq * D).reshape(rows, Hq * D)


def _bf16_cache(seed, Hk, stride, std=1.0):
    k = ol.normal_bf16(seed, 0.0, std, Hk * stride * D)
    v = ol.normal_bf16(seed + 1, 0.0, 1.0, Hk * stride * D)
    return k.view(np.uint8), v.view(np.uint8)


def _f32(b):
    return ol.bf16_to_f32(b)


def _ulps(a, b):
    """Distance in bf16 steps of the larger magnitude."""
    fa, fb = _f32(a).astype(np.float64), _f32(b).astype(np.float64)
    step = np.maximum(np.abs(fa), np.abs(fb))
    step = np.where(step > 0, 2.0 ** (np.floor(np.log2(np.maximum(step, 1e-30))) - 7), 1e-30)
    return np.abs(fa - fb) / step


def _exact_attention(q, k, v, Hk, kv_len, scale):
    """f64 softmax attention, no roundings; q [Hq*D], k/v [Hk][kv_len][D] f64."""
    Hq = q.size // D
    out = np.empty((Hq, D))
    for h in range(Hq):
        hk = h // (Hq // Hk)
        lg = scale * (k[hk, :kv_len] @ q[h * D:(h + 1) * D])
        p = np.exp(lg - lg.max())
        out[h] = (p @ v[hk, :kv_len]) / p.sum()
    return out


@pytest.mark.parametrize("kv_len", [1, 37, 64, 65, 300, 1000])
def test_attn_vs_reference_host_attention(kv_len):
    r = ol.ref_lib()
    if r is None:
        pytest.skip("oracle/_ref not built (no /root/reference)")
    Hq, Hk = 8, 2
    q = _rand_q(0xA1 + kv_len, 1, Hq)
    k, v = _bf16_cache(0xA2 + kv_len, Hk, kv_len, std=0.5)
    want = np.empty(Hq * D, np.uint16)
    r.ref_gqa_attention_bf16(q.ctypes.data_as(ol.u16p), k.view(np.uint16).ctypes.data_as(ol.u16p),
                             v.view(np.uint16).ctypes.data_as(ol.u16p), 1.0 / 16, Hq, Hk, D,
                             kv_len, want.ctypes.data_as(ol.u16p))
    got = ol.attn_split(q, k, v, None, None, 16, D, kv_len, [kv_len - 1], scale=1.0 / 16, Hk=Hk)
    # Tolerance: p is rounded to bf16 at a different scale in the two forms
    # (2^-9 relative per probability); outputs agree within 2 bf16 steps of
    # the larger magnitude, or 2^-9 of max |v| where they nearly cancel.
    u = _ulps(got[0], want)
    absd = np.abs(_f32(got[0]) - _f32(want))
    assert np.all((u <= 2) | (absd <= 2.0 ** -9 * np.abs(_f32(v.view(np.uint16))).max())), u.max()


def test_attn_single_key_and_window_one_are_exact():
    Hq, Hk, stride = 8, 2, 200
    q = _rand_q(0xA3, 3, Hq)
    k, v = _bf16_cache(0xA4, Hk, stride)
    vv = v.view(np.uint16).reshape(Hk, stride, D)
    # one key: out = v[0]
    out = ol.attn_split(q[:1], k, v, None, None, 16, D, stride, [0], Hk=Hk)
    for h in range(Hq):
        np.testing.assert_array_equal(out[0, h * D:(h + 1) * D], vv[h // 4, 0])
    # window 1: out = v[pos]
    pos = [5, 63, 150]
    out = ol.attn_split(q, k, v, None, None, 16, D, stride, pos, window=1, Hk=Hk)
    for r, p in enumerate(pos):
        for h in range(Hq):
            np.testing.assert_array_equal(out[r, h * D:(h + 1) * D], vv[h // 4, p])
    # a window wider than the sequence changes nothing
    a = ol.attn_split(q, k, v, None, None, 16, D, stride, pos, window=1000, Hk=Hk)
    b = ol.attn_split(q, k, v, None, None, 16, D, stride, pos, Hk=Hk)
    np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("bits", [16, 8, 4, 5])
def test_attn_paged_equals_contiguous(bits):
    """A page table that permutes 16-row pages reads the same keys."""
    Hq, Hk, n = 8, 2, 200
    stride = 16 * 20
    rng = np.random.default_rng(bits)
    kb, vb = ol.KV_ROW_BYTES[bits]
    ck = rng.integers(0, 256, Hk * stride * kb, dtype=np.uint8)
    cv = rng.integers(0, 256, Hk * stride * vb, dtype=np.uint8)
    if bits == 16:  # keep the bf16 values finite and moderate
        ck = ol.normal_bf16(0xA5, 0.0, 0.5, Hk * stride * D).view(np.uint8)
        cv = ol.normal_bf16(0xA6, 0.0, 1.0, Hk * stride * D).view(np.uint8)
    ks = (rng.random(Hk * stride, dtype=np.float32) * 0.1 + 0.01).astype(np.float32)
    vs = (rng.random(Hk * stride, dtype=np.float32) * 0.1 + 0.01).astype(np.float32)
    pages = rng.permutation(stride // 16).astype(np.int32)
    pt = ol.row_table(pages, n)
    # the contiguous cache that the paged one permutes
    def gather(c, rb):
        c2 = c.reshape(Hk, stride, rb)
        out = np.zeros_like(c2)
        out[:, :n] = c2[:, pt]
        return out.reshape(-1)
    gs = lambda s: gather(s.view(np.uint8), 4).view(np.float32)
    q = _rand_q(0xA7 + bits, 2, Hq, std=0.3)
    pos = [n - 1, 77]
    a = ol.attn_split(q, ck, cv, ks, vs, bits, D, stride, pos, pts=[pt, pt], Hk=Hk)
    b = ol.attn_split(q, gather(ck, kb), gather(cv, vb), gs(ks), gs(vs), bits, D, stride, pos,
                      Hk=Hk)
    np.testing.assert_array_equal(a, b)


def _dequant_rows(c, bits, is_k, n):
    """Per-row code values (stored value minus offset) of n rows, f32 [n][D]."""
    kb = ol.KV_ROW_BYTES[bits][0 if is_k else 1]
    rows = c.reshape(-1, kb)[:n]
    if bits == 8:
        return rows.view(np.int8).astype(np.float32)
    lo = (rows & 0xF).astype(np.int32)
    hi = (rows >> 4).astype(np.int32)
    nib = np.empty((n, D), np.int32)
    nib[:, 0::2] = lo[:, :D // 2]
    nib[:, 1::2] = hi[:, :D // 2]
    if bits == 5 and is_k:
        plane = rows[:, D // 2:D // 2 + D // 8]
        bit = (plane[:, :, None] >> np.arange(8)) & 1
        return (nib | (bit.reshape(n, D).astype(np.int32) << 4)).astype(np.float32) - 16
    return nib.astype(np.float32) - 8


@pytest.mark.parametrize("bits", [8, 4, 5])
def test_attn_quantised_pow2_scales_equal_bf16_on_dequantised(bits):
    """With power-of-two scales, code * scale is exact in bf16 and both the
    K scale (applied to q . codes) and the V scale (applied to p before its
    bf16 rounding) commute with every rounding: the quantised path must equal
    the bf16 path on the dequantised cache bit for bit."""
    Hq, Hk, n = 8, 2, 150
    stride = n
    rng = np.random.default_rng(10 + bits)
    kb, vb = ol.KV_ROW_BYTES[bits]
    ck = rng.integers(0, 256, Hk * stride * kb, dtype=np.uint8)
    cv = rng.integers(0, 256, Hk * stride * vb, dtype=np.uint8)
    ks = (2.0 ** rng.integers(-8, -3, Hk * stride)).astype(np.float32)
    vs = (2.0 ** rng.integers(-6, -1, Hk * stride)).astype(np.float32)
    kf = _dequant_rows(ck, bits, True, Hk * n) * ks[:, None]
    vf = _dequant_rows(cv, bits, False, Hk * n) * vs[:, None]
    kbf = ol.f32_to_bf16(kf).reshape(-1)
    vbf = ol.f32_to_bf16(vf).reshape(-1)
    assert np.array_equal(ol.bf16_to_f32(kbf).reshape(kf.shape), kf)  # exact in bf16
    q = _rand_q(0xA8 + bits, 3, Hq)
    pos = [n - 1, 64, 3]
    a = ol.attn_split(q, ck, cv, ks, vs, bits, D, stride, pos, Hk=Hk)
    b = ol.attn_split(q, kbf.view(np.uint8), vbf.view(np.uint8), None, None, 16, D, stride, pos,
                      Hk=Hk)
    np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("bits,grp", [(5, 32), (4, 32), (8, 64), (4, 64)])
def test_attn_group_scales_are_the_bf16_path_on_dequantised_values(bits, grp):
    """Scale groups of 32 or 64 (this build's extension; the reference has one
    scale per row): the attention reads each element as bf16(code * scale_g)
    and then runs the bf16 path, so for any scales (not only powers of two)
    it equals the bf16 attention over that dequantised cache bit for bit, in
    the split and in the prefill form."""
    Hq, Hk, n = 8, 2, 130
    ng = D // grp
    rng = np.random.default_rng(77 + bits + grp)
    kb, vb = ol.KV_ROW_BYTES[bits]
    ck = rng.integers(0, 256, Hk * n * kb, dtype=np.uint8)
    cv = rng.integers(0, 256, Hk * n * vb, dtype=np.uint8)
    ks = (rng.random(Hk * n * ng, dtype=np.float32) * 0.05 + 0.001).astype(np.float32)
    vs = (rng.random(Hk * n * ng, dtype=np.float32) * 0.2 + 0.01).astype(np.float32)
    if bits == 8:
        ks *= np.float32(0.1)
    kf = _dequant_rows(ck, bits, True, Hk * n) * np.repeat(ks.reshape(-1, ng), grp, axis=1)
    vf = _dequant_rows(cv, bits, False, Hk * n) * np.repeat(vs.reshape(-1, ng), grp, axis=1)
    kbf, vbf = ol.f32_to_bf16(kf).view(np.uint8), ol.f32_to_bf16(vf).view(np.uint8)
    assert not np.array_equal(ol.bf16_to_f32(ol.f32_to_bf16(kf)), kf)  # the rounding matters
    q = _rand_q(0xA9 + bits, 3, Hq)
    pos = [n - 1, 40, 64]
    a = ol.attn_split(q, ck, cv, ks, vs, bits, grp, n, pos, Hk=Hk)
    b = ol.attn_split(q, kbf, vbf, None, None, 16, D, n, pos, Hk=Hk)
    np.testing.assert_array_equal(a, b)
    qp = _rand_q(0xAA + bits, 20, Hq)
    a = ol.prefill_attn(qp, ck, cv, ks, vs, bits, grp, n, 100, Hk=Hk)
    b = ol.prefill_attn(qp, kbf, vbf, None, None, 16, D, n, 100, Hk=Hk)
    np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("kv_len,tps", [(500, 1), (500, 3), (2000, 1), (2000, 8)])
def test_attn_close_to_f64_softmax(kv_len, tps):
    """Any split layout stays within the bf16 roundings of an exact f64
    softmax attention: |out - exact| <= 2^-6 max |v| (the bf16 logits alone
    move each probability by up to 2^-9 of the logit range)."""
    Hq, Hk = 8, 2
    q = _rand_q(0xAA + kv_len, 1, Hq, std=0.5)
    k, v = _bf16_cache(0xAB + kv_len, Hk, kv_len, std=0.5)
    got = ol.attn_split(q, k, v, None, None, 16, D, kv_len, [kv_len - 1], scale=1.0 / 8, Hk=Hk,
                        tps=tps)
    kf = _f32(k.view(np.uint16)).reshape(Hk, kv_len, D).astype(np.float64)
    vf = _f32(v.view(np.uint16)).reshape(Hk, kv_len, D).astype(np.float64)
    ex = _exact_attention(_f32(q[0]).astype(np.float64), kf, vf, Hk, kv_len, 1.0 / 8)
    err = np.abs(_f32(got[0]).reshape(Hq, D) - ex)
    assert err.max() <= 2.0 ** -6 * np.abs(vf).max(), err.max()


# ----------------------------------------------------------------- prefill (causal) attention
def test_prefill_attn_vs_reference_host_attention_per_row():
    """Row r of the causal prefill attention is the reference's decode
    attention over the first base + r + 1 positions (same tolerance as above)."""
    r = ol.ref_lib()
    if r is None:
        pytest.skip("oracle/_ref not built (no /root/reference)")
    Hq, Hk, base, rows = 8, 2, 90, 40
    n = base + rows
    q = _rand_q(0xB1, rows, Hq)
    k, v = _bf16_cache(0xB2, Hk, n, std=0.5)
    got = ol.prefill_attn(q, k, v, None, None, 16, D, n, base, scale=1.0 / 16, Hk=Hk)
    kk = k.view(np.uint16).reshape(Hk, n, D)
    vv = v.view(np.uint16).reshape(Hk, n, D)
    vmax = np.abs(_f32(v.view(np.uint16))).max()
    for row in range(rows):
        L = base + row + 1
        kc = np.ascontiguousarray(kk[:, :L]).reshape(-1)
        vc = np.ascontiguousarray(vv[:, :L]).reshape(-1)
        want = np.empty(Hq * D, np.uint16)
        r.ref_gqa_attention_bf16(q[row].ctypes.data_as(ol.u16p), kc.ctypes.data_as(ol.u16p),
                                 vc.ctypes.data_as(ol.u16p), 1.0 / 16, Hq, Hk, D, L,
                                 want.ctypes.data_as(ol.u16p))
        u = _ulps(got[row], want)
        absd = np.abs(_f32(got[row]) - _f32(want))
        assert np.all((u <= 2) | (absd <= 2.0 ** -9 * vmax)), (row, u.max())


@pytest.mark.parametrize("bits", [16, 8, 5])
def test_prefill_attn_is_the_single_split_attention(bits):
    """One pass over every tile is the split attention with one split; the
    only difference is the final o / l (split combine) against o * (1 / l)
    (prefill): at most one bf16 step."""
    Hq, Hk, base, rows = 8, 2, 150, 20
    n = base + rows
    rng = np.random.default_rng(bits)
    kb, vb = ol.KV_ROW_BYTES[bits]
    if bits == 16:
        ck, cv = _bf16_cache(0xB3, Hk, n, std=0.5)
        ks = vs = None
    else:
        ck = rng.integers(0, 256, Hk * n * kb, dtype=np.uint8)
        cv = rng.integers(0, 256, Hk * n * vb, dtype=np.uint8)
        ks = (rng.random(Hk * n, dtype=np.float32) * 0.01).astype(np.float32)
        vs = (rng.random(Hk * n, dtype=np.float32) * 0.1).astype(np.float32)
    q = _rand_q(0xB4, rows, Hq)
    a = ol.prefill_attn(q, ck, cv, ks, vs, bits, D, n, base, scale=1.0 / 16, Hk=Hk)
    b = ol.attn_split(q, ck, cv, ks, vs, bits, D, n, [base + r for r in range(rows)],
                      scale=1.0 / 16, Hk=Hk, tps=1000)
    assert _ulps(a, b).max() <= 1
    assert np.mean(a == b) > 0.9


def test_prefill_attn_exact_properties():
    Hq, Hk, n = 8, 2, 130
    q = _rand_q(0xB5, n, Hq)
    k, v = _bf16_cache(0xB6, Hk, n)
    vv = v.view(np.uint16).reshape(Hk, n, D)
    out = ol.prefill_attn(q, k, v, None, None, 16, D, n, 0, Hk=Hk)
    for h in range(Hq):  # position 0 sees one key
        np.testing.assert_array_equal(out[0, h * D:(h + 1) * D], vv[h // 4, 0])
    out = ol.prefill_attn(q, k, v, None, None, 16, D, n, 0, window=1, Hk=Hk)
    for r in (0, 63, 64, 129):  # window 1: each row sees its own key
        for h in range(Hq):
            np.testing.assert_array_equal(out[r, h * D:(h + 1) * D], vv[h // 4, r])
    # paged == contiguous
    stride = 16 * 12
    rng = np.random.default_rng(3)
    pt = ol.row_table(rng.permutation(stride // 16).astype(np.int32), n)
    kp = np.zeros((Hk, stride, D), np.uint16)
    vp = np.zeros((Hk, stride, D), np.uint16)
    kp[:, pt] = k.view(np.uint16).reshape(Hk, n, D)
    vp[:, pt] = vv
    a = ol.prefill_attn(q, kp.view(np.uint8).reshape(-1), vp.view(np.uint8).reshape(-1), None, None,
                        16, D, stride, 0, pt=pt, Hk=Hk)
    b = ol.prefill_attn(q, k, v, None, None, 16, D, n, 0, Hk=Hk)
    np.testing.assert_array_equal(a, b)
