"""CPU checks of the C ABI library: it loads, exports every symbol the header
declares, validates arguments without touching a GPU, and its host-compiled
copy of the kernels' scalar arithmetic (FP8 encode, KV codes) matches the
oracle on exhaustive sweeps."""
import ctypes
import os
import re

import numpy as np
import pytest

import oracle_lib as ol
from pkg import HEADER, layerops


def _have_gpu():
    import torch
    return torch.cuda.is_available()

L = layerops()


def declared_symbols():
    text = open(HEADER).read()
    text = text.split("#ifdef __cplusplus\n}")[0]  # C declarations only
    return sorted(set(re.findall(r"\b(granite4_\w+)\s*\(", text)))


def test_header_symbols_exported():
    syms = declared_symbols()
    assert len(syms) >= 35
    missing = [s for s in syms if not hasattr(L.lib, s)]
    assert not missing, missing
    # every declared symbol also has a ctypes signature in the host module
    assert not [s for s in syms if s not in L._SIG], [s for s in syms if s not in L._SIG]


def test_kv_pool_header_symbols_exported():
    """include/granite4_kv_pool.h: every C entry point is exported and bound."""
    text = open(os.path.join(os.path.dirname(HEADER), "granite4_kv_pool.h")).read()
    text = text.split('extern "C" {')[-1]
    syms = sorted(set(re.findall(r"\b(granite4_\w+)\s*\(", text)))
    assert len(syms) >= 30
    assert not [s for s in syms if not hasattr(L.lib, s)]
    assert not [s for s in syms if s not in L._SIG]


def test_argument_validation_returns_minus_one():
    lib = L.lib
    assert lib.granite4_kernel_rmsnorm(None, None, 1e-5, 1, 4096, None) == -1
    assert lib.granite4_kernel_rmsnorm(8, 8, 0.0, 1, 4096, 8) == -1      # eps must be > 0
    assert lib.granite4_kernel_rmsnorm_batched(8, 8, 1e-5, 17, 4096, 8) == -1  # rows > 16
    assert lib.granite4_add_rmsnorm_fp8(8, 8, 1.0, 8, 1e-5, 4, 4096, 8, 8, 8, None) == -1
    assert lib.granite4_swiglu_fp8(8, 4, 12801, 8, 8, 8, None) == -1
    assert lib.granite4_kernel_kv_append_int8_batched(8, 8, 8, 8, 8, 8, 10, 4, 12, 8, 128,
                                                      None) == -1  # stride < base + rows
    assert lib.granite4_kernel_kv_append_k5v4_batched(8, 8, 8, 8, 8, 8, 0, 4, 12, 8, 64,
                                                      None) == -1  # d != 128
    assert lib.granite4_prefill_rope_split_append_int8(8, 8, 8, 0, 4, 32, 8, 64, 16, 8, 8, 8, 8,
                                                       8, None) == -1  # d != 128
    assert lib.granite4_rope_append(8, 4096, 8, 1024, 8, 1024, 8, 8, 100, 4, 32, 8, 128, 0, None,
                                    None, None, 8, 48, 0, 1, 8, 4096, 8, 8, 8, 8, 16) == -1  # group
    assert lib.granite4_embed_rows(8, 0, 8, 100, 4096, 1.0, 8) == -1
    assert lib.granite4_rope_tables_build(1e7, 127, 16, None, None) == -1
    # a negative segment is rejected even when the total is positive
    assert lib.granite4_gemv_qkv(256, 256, 256, 256, 1.0, 1.0, 1.0, -8, 16, 0, 4096, 256, 256,
                                 256) == -1
    if os.environ.get("HIP_VISIBLE_DEVICES") == "" or not _have_gpu():
        # NULL selects the library's static scratch, which needs a device
        assert lib.granite4_fp8_sync_status(None, 0) == -1
    assert lib.granite4_debug_set_sync_spin_limit(-1) == -1


def test_mode_switches_return_previous_and_reject_others():
    """The process-wide launch switches (FP8 single launch, attention combine
    in the split launch) return the previous mode and reject other values;
    host-only, no device call."""
    for setter, top in ((L.lib.granite4_set_fp8_launch_mode, 2),
                        (L.lib.granite4_set_attn_combine_mode, 1)):
        prev = setter(1)
        assert prev in range(top + 1)
        assert setter(top + 1) == -1 and setter(-1) == -1
        assert setter(top) == 1
        assert setter(0) == top
        assert setter(prev) == 0


def test_attn_scratch_covers_every_layout_up_to_the_arena():
    """granite4_attn_split_scratch_bytes(Hq, rows, stride) holds the partials
    of any split layout a call over that arena may take (max_len <= stride):
    the split count is not monotone (256 tiles give 256 splits of one tile,
    257 tiles 129 splits of two), so a 257-tile arena sized by its own layout
    would be too small for a call laid out by max_len = 256 tiles."""
    f = L.lib.granite4_attn_split_scratch_bytes
    f.restype = ctypes.c_size_t
    per_slot = 8 + 128 * 4 + 4  # (m, l), the partial output, the arrival tag
    for stride, splits in ((64, 1), (16384, 256), (16448, 256), (20480, 256), (524288, 256),
                           (1000, 16)):
        nblk = (splits + 3) // 4
        assert f(32, 8, stride) == 256 + 8 * 32 * nblk * per_slot, stride
    for stride in range(64, 40000, 640):
        assert f(32, 1, stride) >= f(32, 1, min(stride, 16384))


def test_row_table_host_matches_oracle_and_golden():
    G = np.load(ol.os.path.join(ol.ROOT, "tests", "golden", "golden.npz"))
    for s in range(G["pt_blocks"].shape[0]):
        bt = np.ascontiguousarray(G["pt_blocks"][s], np.int32)
        n = G["pt_rows"].shape[1]
        out = np.empty(n, np.int32)
        assert L.lib.granite4_row_table(bt.ctypes.data, n, 16, out.ctypes.data) == 0
        np.testing.assert_array_equal(out, G["pt_rows"][s])


def _host_fp8(y, scale):
    y = np.ascontiguousarray(y, np.float32)
    out = np.empty(y.size, np.uint8)
    assert L.lib.granite4_host_fp8_encode(y.ctypes.data, y.size, scale, out.ctypes.data) == 0
    return out


ALL_BF16 = np.arange(65536, dtype=np.uint16)


@pytest.mark.parametrize("amax", [1.0, 448.0, 3.7, 0.015625, 7.2e-3, 1234.5, 2.5e-29, 6.0e37,
                                  1e-40, 0.0])
def test_fp8_fast_encoder_exhaustive_bf16(amax):
    """Every bf16 value through the kernels' encoder (host build) vs the oracle."""
    scale = ol.lib.g4o_fp8_scale_for(amax)
    got = _host_fp8(ol.bf16_to_f32(ALL_BF16), scale)
    if scale > 0:
        want = ol.fp8_encode_scaled(ALL_BF16, scale)
    else:
        want = np.zeros(65536, np.uint8)
    np.testing.assert_array_equal(got, want)


def test_fp8_fast_encoder_near_midpoints():
    """Values straddling every e4m3 midpoint for awkward scales (the fma decision)."""
    grid = np.array([ol.lib.g4o_fp8_decode(c) for c in range(0x7F)])
    mids = (grid[:-1] + grid[1:]) / 2
    rs = np.random.default_rng(5)
    for scale in [np.float32(1.0), np.float32(3.0 / 448), np.float32(0.1), np.float32(rs.uniform()),
                  np.float32(1e-20), np.float32(7.77e5)]:
        t = np.concatenate([mids, grid])
        y = (t * np.float64(scale)).astype(np.float32)
        ys = np.concatenate([y, np.nextafter(y, np.float32(np.inf)),
                             np.nextafter(y, np.float32(-np.inf))])
        ys = np.concatenate([ys, -ys])
        got = _host_fp8(ys, float(scale))
        want = np.array([ol.lib.g4o_fp8_encode(float(v) / float(scale)) for v in ys], np.uint8)
        np.testing.assert_array_equal(got, want)


def test_kv_codes_host_match_oracle():
    x = ol.bf16_to_f32(ALL_BF16[np.isfinite(ol.bf16_to_f32(ALL_BF16))])
    for qmax in (127, 7, 15):
        for s in (np.float32(0.03), np.float32(1.0) / np.float32(qmax), np.float32(0.0),
                  np.float32(2.5)):
            out = np.empty(x.size, np.int32)
            assert L.lib.granite4_host_kv_codes(x.ctypes.data, x.size, float(s), qmax,
                                                out.ctypes.data) == 0
            want = np.array([ol.lib.g4o_kv_code(float(v), float(s), qmax) for v in x], np.int32)
            np.testing.assert_array_equal(out, want)


def test_kv_codes_host_half_integer_neighbours():
    """Operands within 4 ulps of every (k + 1/2) * s boundary, over scales of
    the form amax / qmax: the reciprocal-and-residual quotient the append
    kernels use must round exactly as the IEEE division (numpy's f32 divide
    is that division; a sample is also checked against the oracle)."""
    rng = np.random.default_rng(11)
    for qmax in (127, 15, 7):
        amax = rng.uniform(-30, 30, 64).astype(np.float32)
        scales = (np.exp2(amax) * rng.uniform(1, 2, 64)).astype(np.float32) / np.float32(qmax)
        for s in scales:
            k = np.arange(-qmax - 1, qmax + 1, dtype=np.float32)
            mid = ((k + np.float32(0.5)) * s).astype(np.float32)
            bits = mid.view(np.int32)[:, None] + np.arange(-4, 5, dtype=np.int32)[None, :]
            x = bits.reshape(-1).view(np.float32)
            out = np.empty(x.size, np.int32)
            assert L.lib.granite4_host_kv_codes(x.ctypes.data, x.size, float(s), qmax,
                                                out.ctypes.data) == 0
            q = x / s
            t = np.trunc(q)  # half away from zero, with the exact fraction q - t
            want = np.clip(t + np.sign(q) * (np.abs(q - t) >= 0.5), -qmax, qmax)
            np.testing.assert_array_equal(out, want.astype(np.int32))
        for i in range(0, x.size, 37):
            assert ol.lib.g4o_kv_code(float(x[i]), float(s), qmax) == out[i]
