"""The host page-table controller driving the kernels: two sessions whose
prompts share a 32-token prefix take their row tables (d_pt) from one
KvPoolController. Session A appends its 48 positions; session B adopts A's
two cached pages and appends only its own 16-token tail. Each session's
rows, gathered through its table, must equal the oracle's contiguous append
of that session's whole sequence (codes and scales bit-exact), and decode
attention through each table must match the oracle attention over the
contiguous cache (the tolerance of tests/test_gpu_attn.py)."""
import numpy as np
import pytest
import torch

import oracle_lib as ol
from pkg import layerops

pytestmark = pytest.mark.gpu

HK, HQ, D, B = 8, 32, 128, 16
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


def gather(arr, table, per_row):
    """Arena [Hk][stride][per_row] -> contiguous [Hk][n][per_row] through table."""
    a = arr.reshape(HK, -1, per_row)
    return a[:, table, :]


@pytest.mark.parametrize("bits,group", [(8, 128), (5, 32)])
def test_controller_tables_drive_append_and_attention(bits, group):
    print(f"kv controller end to end bits={bits} group={group}", flush=True)
    pages = 12
    stride = pages * B
    layer_bytes = B * 2 * 1 * HK * D  # one layer's page at one byte per element
    c = L.KvPoolController(1, HK, D, B, pages * layer_bytes)
    assert c.pool_pages() == pages
    a_slot, b_slot = c.new_slot(), c.new_slot()
    prompt_a = list(range(1000, 1048))
    prompt_b = prompt_a[:32] + list(range(5000, 5016))
    ok, reused = c.prefill(a_slot, prompt_a)
    assert ok and reused == 0
    ok, reused = c.prefill(b_slot, prompt_b)
    assert ok and reused == 32
    pt_a, pt_b = c.row_table(a_slot, 48), c.row_table(b_slot, 48)
    assert list(pt_a[:32]) == list(pt_b[:32]) and not set(pt_a[32:]) & set(pt_b[32:])

    cos_t, sin_t = ol.rope_tables(1e7, D, 64)
    dcos, dsin = dev(cos_t), dev(sin_t)
    # K / V of each position: the shared prefix is identical for both sessions
    k_a = ol.normal_bf16(0xE1, 0.0, 1.0, 48 * HK * D).reshape(48, HK * D)
    v_a = ol.normal_bf16(0xE2, 0.0, 1.0, 48 * HK * D).reshape(48, HK * D)
    k_b, v_b = k_a.copy(), v_a.copy()
    k_b[32:] = ol.normal_bf16(0xE3, 0.0, 1.0, 16 * HK * D).reshape(16, HK * D)
    v_b[32:] = ol.normal_bf16(0xE4, 0.0, 1.0, 16 * HK * D).reshape(16, HK * D)

    arena = L.KvArena(bits, HK, stride, group=group)
    L.rope_append(arena, None, dev(k_a), dev(v_a), dcos, dsin, base_pos=0, d_pt=dev(pt_a))
    # B prefills only what the cache did not supply
    L.rope_append(arena, None, dev(k_b[32:]), dev(v_b[32:]), dcos, dsin, base_pos=32,
                  d_pt=dev(pt_b))
    kb, vb = ol.KV_ROW_BYTES[bits]
    ng = D // group
    ck, cv, ks, vs = host(arena.k), host(arena.v), host(arena.k_scale), host(arena.v_scale)
    conts = {}
    for name, kk, vv, pt in (("A", k_a, v_a, pt_a), ("B", k_b, v_b, pt_b)):
        _, wk, wv, wks, wvs = ol.rope_append(None, kk, vv, cos_t, sin_t, np.arange(48, dtype=np.int32),
                                             np.arange(48, dtype=np.int32), bits, group, 48, HK)
        conts[name] = (wk, wv, wks, wvs)
        np.testing.assert_array_equal(gather(ck, pt, kb), wk.reshape(HK, 48, kb))
        np.testing.assert_array_equal(gather(cv, pt, vb), wv.reshape(HK, 48, vb))
        np.testing.assert_array_equal(gather(ks, pt, ng), wks.reshape(HK, 48, ng))
        np.testing.assert_array_equal(gather(vs, pt, ng), wvs.reshape(HK, 48, ng))

    # decode attention of each session's position 47 through its own table
    for name, pt, seed in (("A", pt_a, 0xE5), ("B", pt_b, 0xE6)):
        q = ol.normal_bf16(seed, 0.0, 1.0, HQ * D).reshape(1, HQ * D)
        scratch = torch.empty(L.call_size("granite4_attn_split_scratch_bytes", HQ, 1, stride),
                              dtype=torch.uint8, device="cuda")
        out = torch.empty((1, HQ * D), dtype=torch.int16, device="cuda")
        L.call("granite4_attn_paged", dev(q), 1, HQ, HK, D, 1.0 / 16, arena.k, arena.v,
               arena.k_scale, arena.v_scale, bits, group, stride, 0,
               dev(np.array([47], np.int32)), dev(pt), None, None, 0, 0, scratch, out)
        got = host(out)
        wk, wv, wks, wvs = conts[name]
        want = ol.attn_split(q, wk, wv, wks, wvs, bits, group, 48, [47], scale=1.0 / 16, Hk=HK)
        fa, fb = ol.bf16_to_f32(got).astype(np.float64), ol.bf16_to_f32(want).astype(np.float64)
        mag = np.maximum(np.abs(fa), np.abs(fb))
        step = 2.0 ** (np.floor(np.log2(np.maximum(mag, 1e-30))) - 7)
        vm = float((127 if bits == 8 else 8) * wvs.max())
        ok = (np.abs(fa - fb) / step <= 2) | (np.abs(fa - fb) <= 2.0 ** -8 * vm)
        print(f"  session {name}: exact {np.mean(got == want):.4f}", flush=True)
        assert ok.all()
