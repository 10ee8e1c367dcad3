"""granite4_add_rmsnorm_fp8_noalloc (the entry point that allocates nothing:
its FP8 workspace is a static device array in the library) against
granite4_add_rmsnorm_fp8 with a caller workspace, through the C ABI: two calls
in a row, the second with a smaller input, in the single-launch and the
two-launch forms. Residual, codes and scale must be bit-identical."""
import sys

import numpy as np
import pytest
import torch

import oracle_lib as ol
from pkg import layerops

pytestmark = pytest.mark.gpu

L = None
COLS = 4096


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
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda()


def host(t):
    a = t.detach().cpu().numpy()
    return a.view(np.uint16) if a.dtype == np.int16 else a


def _inputs(rows, seed):
    res = ol.normal_bf16(seed, 0.0, 1.0, rows * COLS).reshape(rows, COLS)
    br = ol.normal_bf16(seed + 1, 0.0, 1.0, rows * COLS).reshape(rows, COLS)
    return dev(res), dev(br)


def _run(name, rows, res, br, w, mult, work=None):
    ro = torch.empty((rows, COLS), dtype=torch.int16, device="cuda")
    codes = torch.empty((rows, COLS), dtype=torch.uint8, device="cuda")
    scale = torch.empty(1, dtype=torch.float32, device="cuda")
    args = [res, br, mult, w, 1e-5, rows, COLS, ro, codes, scale]
    if work is not None:
        args.append(work)
    L.call(name, *args)
    return host(ro), host(codes), host(scale)[0]


@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("sizes", [(512, 200), (8192, 4097), (40, 1)])
def test_noalloc_matches_workspace_entry(mode, sizes):
    note(f"noalloc mode={mode} sizes={sizes}")
    w = dev(ol.normal_bf16(0x9A, 1.0, 0.1, COLS))
    work = L.fp8_workspace()
    prev = L.set_fp8_launch_mode(mode)
    try:
        for i, rows in enumerate(sizes):
            res, br = _inputs(rows, 0x9B + 7 * i + rows)
            mult = 0.5 if i else 1.0
            want = _run("granite4_add_rmsnorm_fp8", rows, res, br, w, mult, work)
            got = _run("granite4_add_rmsnorm_fp8_noalloc", rows, res, br, w, mult)
            np.testing.assert_array_equal(got[0], want[0])
            np.testing.assert_array_equal(got[1], want[1])
            assert got[2] == want[2]
    finally:
        L.set_fp8_launch_mode(prev)
    assert L.fp8_sync_status(None) == 0


def test_noalloc_rejects_rows_beyond_its_scratch():
    note("noalloc max rows")
    w = dev(ol.normal_bf16(0x9C, 1.0, 0.1, COLS))
    t = torch.empty(8, dtype=torch.int16, device="cuda")
    rc = L.lib.granite4_add_rmsnorm_fp8_noalloc(t.data_ptr(), None, 1.0, w.data_ptr(), 1e-5,
                                                65537, COLS, None, t.data_ptr(), t.data_ptr())
    assert rc == -1
