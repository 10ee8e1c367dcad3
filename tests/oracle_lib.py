"""ctypes bindings of the CPU oracle (oracle/libg4oracle.so) for the tests.

Test infrastructure: the oracle is the checker, never the thing under test.
Arrays are numpy; bf16 values travel as uint16 bit patterns.
"""
import ctypes
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
ORACLE_SO = os.path.join(ORACLE_DIR, "libg4oracle.so")
REF_SO = os.path.join(ORACLE_DIR, "_ref", "libg4ref.so")

_c = ctypes
u8p, u16p, i32p, u32p = (_c.POINTER(_c.c_uint8), _c.POINTER(_c.c_uint16),
                         _c.POINTER(_c.c_int32), _c.POINTER(_c.c_uint32))
f32p = _c.POINTER(_c.c_float)
vp = _c.c_void_p


def _p(a, t):
    return None if a is None else a.ctypes.data_as(t)


def _load():
    if not os.path.exists(ORACLE_SO):
        subprocess.check_call(["make", "-s", "-C", ORACLE_DIR, "all"])
    lib = _c.CDLL(ORACLE_SO)
    sig = {
        "g4o_bf16_to_f32": (_c.c_float, [_c.c_uint16]),
        "g4o_f32_to_bf16": (_c.c_uint16, [_c.c_float]),
        "g4o_fill_uniform_bf16": (None, [_c.c_uint64, _c.c_double, _c.c_size_t, u16p]),
        "g4o_fill_uniform_f32": (None, [_c.c_uint64, _c.c_double, _c.c_size_t, f32p]),
        "g4o_fill_normal_bf16": (None, [_c.c_uint64, _c.c_double, _c.c_double, _c.c_size_t,
                                        u16p]),
        "g4o_fill_u32": (None, [_c.c_uint64, _c.c_size_t, u32p]),
        "g4o_fp8_encode": (_c.c_uint8, [_c.c_double]),
        "g4o_fp8_decode": (_c.c_double, [_c.c_uint8]),
        "g4o_fp8_scale_for": (_c.c_float, [_c.c_double]),
        "g4o_fp8_encode_scaled_bf16": (None, [u16p, _c.c_size_t, _c.c_float, u8p]),
        "g4o_fp8_quantize_bf16": (_c.c_float, [u16p, _c.c_size_t, u8p]),
        "g4o_embed_rows": (None, [i32p, _c.c_int, u16p, _c.c_int, _c.c_float, u16p]),
        "g4o_rmsnorm": (None, [u16p, u16p, _c.c_float, _c.c_int, _c.c_int, u16p]),
        "g4o_add_rmsnorm": (None, [u16p, u16p, _c.c_float, u16p, _c.c_float, _c.c_int,
                                   _c.c_int, u16p, u16p]),
        "g4o_swiglu_bf16": (None, [u16p, _c.c_int, _c.c_int, u16p]),
        "g4o_silu_mul_f32": (None, [f32p, _c.c_int, _c.c_int, u16p]),
        "g4o_gemm_fp8": (None, [u8p, _c.c_int, _c.c_float, u8p, _c.c_int, _c.c_int, _c.c_int,
                                _c.c_float, _c.c_float, _c.c_float, _c.c_int, _c.c_int, f32p]),
        "g4o_gemv_fp8w": (None, [u16p, u8p, _c.c_int, _c.c_int, _c.c_float, f32p]),
        "g4o_gemm_bf16w": (None, [u16p, _c.c_int, u8p, _c.c_int, _c.c_int, _c.c_int, _c.c_float,
                                  _c.c_float, _c.c_float, _c.c_int, _c.c_int, f32p]),
        "g4o_rope_tables": (None, [_c.c_double, _c.c_int, _c.c_int, f32p, f32p]),
        "g4o_rope_rows": (None, [u16p, _c.c_int, _c.c_int, _c.c_int, i32p, f32p, f32p, u16p]),
        "g4o_kv_scale": (_c.c_float, [_c.c_float, _c.c_int]),
        "g4o_kv_code": (_c.c_int, [_c.c_float, _c.c_float, _c.c_int]),
        "g4o_k5_pack_row": (None, [u8p, u8p]),
        "g4o_rope_append": (None, [u16p, _c.c_long, u16p, _c.c_long, u16p, _c.c_long, f32p,
                                   f32p, _c.c_int, _c.c_int, _c.c_int, _c.c_int, i32p, i32p,
                                   _c.c_int, _c.c_int, _c.c_int, _c.c_int, u16p, _c.c_long,
                                   vp, vp, f32p, f32p, _c.c_int]),
        "g4o_row_table": (None, [i32p, _c.c_int, _c.c_int, i32p]),
        "g4o_prefill_attn": (None, [u16p, _c.c_int, _c.c_int, _c.c_int, _c.c_int, _c.c_float, vp,
                                    vp, f32p, f32p, _c.c_int, _c.c_int, _c.c_int, _c.c_int,
                                    i32p, _c.c_int, u16p]),
        "g4o_attn_split": (None, [u16p, _c.c_int, _c.c_int, _c.c_int, _c.c_int, _c.c_float, vp,
                                  vp, f32p, f32p, _c.c_int, _c.c_int, _c.c_int, i32p,
                                  _c.POINTER(i32p), _c.c_int, _c.c_int, u16p]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def bf16_to_f32(b):
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(f):
    """Vectorised twin of g4o_f32_to_bf16 (the reference's RNE formula)."""
    u = np.asarray(f, np.float32).view(np.uint32).astype(np.uint64)
    u = u + 0x7FFF + ((u >> 16) & 1)
    return ((u >> 16) & 0xFFFF).astype(np.uint16)


def uniform_bf16(seed, a, n):
    out = np.empty(n, np.uint16)
    lib.g4o_fill_uniform_bf16(seed, a, n, _p(out, u16p))
    return out


def normal_bf16(seed, mean, std, n):
    out = np.empty(n, np.uint16)
    lib.g4o_fill_normal_bf16(seed, mean, std, n, _p(out, u16p))
    return out


def u32(seed, n):
    out = np.empty(n, np.uint32)
    lib.g4o_fill_u32(seed, n, _p(out, u32p))
    return out


def fp8_quantize(x):
    x = np.ascontiguousarray(x, np.uint16)
    codes = np.empty(x.size, np.uint8)
    s = lib.g4o_fp8_quantize_bf16(_p(x, u16p), x.size, _p(codes, u8p))
    return codes.reshape(x.shape), s


def fp8_encode_scaled(x, scale):
    x = np.ascontiguousarray(x, np.uint16)
    codes = np.empty(x.size, np.uint8)
    lib.g4o_fp8_encode_scaled_bf16(_p(x, u16p), x.size, scale, _p(codes, u8p))
    return codes.reshape(x.shape)


def embed_rows(tokens, emb, mult):
    tokens = np.ascontiguousarray(tokens, np.int32)
    H = emb.shape[1]
    out = np.empty((tokens.size, H), np.uint16)
    lib.g4o_embed_rows(_p(tokens, i32p), tokens.size, _p(emb, u16p), H, mult, _p(out, u16p))
    return out


def rmsnorm(x, w, eps):
    rows, cols = x.shape
    out = np.empty_like(x)
    lib.g4o_rmsnorm(_p(x, u16p), _p(w, u16p), eps, rows, cols, _p(out, u16p))
    return out


def add_rmsnorm(res, branch, mult, w, eps):
    rows, cols = res.shape
    ro = np.empty_like(res)
    no = np.empty_like(res)
    lib.g4o_add_rmsnorm(_p(res, u16p), _p(branch, u16p), mult, _p(w, u16p), eps, rows, cols,
                        _p(ro, u16p), _p(no, u16p))
    return ro, no


def swiglu(gu):
    rows, two_i = gu.shape
    act = np.empty((rows, two_i // 2), np.uint16)
    lib.g4o_swiglu_bf16(_p(np.ascontiguousarray(gu), u16p), rows, two_i // 2, _p(act, u16p))
    return act


def silu_mul_f32(gu):
    """act = bf16(silu(g) * u) of f32 gu [rows][2I] (g4o_silu_mul_f32)."""
    gu = np.ascontiguousarray(gu, np.float32)
    rows, two_i = gu.shape
    act = np.empty((rows, two_i // 2), np.uint16)
    lib.g4o_silu_mul_f32(_p(gu, f32p), two_i // 2, rows, _p(act, u16p))
    return act


def gemm_fp8(A, a_scale, W, scales=(1.0, 1.0, 1.0), segs=None):
    """y [M][N] f32 (g4o_gemm_fp8): exact products, double accumulation."""
    A = np.ascontiguousarray(A, np.uint8)
    W = np.ascontiguousarray(W, np.uint8)
    M, K = A.shape
    N = W.shape[0]
    s1, s2 = segs if segs is not None else (N, N)
    y = np.empty((M, N), np.float32)
    lib.g4o_gemm_fp8(_p(A, u8p), K, a_scale, _p(W, u8p), M, N, K, scales[0], scales[1], scales[2],
                     s1, s2, _p(y, f32p))
    return y


def gemm_bf16w(A, W, scales=(1.0, 1.0, 1.0), segs=None):
    """y [M][N] f32 (g4o_gemm_bf16w): bf16 A [M][K] x e4m3 W [N][K]^T, exact
    products, double accumulation, scale by column segment."""
    A = np.ascontiguousarray(A, np.uint16)
    W = np.ascontiguousarray(W, np.uint8)
    M, K = A.shape
    N = W.shape[0]
    s1, s2 = segs if segs is not None else (N, N)
    y = np.empty((M, N), np.float32)
    lib.g4o_gemm_bf16w(_p(A, u16p), K, _p(W, u8p), M, N, K, scales[0], scales[1], scales[2], s1,
                       s2, _p(y, f32p))
    return y


def gemv_fp8w(a, W, scale):
    """y [N] f32 (g4o_gemv_fp8w): bf16 a [K] x e4m3 W [N][K], double sum."""
    a = np.ascontiguousarray(a, np.uint16)
    W = np.ascontiguousarray(W, np.uint8)
    N, K = W.shape
    y = np.empty(N, np.float32)
    lib.g4o_gemv_fp8w(_p(a, u16p), _p(W, u8p), N, K, scale, _p(y, f32p))
    return y


def fp8_codes(seed, shape, std=1.0):
    """Seeded e4m3 codes of N(0, std) values (finite codes only)."""
    x = normal_bf16(seed, 0.0, std, int(np.prod(shape)))
    codes = fp8_encode_scaled(x, 1.0)
    return codes.reshape(shape)


def rope_tables(theta, d, max_pos):
    c = np.empty((max_pos, d // 2), np.float32)
    s = np.empty((max_pos, d // 2), np.float32)
    lib.g4o_rope_tables(theta, d, max_pos, _p(c, f32p), _p(s, f32p))
    return c, s


def rope_rows(x, pos, cos_t, sin_t):
    rows, heads, d = x.shape
    out = np.empty_like(x)
    pos = np.ascontiguousarray(pos, np.int32)
    lib.g4o_rope_rows(_p(x, u16p), rows, heads, d, _p(pos, i32p), _p(cos_t, f32p),
                      _p(sin_t, f32p), _p(out, u16p))
    return out


KV_ROW_BYTES = {16: (256, 256), 8: (128, 128), 4: (64, 64), 5: (80, 64)}


def rope_append(q, k, v, cos_t, sin_t, pos, arena_row, bits, group, stride, Hk, d=128,
                rotate_k=True, k_round_bf16=False, cache_k=None, cache_v=None,
                k_scale=None, v_scale=None):
    """q: [rows][Hq*d] or None; k, v: [rows][Hk*d] (uint16 arrays, any row stride).
    Returns q_rot, cache_k, cache_v, k_scale, v_scale (caches updated in place when given)."""
    rows = k.shape[0]
    Hq = 0 if q is None else q.shape[1] // d
    kb, vb = {16: (2 * d, 2 * d), 8: (d, d), 4: (d // 2, d // 2),
              5: (d // 2 + d // 8, d // 2)}[bits]
    if cache_k is None:
        cache_k = np.zeros(Hk * stride * kb, np.uint8)
        cache_v = np.zeros(Hk * stride * vb, np.uint8)
        k_scale = np.zeros(Hk * stride * (d // group), np.float32)
        v_scale = np.zeros(Hk * stride * (d // group), np.float32)
    q_rot = None if q is None else np.empty((rows, Hq * d), np.uint16)
    pos = np.ascontiguousarray(pos, np.int32)
    arena_row = np.ascontiguousarray(arena_row, np.int32)
    lib.g4o_rope_append(_p(q, u16p), 0 if q is None else q.strides[0] // 2,
                        _p(k, u16p), k.strides[0] // 2, _p(v, u16p), v.strides[0] // 2,
                        _p(cos_t, f32p), _p(sin_t, f32p), rows, Hq, Hk, d, _p(pos, i32p),
                        _p(arena_row, i32p), bits, group, int(rotate_k), int(k_round_bf16),
                        _p(q_rot, u16p), Hq * d, cache_k.ctypes.data, cache_v.ctypes.data,
                        _p(k_scale, f32p), _p(v_scale, f32p), stride)
    return q_rot, cache_k, cache_v, k_scale, v_scale


def row_table(block_table, n, page=16):
    bt = np.ascontiguousarray(block_table, np.int32)
    out = np.empty(n, np.int32)
    lib.g4o_row_table(_p(bt, i32p), n, page, _p(out, i32p))
    return out


def config2_page_tables(rs, n, pool_pages, max_pos=65536):
    """BASELINE config 2's sessions: n positions drawn from [0, max_pos), each
    session with a page table over all max_pos / 16 of its pages. Every page
    maps to a random page of a small pool (repeats allowed, as no other page
    is written); the n pages that hold the sessions' positions map to n
    distinct pool pages, so the n rows written never collide. Returns the
    positions and the per-session row tables (int32 [max_pos])."""
    pos = rs.integers(0, max_pos, n).astype(np.int32)
    own = rs.permutation(pool_pages)[:n].astype(np.int32)
    pts = []
    for i in range(n):
        bt = rs.integers(0, pool_pages, max_pos // 16).astype(np.int32)
        bt[pos[i] // 16] = own[i]
        pts.append(row_table(bt, max_pos))
    return pos, pts


ATTN_TILE = 64
ATTN_MAX_SPLITS = 256


def attn_tiles_per_split(max_len):
    """Tiles per split of the split-KV attention (attention_split.cu:61-76):
    at most 256 splits of the longest sequence, 64-position tiles."""
    tiles = (max_len + ATTN_TILE - 1) // ATTN_TILE
    return (tiles + ATTN_MAX_SPLITS - 1) // ATTN_MAX_SPLITS


def attn_split(q, cache_k, cache_v, k_scale, v_scale, bits, group, stride, pos, pts=None,
               window=0, scale=1.0 / 128, Hk=8, d=128, tps=None, max_len=None):
    """Oracle split-KV attention. q: uint16 [rows][Hq*d]; pos: per-row positions;
    pts: None or a list of per-row int32 position -> arena-row tables.
    Returns uint16 [rows][Hq*d]."""
    q = np.ascontiguousarray(q, np.uint16)
    rows, Hq = q.shape[0], q.shape[1] // d
    pos = np.ascontiguousarray(pos, np.int32)
    if tps is None:
        tps = attn_tiles_per_split(max_len if max_len else stride)
    out = np.empty((rows, Hq * d), np.uint16)
    keep = None
    arr = None
    if pts is not None:
        keep = [np.ascontiguousarray(t, np.int32) for t in pts]
        arr = (i32p * rows)(*[_p(t, i32p) for t in keep])
    ks = None if k_scale is None else np.ascontiguousarray(k_scale, np.float32)
    vs = None if v_scale is None else np.ascontiguousarray(v_scale, np.float32)
    lib.g4o_attn_split(_p(q, u16p), rows, Hq, Hk, d, scale, cache_k.ctypes.data,
                       cache_v.ctypes.data, _p(ks, f32p), _p(vs, f32p), bits, group, stride,
                       _p(pos, i32p), arr, window, tps, _p(out, u16p))
    return out


def prefill_attn(q, cache_k, cache_v, k_scale, v_scale, bits, group, stride, base_pos, pt=None,
                 window=0, scale=1.0 / 128, Hk=8, d=128):
    """Oracle causal prefill attention: rows q [rows][Hq*d] at positions
    base_pos + r. Returns uint16 [rows][Hq*d]."""
    q = np.ascontiguousarray(q, np.uint16)
    rows, Hq = q.shape[0], q.shape[1] // d
    out = np.empty((rows, Hq * d), np.uint16)
    ks = None if k_scale is None else np.ascontiguousarray(k_scale, np.float32)
    vs = None if v_scale is None else np.ascontiguousarray(v_scale, np.float32)
    ptc = None if pt is None else np.ascontiguousarray(pt, np.int32)
    lib.g4o_prefill_attn(_p(q, u16p), rows, Hq, Hk, d, scale, cache_k.ctypes.data,
                         cache_v.ctypes.data, _p(ks, f32p), _p(vs, f32p), bits, group, stride,
                         base_pos, _p(ptc, i32p), window, _p(out, u16p))
    return out


_REF = []


def ref_lib():
    """The reference-host-math shim (oracle/_ref), or None where it is not built."""
    if _REF:
        return _REF[0]
    if not os.path.exists(REF_SO):
        return None
    r = _c.CDLL(REF_SO)
    r.ref_silu.restype = _c.c_float
    r.ref_silu.argtypes = [_c.c_float]
    r.ref_fp8_encode.restype = _c.c_uint8
    r.ref_fp8_encode.argtypes = [_c.c_double]
    r.ref_rmsnorm_bf16.argtypes = [u16p, u16p, _c.c_float, _c.c_int, _c.c_int, u16p]
    r.ref_rope_tables.argtypes = [_c.c_double, _c.c_int, _c.c_int, f32p, f32p]
    r.ref_gqa_attention_bf16.argtypes = [u16p, u16p, u16p, _c.c_float, _c.c_int, _c.c_int,
                                         _c.c_int, _c.c_int, u16p]
    _REF.append(r)
    return r
