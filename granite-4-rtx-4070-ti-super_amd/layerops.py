"""Host-side mirror of the reference engine's layer-op launchers over the
gfx950 library (lib/libgranite4_layerops.so, built by build.py).

The names and argument meaning follow the reference's C ABI and C++ launchers
(kernels_phase2.cu:868-1181, prefill_gemm.h:41-105, forward_gpu_api.h:219-229);
the fused entry points the MI355X build adds are documented in
include/granite4_layerops.h. Every call goes through the C ABI with plain
device pointers; a -1 return raises Granite4Error, as the reference's callers
treat -1 as a hard failure. There is no CPU fallback: if the library is not
built, importing this module fails.

PyTorch provides device memory and streams only. Tensors are passed by
data_ptr(); bf16 values may be torch.bfloat16 or int16/uint16 bit patterns.
"""
import ctypes
import os

import torch  # noqa: F401  (loads the HIP runtime first, so the library binds to it)

PKG = os.path.dirname(os.path.abspath(__file__))
# G4_LAYEROPS_LIB selects another build of the same library (A/B measurements).
LIB_PATH = os.environ.get("G4_LAYEROPS_LIB") or os.path.join(PKG, "lib", "libgranite4_layerops.so")

FP8_MAX_PARTIALS = 1024
MAX_VERIFY_ROWS = 16


class Granite4Error(RuntimeError):
    pass


if not os.path.exists(LIB_PATH):
    raise ImportError(f"{LIB_PATH} is not built: run python granite-4-rtx-4070-ti-super_amd/build.py")

_c = ctypes
_lib = _c.CDLL(LIB_PATH)
P = _c.c_void_p
I = _c.c_int
F = _c.c_float
D = _c.c_double
L = _c.c_long



class GemmEpilogue(_c.Structure):
    """Granite4GemmEpilogue (include/granite4_layerops.h)."""
    _fields_ = [("scale0", F), ("scale1", F), ("scale2", F), ("seg1", I), ("seg2", I),
                ("out_bf16", P), ("out_f32", P), ("residual", P), ("resid_scale", F), ("ldc", I)]


GEMM_BF16, GEMM_F32, GEMM_RESIDUAL = 0, 1, 2

_SIG = {
    "granite4_set_stream": [P],
    "granite4_get_stream": [],
    "granite4_device_arch": [_c.c_char_p, I],
    "granite4_rope_tables_build": [D, I, I, _c.POINTER(P), _c.POINTER(P)],
    "granite4_rope_tables_free": [P, P],
    "granite4_rope_tables_fill": [D, I, I, P, P],
    "granite4_kernel_rmsnorm": [P, P, F, I, I, P],
    "granite4_kernel_rmsnorm_batched": [P, P, F, I, I, P],
    "granite4_kernel_rope": [P, P, P, I, I, P],
    "granite4_kernel_rope_at_pos": [P, P, P, I, I, P],
    "granite4_kernel_rope_at_pos_batched": [P, P, P, I, I, I, P],
    "granite4_kernel_kv_append_batched": [P, P, P, P, I, I, I, I, I, P],
    "granite4_kernel_kv_append_int8_batched": [P, P, P, P, P, P, I, I, I, I, I, P],
    "granite4_kernel_kv_append_int4_batched": [P, P, P, P, P, P, I, I, I, I, I, P],
    "granite4_kernel_kv_append_k5v4_batched": [P, P, P, P, P, P, I, I, I, I, I, P],
    "granite4_kernel_verify_qkv_stage": [P, P, P, P, P, I, I, I, I, I, I, P, P, P, P, P],
    "granite4_prefill_embed_rows": [P, I, I, P, F, P, I],
    "granite4_prefill_rope_split_append": [P, P, P, I, I, I, I, I, I, P, P, P, P],
    "granite4_prefill_rope_split_append_int8": [P, P, P, I, I, I, I, I, I, P, P, P, P, P, P],
    "granite4_prefill_rope_split_append_int4": [P, P, P, I, I, I, I, I, I, P, P, P, P, P, P],
    "granite4_prefill_rope_split_append_k5v4": [P, P, P, I, I, I, I, I, I, P, P, P, P, P, P],
    "granite4_prefill_silu_mul": [P, I, I, P],
    "granite4_multi_rope": [P, P, P, P, I, I, I, P],
    "granite4_multi_rope_append": [P, P, P, P, P, P, I, I, I, I, I, P, P, P, P, I, P],
    "granite4_multi_kv_append": [P, P, I, P, P, P, P, P, I, I, I, I],
    "granite4_embed_rows": [P, I, P, I, I, F, P],
    "granite4_embed_at_pos": [P, P, P, I, I, F, P],
    "granite4_add_rmsnorm": [P, P, F, P, F, I, I, P, P],
    "granite4_add_rmsnorm_fp8": [P, P, F, P, F, I, I, P, P, P, P],
    "granite4_swiglu": [P, I, I, P],
    "granite4_swiglu_fp8": [P, I, I, P, P, P, P],
    "granite4_rope_append": [P, L, P, L, P, L, P, P, I, I, I, I, I, I, P, P, P, I, I, I, I, P, L,
                             P, P, P, P, I],
    "granite4_rope_append_at_pos": [P, P, P, P, P, I, P, P, I, I, I, I, I, P, P, P, P, P, I],
    "granite4_row_table": [P, I, I, P],
    "granite4_fp8_work_bytes": [I],
    "granite4_set_fp8_launch_mode": [I],
    "granite4_attn_split_scratch_bytes": [I, I, I],
    "granite4_attn_split": [P, P, P, F, I, I, I, I, P, I, I, P, P, P, P, P, P, I, P, P, I, P, I,
                            P, P, P, I, P, P, I, I, I],
    "granite4_attn_paged": [P, I, I, I, I, F, P, P, P, P, I, I, I, I, P, P, P, P, I, I, P, P],
    "granite4_prefill_attn": [P, I, I, I, I, F, P, P, P, P, I, I, I, I, P, I, P],
    "granite4_prefill_attention": [P, P, P, F, I, I, I, I, I, I, P, P, P, P, P, I, P, P, I, P, I,
                                   I],
    "granite4_gemm_fp8": [I, P, I, P, P, I, I, I, _c.POINTER(GemmEpilogue)],
    "granite4_gemm_fp8_swiglu": [P, I, P, P, I, I, I, F, F, P, P, P, P],
    "granite4_gemm_fp8_residual_rmsnorm_fp8": [P, I, P, P, I, I, I, F, P, F, P, F, P, P, P],
    "granite4_host_fp8_encode": [P, _c.c_size_t, F, P],
    "granite4_host_kv_codes": [P, _c.c_size_t, F, I, P],
    "granite4_selftest_bf16": [P],
    "granite4_bw_probe": [P, P, _c.c_size_t, I, I],
    "granite4_selftest_fp8": [F, P],
}
for _name, _args in _SIG.items():
    _fn = getattr(_lib, _name)
    _fn.argtypes = _args
    _fn.restype = {"granite4_get_stream": P, "granite4_fp8_work_bytes": _c.c_size_t,
                   "granite4_attn_split_scratch_bytes": _c.c_size_t}.get(_name, I)

lib = _lib


def _ptr(t):
    if t is None:
        return None
    if isinstance(t, int):
        return t
    return t.data_ptr()


def _check(rc, name):
    if rc != 0:
        raise Granite4Error(f"{name} returned {rc}")


def call(name, *args):
    """Calls a C entry point by name; tensors are passed as device pointers."""
    conv = [(_ptr(a) if (a is None or isinstance(a, torch.Tensor)) else a) for a in args]
    _check(getattr(_lib, name)(*conv), name)


def call_size(name, *args):
    """Calls a C entry point that returns a size (not a status)."""
    return getattr(_lib, name)(*args)


def use_stream(stream=None):
    """Launch on `stream` (a torch.cuda.Stream) or torch's current stream."""
    if stream is None:
        stream = torch.cuda.current_stream()
    _lib.granite4_set_stream(stream.cuda_stream)


def set_fp8_launch_mode(mode):
    """granite4_set_fp8_launch_mode: 0 = single launch where it fits, 1 = two
    launches. Returns the previous mode."""
    prev = _lib.granite4_set_fp8_launch_mode(mode)
    if prev < 0:
        raise ValueError(f"FP8 launch mode {mode}")
    return prev


def device_arch():
    buf = _c.create_string_buffer(64)
    if _lib.granite4_device_arch(buf, 64) != 0:
        return None
    return buf.value.decode()


# ----------------------------------------------------------------------------
# Reference-named operators (tensor in, tensor out). Shapes as in the reference.
# ----------------------------------------------------------------------------

def rope_tables(theta, head_dim, max_pos, device="cuda"):
    """Non-allocating table build into torch tensors ([max_pos][head_dim/2] f32)."""
    c = torch.empty((max_pos, head_dim // 2), dtype=torch.float32, device=device)
    s = torch.empty_like(c)
    call("granite4_rope_tables_fill", theta, head_dim, max_pos, c, s)
    return c, s


def rmsnorm(x, w, eps, out=None):
    rows, cols = x.shape
    out = torch.empty_like(x) if out is None else out
    call("granite4_kernel_rmsnorm", x, w, eps, rows, cols, out)
    return out


def add_rmsnorm(res, branch, w, eps, resid_mult=1.0, res_out=None, normed=None):
    rows, cols = res.shape
    res_out = torch.empty_like(res) if res_out is None else res_out
    normed = torch.empty_like(res) if normed is None else normed
    call("granite4_add_rmsnorm", res, branch, resid_mult, w, eps, rows, cols, res_out, normed)
    return res_out, normed


def fp8_work_bytes(rows):
    """GRANITE4_FP8_WORK_BYTES(rows): partials, grid-sync slots, per-row 1/rms."""
    return 12544 + 4 * rows


def fp8_workspace(rows=65536, device="cuda"):
    """Workspace for the FP8 ops on tensors of up to `rows` rows (zero-filled,
    as the single-launch forms' synchronisation slots require)."""
    return torch.zeros(fp8_work_bytes(rows), dtype=torch.uint8, device=device)


def add_rmsnorm_fp8(res, branch, w, eps, work, resid_mult=1.0, res_out=None, codes=None,
                    scale=None):
    rows, cols = res.shape
    res_out = torch.empty_like(res) if res_out is None else res_out
    codes = torch.empty((rows, cols), dtype=torch.uint8, device=res.device) if codes is None else codes
    scale = torch.empty(1, dtype=torch.float32, device=res.device) if scale is None else scale
    call("granite4_add_rmsnorm_fp8", res, branch, resid_mult, w, eps, rows, cols, res_out, codes,
         scale, work)
    return res_out, codes, scale


def _scale_tensor(a_scale, device):
    """A device f32 [1] for an activation scale given as a tensor or a number."""
    if isinstance(a_scale, torch.Tensor):
        return a_scale
    return torch.tensor([float(a_scale)], dtype=torch.float32, device=device)


def gemm_fp8(A, a_scale, W, out_kind=GEMM_BF16, scales=(1.0, 1.0, 1.0), segs=None, out=None,
             residual=None, resid_scale=1.0):
    """granite4_gemm_fp8: A [M][K] and W [N][K] e4m3 codes (uint8 tensors);
    a_scale a device f32 [1] (or a number, copied to the device). Returns out
    [M][N] (bf16, or f32 for GEMM_F32; in place for GEMM_RESIDUAL when out is
    residual)."""
    M, K = A.shape
    a_scale = _scale_tensor(a_scale, A.device)
    N = W.shape[0]
    if out is None:
        out = torch.empty((M, N), dtype=torch.float32 if out_kind == GEMM_F32 else torch.bfloat16,
                          device=A.device)
    s1, s2 = segs if segs is not None else (N, N)
    ep = GemmEpilogue(float(scales[0]), float(scales[1]), float(scales[2]), int(s1), int(s2),
                      None if out_kind == GEMM_F32 else out.data_ptr(),
                      out.data_ptr() if out_kind == GEMM_F32 else None,
                      None if residual is None else residual.data_ptr(), float(resid_scale),
                      out.stride(0))
    call("granite4_gemm_fp8", out_kind, A, A.stride(0), a_scale, W, M, N, K, ep)
    return out


def gemm_fp8_swiglu(A, a_scale, W_gu, gate_scale, up_scale, work, act=None, fp8=True):
    """granite4_gemm_fp8_swiglu: returns act (and codes, scale when fp8)."""
    M, K = A.shape
    a_scale = _scale_tensor(a_scale, A.device)
    I_ = W_gu.shape[0] // 2
    act = torch.empty((M, I_), dtype=torch.bfloat16, device=A.device) if act is None else act
    codes = torch.empty((M, I_), dtype=torch.uint8, device=A.device) if fp8 else None
    scale = torch.empty(1, dtype=torch.float32, device=A.device) if fp8 else None
    call("granite4_gemm_fp8_swiglu", A, A.stride(0), a_scale, W_gu, M, I_, K,
         float(gate_scale), float(up_scale), act, codes, scale, work)
    return (act, codes, scale) if fp8 else act


def swiglu(gu, act=None):
    rows, two_i = gu.shape
    act = torch.empty((rows, two_i // 2), dtype=gu.dtype, device=gu.device) if act is None else act
    call("granite4_swiglu", gu, rows, two_i // 2, act)
    return act


def swiglu_fp8(gu, work, codes=None, scale=None, act=None):
    rows, two_i = gu.shape
    codes = torch.empty((rows, two_i // 2), dtype=torch.uint8, device=gu.device) if codes is None else codes
    scale = torch.empty(1, dtype=torch.float32, device=gu.device) if scale is None else scale
    call("granite4_swiglu_fp8", gu, rows, two_i // 2, codes, scale, work, act)
    return codes, scale


def prefill_embed_rows(tokens, start, rows, emb, mult, out, H):
    call("granite4_prefill_embed_rows", tokens, start, rows, emb, mult, out, H)
    return out


def prefill_silu_mul(gu, I_, rows, act):
    call("granite4_prefill_silu_mul", gu, I_, rows, act)
    return act


_PREFILL = {16: "granite4_prefill_rope_split_append",
            8: "granite4_prefill_rope_split_append_int8",
            4: "granite4_prefill_rope_split_append_int4",
            5: "granite4_prefill_rope_split_append_k5v4"}


def prefill_rope_split_append(bits, qkv, cos, sin, base_pos, rows, Hq, Hk, d, stride, q_rot,
                              cache_k, cache_v, k_scale=None, v_scale=None, d_pt=None):
    if bits == 16:
        call(_PREFILL[16], qkv, cos, sin, base_pos, rows, Hq, Hk, d, stride, q_rot, cache_k,
             cache_v, d_pt)
    else:
        call(_PREFILL[bits], qkv, cos, sin, base_pos, rows, Hq, Hk, d, stride, q_rot, cache_k,
             cache_v, k_scale, v_scale, d_pt)


def kv_row_bytes(bits, d=128):
    return {16: (2 * d, 2 * d), 8: (d, d), 4: (d // 2, d // 2), 5: (d // 2 + d // 8, d // 2)}[bits]


class KvArena:
    """One layer's paged KV arena: K / V [Hk][stride][row bytes] + f32 scales
    [Hk][stride][d / group] (forward_gpu.cu:1315-1343 layout)."""

    def __init__(self, bits, Hk, stride, d=128, group=128, device="cuda", fill=0):
        kb, vb = kv_row_bytes(bits, d)
        self.bits, self.Hk, self.stride, self.d, self.group = bits, Hk, stride, d, group
        self.k = torch.full((Hk, stride, kb), fill, dtype=torch.uint8, device=device)
        self.v = torch.full((Hk, stride, vb), fill, dtype=torch.uint8, device=device)
        ng = d // group
        self.k_scale = torch.zeros((Hk, stride, ng), dtype=torch.float32, device=device)
        self.v_scale = torch.zeros((Hk, stride, ng), dtype=torch.float32, device=device)


def rope_append(arena, q, k, v, cos, sin, base_pos=0, pos_rows=None, d_pt=None,
                arena_rows=None, k_round_bf16=False, rotate_k=True, q_rot=None):
    """Fused RoPE(q, k) + KV write. q: [rows][>= Hq*d] view or None; k, v
    [rows][>= Hk*d] views (row strides honoured)."""
    rows = k.shape[0]
    d = arena.d
    Hq = 0 if q is None else q.shape[1] // d
    if q is not None and q_rot is None:
        q_rot = torch.empty((rows, Hq * d), dtype=q.dtype, device=q.device)
    call("granite4_rope_append", q, 0 if q is None else q.stride(0), k, k.stride(0), v,
         v.stride(0), cos, sin, cos.shape[0], rows, Hq, arena.Hk, d, base_pos, pos_rows, d_pt,
         arena_rows, arena.bits, arena.group, int(k_round_bf16), int(rotate_k), q_rot,
         0 if q_rot is None else q_rot.stride(0), arena.k, arena.v, arena.k_scale,
         arena.v_scale, arena.stride)
    return q_rot


def multi_rows_struct():
    """ctypes twin of GpuMultiRows (forward_gpu_api.h:163-182)."""
    R, T = MAX_VERIFY_ROWS, 8

    class GpuMultiRows(_c.Structure):
        _fields_ = [("n", _c.c_int), ("pos", _c.c_int * R), ("pt", _c.c_void_p * R),
                    ("tok", _c.c_void_p * R), ("grp", _c.c_int * R), ("tree", _c.c_int),
                    ("slot", _c.c_int * R), ("tbase", _c.c_int * R),
                    ("tail", (_c.c_int * T) * R)]
    return GpuMultiRows
