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
Z = _c.c_size_t



class GemmEpilogue(_c.Structure):
    """Granite4GemmEpilogue (include/granite4_layerops.h)."""
    _fields_ = [("scale0", F), ("scale1", F), ("scale2", F), ("seg1", I), ("seg2", I),
                ("out_bf16", P), ("out_f32", P), ("residual", P), ("resid_scale", F), ("ldc", I)]


GEMM_BF16, GEMM_F32, GEMM_RESIDUAL = 0, 1, 2


class DecodeLayer(_c.Structure):
    """Granite4DecodeLayer (include/granite4_layerops.h)."""
    _fields_ = [("attn_norm", P), ("wq", P), ("wk", P), ("wv", P), ("wo", P), ("ffn_norm", P),
                ("wg", P), ("wu", P), ("wd", P), ("sq", F), ("sk", F), ("sv", F), ("so", F),
                ("sg", F), ("su", F), ("sd", F), ("cache_k", P), ("cache_v", P),
                ("k_scale", P), ("v_scale", P)]


class DecodeModel(_c.Structure):
    """Granite4DecodeModel (include/granite4_layerops.h)."""
    _fields_ = [("layers", I), ("H", I), ("I", I), ("Hq", I), ("Hk", I), ("vocab", I),
                ("eps", F), ("emb_mult", F), ("resid_mult", F), ("attn_scale", F),
                ("emb", P), ("layer", _c.POINTER(DecodeLayer)), ("final_norm", P),
                ("lm_head", P), ("lm_scale", F), ("cos_tbl", P), ("sin_tbl", P),
                ("max_pos", I), ("kv_bits", I), ("kv_group", I), ("kv_stride", I)]


class DecodeBuffers(_c.Structure):
    """Granite4DecodeBuffers (include/granite4_layerops.h)."""
    _fields_ = [("hidden", P), ("q_rot", P), ("k_rot", P), ("v", P), ("attn_out", P),
                ("act", P), ("attn_scratch", P)]


class BatchBuffers(_c.Structure):
    """Granite4BatchBuffers (include/granite4_layerops.h)."""
    _fields_ = [("max_rows", I), ("hidden", P), ("normed", P), ("qkv", P), ("q_rot", P),
                ("attn", P), ("act", P), ("gu", P), ("codes", P), ("act_codes", P),
                ("scales", P), ("fp8_work", P), ("attn_scratch", P)]


OPS_BF16, OPS_FP8 = 0, 1

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
    "granite4_add_rmsnorm_fp8_noalloc": [P, P, F, P, F, I, I, P, P, P],
    "granite4_swiglu": [P, I, I, P],
    "granite4_swiglu_fp8": [P, I, I, P, P, P, P],
    "granite4_rope_append": [P, L, P, L, P, L, P, P, I, I, I, I, I, I, P, P, P, I, I, I, I, P, L,
                             P, P, P, P, I],
    "granite4_rope_append_at_pos": [P, P, P, P, P, I, P, P, I, I, I, I, I, P, P, P, P, P, I],
    "granite4_row_table": [P, I, I, P],
    "granite4_fp8_work_bytes": [I],
    "granite4_set_fp8_launch_mode": [I],
    "granite4_fp8_sync_status": [P, I],
    "granite4_debug_set_sync_spin_limit": [I],
    "granite4_attn_split_scratch_bytes": [I, I, I],
    "granite4_set_attn_combine_mode": [I],
    "granite4_attn_sync_status": [P, I],
    "granite4_attn_split": [P, P, P, F, I, I, I, I, P, I, I, P, P, P, P, P, P, I, P, P, I, P, I,
                            P, P, P, I, P, P, I, I, I],
    "granite4_attn_paged": [P, I, I, I, I, F, P, P, P, P, I, I, I, I, P, P, P, P, I, I, P, P],
    "granite4_prefill_attn": [P, I, I, I, I, F, P, P, P, P, I, I, I, I, P, I, P],
    "granite4_attn_decode_append": [P, P, P, P, P, I, P, P, I, I, F, P, P, P, P, I, I, I, P, P],
    "granite4_attn_decode_append_rotated": [P, P, P, I, P, P, I, I, F, P, P, P, P, I, I, I, P, P],
    "granite4_prefill_attention": [P, P, P, F, I, I, I, I, I, I, P, P, P, P, P, I, P, P, I, P, I,
                                   I],
    "granite4_gemm_fp8": [I, P, I, P, P, I, I, I, _c.POINTER(GemmEpilogue)],
    "granite4_prefill_gemm": [I, P, I, P, I, I, I, _c.POINTER(GemmEpilogue), P, Z],
    "granite4_prefill_gemm_workspace_bytes": [I, I],
    "granite4_gemm_fp8_swiglu": [P, I, P, P, I, I, I, F, F, P, P, P, P],
    "granite4_gemm_fp8_residual_rmsnorm_fp8": [P, I, P, P, I, I, I, F, P, F, P, F, P, P, P],
    "granite4_kv_layout_offset": [Z, Z, Z, Z, Z, Z, I, Z, Z],
    "granite4_kv_pool_create": [Z, Z, Z, Z, Z],
    "granite4_kv_pool_destroy": [P],
    "granite4_kv_pool_stat": [P, I],
    "granite4_kv_pool_create_sequence": [P],
    "granite4_kv_pool_match_prefix": [P, I, P, Z],
    "granite4_kv_pool_reserve": [P, I, Z, P, Z],
    "granite4_kv_pool_mark_written": [P, I, Z],
    "granite4_kv_pool_locate": [P, I, Z, P],
    "granite4_kv_pool_row_table": [P, I, Z, P],
    "granite4_kv_pool_reset_sequence": [P, I],
    "granite4_kv_pool_truncate_sequence": [P, I, Z],
    "granite4_kv_pool_release": [P, I],
    "granite4_kv_pool_clear": [P],
    "granite4_kv_pool_block_table": [P, I, P, Z],
    "granite4_kv_pool_sequence_tokens": [P, I],
    "granite4_kv_pool_ref_count": [P, Z],
    "granite4_kv_pool_page_in_cache": [P, Z],
    "granite4_kv_ctrl_create": [Z, Z, Z, Z, Z],
    "granite4_kv_ctrl_destroy": [P],
    "granite4_kv_ctrl_stat": [P, I],
    "granite4_kv_ctrl_new_slot": [P],
    "granite4_kv_ctrl_release_slot": [P, I],
    "granite4_kv_ctrl_shutdown": [P],
    "granite4_kv_ctrl_prefill": [P, I, P, Z, P],
    "granite4_kv_ctrl_commit": [P, I, P, Z],
    "granite4_kv_ctrl_open_slot": [P],
    "granite4_kv_ctrl_ensure": [P, I, Z],
    "granite4_kv_ctrl_trim": [P, I, Z],
    "granite4_kv_ctrl_drop": [P, I],
    "granite4_kv_ctrl_pages_missing": [P, I, Z],
    "granite4_kv_ctrl_slot_pages": [P, I],
    "granite4_kv_ctrl_row_table": [P, I, Z, P],
    "granite4_kv_ctrl_committed": [P, I],
    "granite4_kv_ctrl_last_reused": [P, I],
    "granite4_gemv_fp8w": [P, P, F, I, I, P],
    "granite4_gemv_fp8w_resid": [P, P, F, P, F, I, I, P],
    "granite4_gemv_qkv": [P, P, P, P, F, F, F, I, I, I, I, P, P, P],
    "granite4_gemv_rmsnorm_qkv": [P, P, F, P, P, P, F, F, F, I, I, I, I, P, P, P],
    "granite4_gemv_rmsnorm_qkv_rope": [P, P, F, P, P, P, F, F, F, P, P, I, P, I, I, I, P, P, P],
    "granite4_gemv_embed_rmsnorm_qkv_rope": [P, P, I, F, P, P, F, P, P, P, F, F, F, P, P, I, P, I, I,
                                             I, P, P, P],
    "granite4_gemv_qkv_rope": [P, P, P, P, F, F, F, P, P, I, P, I, I, I, P, P, P],
    "granite4_kernel_silu_gate_up": [P, P, P, F, F, I, I, P],
    "granite4_gemv_rmsnorm_silu_gate_up": [P, P, F, P, P, F, F, I, I, P],
    "granite4_gemv_rmsnorm_qkv_rope_append": [P, P, F, P, P, P, F, F, F, P, P, I, P, P, I, I, I, I,
                                              P, P, P, P, P, I],
    "granite4_decode_step": [_c.POINTER(DecodeModel), _c.POINTER(DecodeBuffers), P, P, P, P, P],
    "granite4_prefill_layers": [_c.POINTER(DecodeModel), _c.POINTER(BatchBuffers), P, I, I, P, I,
                                P, P],
    "granite4_decode_step_multi": [_c.POINTER(DecodeModel), _c.POINTER(BatchBuffers), P, I, I, P,
                                   P],
    "granite4_multi_embed": [P, I, P, I, I, F, P],
    "granite4_host_fp8_encode": [P, _c.c_size_t, F, P],
    "granite4_host_kv_codes": [P, _c.c_size_t, F, I, P],
    "granite4_selftest_bf16": [P],
    "granite4_bw_probe": [P, P, _c.c_size_t, I, I],
    "granite4_floor_probe": [P, Z, P, Z, P, I, I],
    "granite4_selftest_fp8": [F, P],
}
_RESTYPE = {"granite4_get_stream": P, "granite4_fp8_work_bytes": Z,
            "granite4_prefill_gemm_workspace_bytes": Z,
            "granite4_attn_split_scratch_bytes": Z, "granite4_kv_pool_create": P,
            "granite4_kv_ctrl_create": P}
for _name, _args in _SIG.items():
    if os.environ.get("G4_LAYEROPS_LIB") and not hasattr(_lib, _name):
        continue  # another build under A/B measurement may predate this entry point
    _fn = getattr(_lib, _name)
    _fn.argtypes = _args
    if _name in _RESTYPE:
        _fn.restype = _RESTYPE[_name]
    elif _name.endswith(("_destroy", "_reset_sequence", "_truncate_sequence", "_release",
                         "_clear", "_release_slot", "_shutdown", "_commit", "_trim", "_drop")):
        _fn.restype = None
    elif _name.startswith("granite4_kv_") and not _name.endswith(
            ("_create_sequence", "_reserve", "_mark_written", "_locate", "_row_table",
             "_page_in_cache", "_new_slot", "_prefill", "_open_slot", "_ensure")):
        _fn.restype = Z
    else:
        _fn.restype = I

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


def set_attn_combine_mode(mode):
    """granite4_set_attn_combine_mode: 0 = the split blocks' partials combined
    inside the split launch, 1 = by a second launch. Returns the previous
    mode."""
    prev = _lib.granite4_set_attn_combine_mode(mode)
    if prev < 0:
        raise ValueError(f"attention combine mode {mode}")
    return prev


def attn_sync_status(scratch, clear=False):
    """granite4_attn_sync_status: 1 if a fused-combine wait on this attention
    scratch gave up since the last clear (or zero fill), else 0."""
    rc = _lib.granite4_attn_sync_status(_ptr(scratch), int(bool(clear)))
    if rc < 0:
        raise Granite4Error("granite4_attn_sync_status failed")
    return rc


class LayerSteps:
    """granite4_prefill_layers / granite4_decode_step_multi over torch
    tensors: the model as DecodeStep takes it (`layers` dicts, keyword model
    fields); device buffers for up to `max_rows` rows are allocated once.
    prefill(tokens, start, rows, pt, ops) and multi(d_rows, rows, ops) launch
    on the current library stream (capturable)."""

    def __init__(self, layers, H, I, Hq, Hk, vocab, emb, cos, sin, max_rows, eps=1e-5,
                 emb_mult=1.0, resid_mult=1.0, attn_scale=1.0 / 128, final_norm=None,
                 lm_head=None, lm_scale=1.0, kv_bits=16, kv_group=128, kv_stride=0,
                 device="cuda"):
        self._keep = [layers, emb, cos, sin, final_norm, lm_head]
        arr = (DecodeLayer * len(layers))()
        for i, ly in enumerate(layers):
            for f in DecodeStep._LAYER_PTRS:
                setattr(arr[i], f, _ptr(ly.get(f)))
            for f in ("sq", "sk", "sv", "so", "sg", "su", "sd"):
                setattr(arr[i], f, float(ly[f]))
        self._arr = arr
        self.model = DecodeModel(len(layers), H, I, Hq, Hk, vocab, eps, emb_mult, resid_mult,
                                 attn_scale, _ptr(emb), arr, _ptr(final_norm), _ptr(lm_head),
                                 lm_scale, _ptr(cos), _ptr(sin), cos.shape[0], kv_bits, kv_group,
                                 kv_stride)
        bf, R = torch.bfloat16, max_rows
        nq, nqkv = Hq * 128, (Hq + 2 * Hk) * 128
        self.hidden = torch.empty((R, H), dtype=bf, device=device)
        self.normed = torch.empty((R, H), dtype=bf, device=device)
        self.qkv = torch.empty((R, nqkv), dtype=bf, device=device)
        self.q_rot = torch.empty((R, nq), dtype=bf, device=device)
        self.attn = torch.empty((R, nq), dtype=bf, device=device)
        self.act = torch.empty((R, I), dtype=bf, device=device)
        self.gu = torch.empty((R, 2 * I), dtype=torch.float32, device=device)
        self.codes = torch.empty((R, H), dtype=torch.uint8, device=device)
        self.act_codes = torch.empty((R, I), dtype=torch.uint8, device=device)
        self.scales = torch.zeros(2, dtype=torch.float32, device=device)
        self.fp8_work = fp8_workspace(R, device)
        self.attn_scratch = torch.zeros(
            _lib.granite4_attn_split_scratch_bytes(Hq, min(R, MAX_VERIFY_ROWS), kv_stride),
            dtype=torch.uint8, device=device)
        self.buffers = BatchBuffers(R, *[_ptr(t) for t in (
            self.hidden, self.normed, self.qkv, self.q_rot, self.attn, self.act, self.gu,
            self.codes, self.act_codes, self.scales, self.fp8_work, self.attn_scratch)])

    def prefill(self, tokens, start, rows, pt=None, ops=OPS_BF16, hidden_out=None, logits=None):
        _check(_lib.granite4_prefill_layers(_c.byref(self.model), _c.byref(self.buffers),
                                            _ptr(tokens), int(start), int(rows), _ptr(pt),
                                            int(ops), _ptr(hidden_out), _ptr(logits)),
               "granite4_prefill_layers")

    def multi(self, d_rows, rows, ops=OPS_BF16, hidden_out=None, logits=None):
        _check(_lib.granite4_decode_step_multi(_c.byref(self.model), _c.byref(self.buffers),
                                               _ptr(d_rows), int(rows), int(ops),
                                               _ptr(hidden_out), _ptr(logits)),
               "granite4_decode_step_multi")


class DecodeStep:
    """granite4_decode_step over torch tensors: `layers` is a list of dicts
    with the Granite4DecodeLayer fields (tensors or pointers, floats for the
    scales); the model fields are keyword arguments. Allocates the step's
    device buffers once; __call__ launches one step on the current library
    stream (capturable)."""

    _LAYER_PTRS = ("attn_norm", "wq", "wk", "wv", "wo", "ffn_norm", "wg", "wu", "wd", "cache_k",
                   "cache_v", "k_scale", "v_scale")

    def __init__(self, layers, H, I, Hq, Hk, vocab, emb, cos, sin, eps=1e-5, emb_mult=1.0,
                 resid_mult=1.0, attn_scale=1.0 / 128, final_norm=None, lm_head=None,
                 lm_scale=1.0, kv_bits=16, kv_group=128, kv_stride=0, device="cuda"):
        self._keep = [layers, emb, cos, sin, final_norm, lm_head]
        arr = (DecodeLayer * len(layers))()
        for i, ly in enumerate(layers):
            for f in self._LAYER_PTRS:
                setattr(arr[i], f, _ptr(ly.get(f)))
            for f in ("sq", "sk", "sv", "so", "sg", "su", "sd"):
                setattr(arr[i], f, float(ly[f]))
        self._arr = arr
        self.model = DecodeModel(len(layers), H, I, Hq, Hk, vocab, eps, emb_mult, resid_mult,
                                 attn_scale, _ptr(emb), arr, _ptr(final_norm), _ptr(lm_head),
                                 lm_scale, _ptr(cos), _ptr(sin), cos.shape[0], kv_bits, kv_group,
                                 kv_stride)
        bf = torch.bfloat16
        self.hidden = torch.empty(H, dtype=bf, device=device)
        self.q_rot = torch.empty(Hq * 128, dtype=bf, device=device)
        self.k_rot = torch.empty(Hk * 128, dtype=bf, device=device)
        self.v = torch.empty(Hk * 128, dtype=bf, device=device)
        self.attn_out = torch.empty(Hq * 128, dtype=bf, device=device)
        self.act = torch.empty(I, dtype=bf, device=device)
        self.scratch = torch.zeros(_lib.granite4_attn_split_scratch_bytes(Hq, 1, kv_stride),
                                   dtype=torch.uint8, device=device)
        self.buffers = DecodeBuffers(*[_ptr(t) for t in (self.hidden, self.q_rot, self.k_rot,
                                                          self.v, self.attn_out, self.act,
                                                          self.scratch)])

    def __call__(self, tokens, pos, pt=None, hidden_out=None, logits=None):
        _check(_lib.granite4_decode_step(_c.byref(self.model), _c.byref(self.buffers),
                                         _ptr(tokens), _ptr(pos), _ptr(pt), _ptr(hidden_out),
                                         _ptr(logits)), "granite4_decode_step")


def fp8_sync_status(work, clear=False):
    """granite4_fp8_sync_status: 0 if no single-launch FP8 call on `work`
    gave up waiting (NaN scale) since the last clear, 1 if one did."""
    rc = _lib.granite4_fp8_sync_status(_ptr(work), int(bool(clear)))
    if rc < 0:
        raise Granite4Error("granite4_fp8_sync_status failed")
    return rc


def set_sync_spin_limit(limit):
    """granite4_debug_set_sync_spin_limit (test hook). Returns the previous limit."""
    prev = _lib.granite4_debug_set_sync_spin_limit(int(limit))
    if prev < 0:
        raise ValueError(f"spin limit {limit}")
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


def prefill_gemm(A, W, out_kind=GEMM_BF16, scales=(1.0, 1.0, 1.0), segs=None, out=None,
                 residual=None, resid_scale=1.0):
    """granite4_prefill_gemm (the reference's prefill_gemm): A [M][K] bf16
    (row pitch A.stride(0)), W [N][K] e4m3 codes (uint8). Returns out [M][N]
    (bf16, or f32 for GEMM_F32; in place for GEMM_RESIDUAL when out is
    residual)."""
    M, K = A.shape
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
    call("granite4_prefill_gemm", out_kind, A, A.stride(0), W, M, N, K, ep, None, 0)
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


# ----------------------------------------------------------------------------
# Host page-table controller (include/granite4_kv_pool.h): the reference's
# PagedKV / KvPoolController (kv_pool.h, kv_pool_controller.h) by name.
# ----------------------------------------------------------------------------

import numpy as _np  # noqa: E402

KV_STATS = {"pool_pages": 0, "free_pages": 1, "used_pages": 2, "shared_pages": 3,
            "cached_pages": 4, "retained_pages": 5, "evicted_pages": 6, "live_sequences": 7,
            "capacity_tokens": 8, "page_bytes": 9, "tokens_per_page": 10}
NO_INDEX = (1 << (8 * _c.sizeof(Z))) - 1


def _ids(tokens):
    a = _np.ascontiguousarray(_np.asarray(tokens, dtype=_np.uint32))
    return a, a.ctypes.data, a.size


def kv_layout_offset(layers, kv_heads, head_dim, tokens_per_page, token_local, layer, kv, head,
                     dim):
    return _lib.granite4_kv_layout_offset(layers, kv_heads, head_dim, tokens_per_page,
                                          token_local, layer, kv, head, dim)


class _Handle:
    _prefix = ""

    def __getattr__(self, name):
        if name in KV_STATS:
            return lambda: getattr(_lib, self._prefix + "stat")(self._h, KV_STATS[name])
        raise AttributeError(name)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            getattr(_lib, self._prefix + "destroy")(h)
            self._h = None


class PagedKV(_Handle):
    """granite4::PagedKV over the C ABI (sized as KvPoolConfig::from_budget)."""
    _prefix = "granite4_kv_pool_"

    def __init__(self, layers, kv_heads, head_dim, tokens_per_page, budget_bytes):
        self._h = _lib.granite4_kv_pool_create(layers, kv_heads, head_dim, tokens_per_page,
                                               budget_bytes)
        if not self._h:
            raise Granite4Error("granite4_kv_pool_create failed")

    def create_sequence(self):
        return _lib.granite4_kv_pool_create_sequence(self._h)

    def match_prefix(self, seq, tokens):
        _a, p, n = _ids(tokens)
        return _lib.granite4_kv_pool_match_prefix(self._h, seq, p, n)

    def reserve(self, seq, token_count, tokens):
        _a, p, n = _ids(tokens)
        return bool(_lib.granite4_kv_pool_reserve(self._h, seq, token_count, p, n))

    def mark_written(self, seq, page_index):
        return bool(_lib.granite4_kv_pool_mark_written(self._h, seq, page_index))

    def locate(self, seq, token):
        out = (Z * 2)()
        _lib.granite4_kv_pool_locate(self._h, seq, token, out)
        return (out[0], out[1])

    def row_table(self, seq, n):
        out = _np.empty(n, _np.int32)
        if _lib.granite4_kv_pool_row_table(self._h, seq, n, out.ctypes.data) != 0:
            return None
        return out

    def reset_sequence(self, seq):
        _lib.granite4_kv_pool_reset_sequence(self._h, seq)

    def truncate_sequence(self, seq, n_tokens):
        _lib.granite4_kv_pool_truncate_sequence(self._h, seq, n_tokens)

    def release(self, seq):
        _lib.granite4_kv_pool_release(self._h, seq)

    def clear(self):
        _lib.granite4_kv_pool_clear(self._h)

    def block_table(self, seq):
        n = _lib.granite4_kv_pool_block_table(self._h, seq, None, 0)
        out = (Z * max(1, n))()
        _lib.granite4_kv_pool_block_table(self._h, seq, out, n)
        return [out[i] for i in range(n)]

    def sequence_tokens(self, seq):
        return _lib.granite4_kv_pool_sequence_tokens(self._h, seq)

    def ref_count(self, page_id):
        return _lib.granite4_kv_pool_ref_count(self._h, page_id)

    def page_in_cache(self, page_id):
        return bool(_lib.granite4_kv_pool_page_in_cache(self._h, page_id))


class KvPoolController(_Handle):
    """granite4::KvPoolController over the C ABI."""
    _prefix = "granite4_kv_ctrl_"

    def __init__(self, layers, kv_heads, head_dim, tokens_per_page, budget_bytes):
        self._h = _lib.granite4_kv_ctrl_create(layers, kv_heads, head_dim, tokens_per_page,
                                               budget_bytes)
        if not self._h:
            raise Granite4Error("granite4_kv_ctrl_create failed")

    def max_slots(self):
        return self.pool_pages()

    def new_slot(self):
        return _lib.granite4_kv_ctrl_new_slot(self._h)

    def release_slot(self, slot):
        _lib.granite4_kv_ctrl_release_slot(self._h, slot)

    def shutdown(self):
        _lib.granite4_kv_ctrl_shutdown(self._h)

    def prefill(self, slot, prompt):
        """Returns (ok, reused)."""
        _a, p, n = _ids(prompt)
        reused = Z(0)
        ok = _lib.granite4_kv_ctrl_prefill(self._h, slot, p, n, _c.byref(reused)) == 0
        return ok, reused.value

    def commit(self, slot, tokens):
        _a, p, n = _ids(tokens)
        _lib.granite4_kv_ctrl_commit(self._h, slot, p, n)

    def open_slot(self):
        return _lib.granite4_kv_ctrl_open_slot(self._h)

    def ensure(self, slot, n_tokens):
        return bool(_lib.granite4_kv_ctrl_ensure(self._h, slot, n_tokens))

    def trim(self, slot, n_tokens):
        _lib.granite4_kv_ctrl_trim(self._h, slot, n_tokens)

    def drop(self, slot):
        _lib.granite4_kv_ctrl_drop(self._h, slot)

    def pages_missing(self, slot, n_tokens):
        return _lib.granite4_kv_ctrl_pages_missing(self._h, slot, n_tokens)

    def slot_pages(self, slot):
        return _lib.granite4_kv_ctrl_slot_pages(self._h, slot)

    def row_table(self, slot, n):
        out = _np.empty(n, _np.int32)
        if _lib.granite4_kv_ctrl_row_table(self._h, slot, n, out.ctypes.data) != 0:
            return None
        return out

    def committed(self, slot):
        return _lib.granite4_kv_ctrl_committed(self._h, slot)

    def last_reused(self, slot):
        return _lib.granite4_kv_ctrl_last_reused(self._h, slot)
