"""Writes tests/golden/golden.npz from the reference's OWN host math.

Run in a container that holds the reference tree: it builds oracle/_ref
(`make -C oracle ref`, which compiles /root/reference/engine/src/fp8_convert.cc,
kv_pool.cc and oracle/ref_shim.cc over kernel_math.h) and calls it through
ctypes. Only the resulting vectors (inputs and expected outputs) are committed;
the reference itself never travels.

Seeds follow the reference's device tests where they exist
(test_kernels.cu: 0x4242 RMSNorm, 0x1337 RoPE, 0x8abc KV8, 0x5a5a K5V4).
"""
import ctypes
import os
import subprocess
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libg4ref.so")

u16p = ctypes.POINTER(ctypes.c_uint16)
f32p = ctypes.POINTER(ctypes.c_float)


def ptr(a, t):
    return a.ctypes.data_as(t)


def load_ref():
    subprocess.check_call(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "ref"])
    lib = ctypes.CDLL(REF_SO)
    lib.ref_f32_to_bf16.restype = ctypes.c_uint16
    lib.ref_f32_to_bf16.argtypes = [ctypes.c_float]
    lib.ref_fp8_encode.restype = ctypes.c_uint8
    lib.ref_fp8_encode.argtypes = [ctypes.c_double]
    lib.ref_fp8_to_bf16.restype = ctypes.c_uint16
    lib.ref_fp8_to_bf16.argtypes = [ctypes.c_uint8]
    lib.ref_fp8_scale_for.restype = ctypes.c_float
    lib.ref_fp8_scale_for.argtypes = [ctypes.c_double]
    lib.ref_fp8_encode_scaled.restype = ctypes.c_uint8
    lib.ref_fp8_encode_scaled.argtypes = [ctypes.c_float, ctypes.c_float]
    lib.ref_residual_add.restype = ctypes.c_uint16
    lib.ref_residual_add.argtypes = [ctypes.c_uint16, ctypes.c_uint16, ctypes.c_float]
    lib.ref_silu.restype = ctypes.c_float
    lib.ref_silu.argtypes = [ctypes.c_float]
    for n in ("kv8", "q4", "k5"):
        getattr(lib, f"ref_{n}_scale").restype = ctypes.c_float
        getattr(lib, f"ref_{n}_scale").argtypes = [ctypes.c_float]
        getattr(lib, f"ref_{n}_quant").restype = ctypes.c_int
        getattr(lib, f"ref_{n}_quant").argtypes = [ctypes.c_float, ctypes.c_float]
    lib.ref_rng_fill_u64.restype = ctypes.c_uint64
    lib.ref_rng_fill_u64.argtypes = [ctypes.c_uint64, ctypes.c_int,
                                     ctypes.POINTER(ctypes.c_uint64)]
    lib.ref_rng_fill_range.argtypes = [ctypes.c_uint64, ctypes.c_double, ctypes.c_int, f32p]
    lib.ref_rope_tables.argtypes = [ctypes.c_double, ctypes.c_int, ctypes.c_int, f32p, f32p]
    lib.ref_rope_half.argtypes = [u16p, f32p, f32p, ctypes.c_int, f32p]
    lib.ref_rmsnorm_bf16.argtypes = [u16p, u16p, ctypes.c_float, ctypes.c_int, ctypes.c_int,
                                     u16p]
    lib.ref_k5_pack_row.argtypes = [ctypes.POINTER(ctypes.c_uint8),
                                    ctypes.POINTER(ctypes.c_uint8)]
    lib.ref_paged_row_tables.restype = ctypes.c_int
    lib.ref_paged_row_tables.argtypes = [ctypes.c_int, ctypes.c_int,
                                         ctypes.POINTER(ctypes.c_int32),
                                         ctypes.POINTER(ctypes.c_int32)]
    return lib


def bf16_of(lib, f32):
    return np.array([lib.ref_f32_to_bf16(float(v)) for v in f32.ravel()],
                    dtype=np.uint16).reshape(f32.shape)


def rng_range(lib, seed, a, n):
    out = np.empty(n, np.float32)
    lib.ref_rng_fill_range(seed, a, n, ptr(out, f32p))
    return out


def main():
    lib = load_ref()
    g = {}

    # --- RNG: first outputs of the reference's xorshift64* ---------------
    for seed in (0x4242, 0x1337, 0):
        out = np.empty(64, np.uint64)
        lib.ref_rng_fill_u64(seed, 64, out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64)))
        g[f"rng_u64_{seed:x}"] = out
    g["rng_range4_4242"] = rng_range(lib, 0x4242, 4.0, 256)

    # --- bf16 rounding of awkward floats ----------------------------------
    f = np.concatenate([rng_range(lib, 0xB16, 1e4, 2048),
                        np.array([1.0 + 2**-8, 1.0 + 3.5 * 2**-7, -0.0, 2**-133, 3.4e38,
                                  -3.4e38, 1e-40], np.float32)]).astype(np.float32)
    g["bf16_in"] = f
    g["bf16_out"] = bf16_of(lib, f)

    # --- FP8 e4m3: every bf16 input, random doubles, every decode ---------
    allbf = np.arange(65536, dtype=np.uint32)
    vals = (allbf << 16).view(np.float32).astype(np.float64)
    g["fp8_enc_allbf16"] = np.array([lib.ref_fp8_encode(float(v)) for v in vals], np.uint8)
    rs = np.random.default_rng(0xC0FFEE)
    mags = np.exp2(rs.uniform(-14.0, 9.5, 8192)) * rs.choice([-1.0, 1.0], 8192)
    ties = []
    for e in range(-6, 9):  # exact midpoints between neighbouring normals
        step = 2.0 ** (e - 3)
        for k in range(8, 16):
            ties.append((k + 0.5) * step)
    ties += [(k + 0.5) * 2.0**-9 for k in range(0, 8)]
    dbl = np.concatenate([mags, np.array(ties), -np.array(ties),
                          np.array([448.0, 463.999, 464.0, 480.0, 1e30, 2**-10, 2**-11])])
    g["fp8_dbl_in"] = dbl
    g["fp8_dbl_out"] = np.array([lib.ref_fp8_encode(float(v)) for v in dbl], np.uint8)
    g["fp8_decode_bf16"] = np.array([lib.ref_fp8_to_bf16(c) for c in range(256)], np.uint16)
    # Scaled encode (the weight quantiser) on bf16 values and several scales.
    xs = bf16_of(lib, rng_range(lib, 0xF8, 8.0, 4096))
    xsf = (xs.astype(np.uint32) << 16).view(np.float32)
    amax = float(np.max(np.abs(xsf)))
    scales = [lib.ref_fp8_scale_for(amax), lib.ref_fp8_scale_for(1.0),
              lib.ref_fp8_scale_for(1e-3), lib.ref_fp8_scale_for(3e4)]
    g["fp8s_x"] = xs
    g["fp8s_amax"] = np.float64(amax)
    g["fp8s_scales"] = np.array(scales, np.float32)
    g["fp8s_codes"] = np.array([[lib.ref_fp8_encode_scaled(float(v), s) for v in xsf]
                                for s in scales], np.uint8)

    # --- residual add -------------------------------------------------------
    ra = bf16_of(lib, rng_range(lib, 0xADD1, 4.0, 4096))
    rb = bf16_of(lib, rng_range(lib, 0xADD2, 4.0, 4096))
    g["resadd_a"], g["resadd_b"] = ra, rb
    for m in (1.0, 0.22):
        g[f"resadd_out_{m}"] = np.array([lib.ref_residual_add(int(a), int(b), m)
                                         for a, b in zip(ra, rb)], np.uint16)

    # --- RMSNorm: 4 rows x 4096 (gen_bf16 seed 0x4242) + a zero row --------
    rows, cols = 5, 4096
    x = bf16_of(lib, rng_range(lib, 0x4242, 4.0, rows * cols)).reshape(rows, cols)
    x[4, :] = 0
    w = bf16_of(lib, rng_range(lib, 0x4243, 1.5, cols))
    out = np.empty_like(x)
    lib.ref_rmsnorm_bf16(ptr(x, u16p), ptr(w, u16p), 1e-5, rows, cols, ptr(out, u16p))
    g["rms_x"], g["rms_w"], g["rms_out"] = x, w, out

    # --- SwiGLU pieces: silu(x) -----------------------------------------------
    sx = np.concatenate([rng_range(lib, 0x5111, 12.0, 2048), np.array([0.0, -0.0, 88.0, -88.0,
                                                                       -104.0, 30.0],
                                                                      np.float32)])
    g["silu_x"] = sx
    g["silu_y"] = np.array([lib.ref_silu(float(v)) for v in sx], np.float32)

    # --- RoPE tables (theta 1e7, d 128) at selected positions + rotations ---
    d, half = 128, 64
    maxp = 65536
    ct = np.empty(maxp * half, np.float32)
    st = np.empty(maxp * half, np.float32)
    lib.ref_rope_tables(1e7, d, maxp, ptr(ct, f32p), ptr(st, f32p))
    sel = np.array([0, 1, 2, 7, 100, 511, 4095, 8191, 57344, 60000, 65535], np.int32)
    g["rope_pos"] = sel
    g["rope_cos"] = ct.reshape(maxp, half)[sel]
    g["rope_sin"] = st.reshape(maxp, half)[sel]
    hx = bf16_of(lib, rng_range(lib, 0x1337, 4.0, len(sel) * 4 * d)).reshape(len(sel), 4, d)
    rot = np.empty((len(sel), 4, d), np.float32)
    for i, p in enumerate(sel):
        for h in range(4):
            lib.ref_rope_half(ptr(np.ascontiguousarray(hx[i, h]), u16p),
                              ptr(np.ascontiguousarray(ct[p * half:(p + 1) * half]), f32p),
                              ptr(np.ascontiguousarray(st[p * half:(p + 1) * half]), f32p),
                              d, ptr(rot[i, h], f32p))
    g["rope_x"], g["rope_out_f32"] = hx, rot
    g["rope_out_bf16"] = bf16_of(lib, rot)

    # --- KV quantisation (test_kernels.cu:355-379 magnitude mix) -----------
    kr, kd = 64, 128
    kvx = np.empty((kr, kd), np.float32)
    for r in range(kr):
        sc = [0.0, 1e-5][r] if r < 2 else [0.25, 3.0, 32.0, 256.0][r % 4]
        kvx[r] = rng_range(lib, 0x8ABC + r, sc, kd)
    kvb = bf16_of(lib, kvx)
    kvf = (kvb.astype(np.uint32) << 16).view(np.float32)
    g["kv_x"] = kvb
    for n in ("kv8", "q4", "k5"):
        sfun = getattr(lib, f"ref_{n}_scale")
        qfun = getattr(lib, f"ref_{n}_quant")
        s = np.array([sfun(float(np.max(np.abs(kvf[r])))) for r in range(kr)], np.float32)
        c = np.array([[qfun(float(v), float(s[r])) for v in kvf[r]] for r in range(kr)],
                     np.int32)
        g[f"{n}_scale"], g[f"{n}_code"] = s, c
    k5c = g["k5_code"].astype(np.uint8)
    packed = np.empty((kr, 80), np.uint8)
    for r in range(kr):
        lib.ref_k5_pack_row(np.ascontiguousarray(k5c[r]).ctypes.data_as(
            ctypes.POINTER(ctypes.c_uint8)), packed[r].ctypes.data_as(
            ctypes.POINTER(ctypes.c_uint8)))
    g["k5_packed"] = packed

    # --- paged row tables -----------------------------------------------------
    seqs, toks = 3, 100
    npg = (toks + 15) // 16
    blocks = np.empty(seqs * npg, np.int32)
    rowt = np.empty(seqs * toks, np.int32)
    rc = lib.ref_paged_row_tables(seqs, toks, blocks.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
                                  rowt.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)))
    assert rc == npg, rc
    g["pt_blocks"], g["pt_rows"] = blocks.reshape(seqs, npg), rowt.reshape(seqs, toks)

    out_path = os.path.join(HERE, "golden.npz")
    np.savez_compressed(out_path, **g)
    print("wrote", out_path, os.path.getsize(out_path), "bytes")


if __name__ == "__main__":
    sys.exit(main())
