"""The FP8 x FP8 GEMM oracle (g4o_gemm_fp8) pinned without retyping it:
against numpy's float64 matmul of the decoded codes, an exact one-hot case,
and the column-segment scale selection of the reference's GemmEpilogue
(prefill_gemm.h:12-28)."""
import numpy as np
import pytest

import oracle_lib as ol

DEC = np.array([ol.lib.g4o_fp8_decode(c) for c in range(256)])


def test_fp8_decode_table_is_e4m3():
    # e4m3: 1 sign, 4 exponent (bias 7), 3 mantissa bits; 0x7f / 0xff are NaN, no inf.
    assert DEC[0x38] == 1.0 and DEC[0xb8] == -1.0
    assert DEC[0x7e] == 448.0 and DEC[0x01] == 2.0 ** -9
    assert np.isnan(DEC[0x7f]) and np.isnan(DEC[0xff])
    finite = DEC[np.isfinite(DEC)]
    assert finite.size == 254 and np.all(np.abs(finite) <= 448.0)


@pytest.mark.parametrize("M,N,K", [(1, 8, 128), (7, 33, 256), (40, 64, 512)])
def test_gemm_oracle_matches_float64_matmul(M, N, K):
    A = ol.fp8_codes(0x61 + M, (M, K))
    W = ol.fp8_codes(0x62 + N, (N, K), std=0.5)
    y = ol.gemm_fp8(A, 0.37, W, scales=(0.011, 0.011, 0.011))
    want = (np.float64(np.float32(0.37) * np.float32(0.011)) * (DEC[A] @ DEC[W].T)).astype(np.float32)
    np.testing.assert_array_equal(y, want)


def test_gemm_oracle_one_hot_rows_pick_weight_columns():
    K, N = 128, 16
    A = np.zeros((K, K), np.uint8)
    A[np.arange(K), np.arange(K)] = 0x38  # 1.0
    W = ol.fp8_codes(0x63, (N, K))
    y = ol.gemm_fp8(A, 1.0, W, scales=(2.0, 2.0, 2.0))
    np.testing.assert_array_equal(y, (2.0 * DEC[W].T).astype(np.float32))


def test_gemm_oracle_segment_scales():
    K, N = 128, 12
    A = ol.fp8_codes(0x64, (3, K))
    W = ol.fp8_codes(0x65, (N, K))
    y1 = ol.gemm_fp8(A, 1.0, W)
    y = ol.gemm_fp8(A, 1.0, W, scales=(1.0, 0.5, 0.25), segs=(4, 8))
    np.testing.assert_array_equal(y[:, :4], y1[:, :4])
    np.testing.assert_array_equal(y[:, 4:8], (0.5 * y1[:, 4:8].astype(np.float64)).astype(np.float32))
    np.testing.assert_array_equal(y[:, 8:], (0.25 * y1[:, 8:].astype(np.float64)).astype(np.float32))


def test_gemv_oracle_matches_float64_dot():
    K, N = 256, 24
    a = ol.normal_bf16(0x66, 0.0, 1.0, K)
    W = ol.fp8_codes(0x67, (N, K), std=0.5)
    y = ol.gemv_fp8w(a, W, 0.0123)
    exact = DEC[W] @ ol.bf16_to_f32(a).astype(np.float64)
    np.testing.assert_array_equal(y, np.float32(0.0123) * exact.astype(np.float32))


@pytest.mark.parametrize("M,N,K", [(1, 8, 32), (5, 31, 96), (33, 40, 256)])
def test_gemm_bf16w_oracle_matches_float64_matmul(M, N, K):
    """The reference prefill GEMM's value (bf16 A x fp8 W): numpy float64
    matmul of the decoded operands, segment scales applied in double."""
    A = ol.normal_bf16(0x71 + M, 0.0, 1.0, M * K).reshape(M, K)
    W = ol.fp8_codes(0x72 + N, (N, K), std=0.5)
    s1, s2 = N // 3, 2 * N // 3
    y = ol.gemm_bf16w(A, W, scales=(0.011, 0.5, 3.0), segs=(s1, s2))
    S = ol.bf16_to_f32(A).astype(np.float64) @ DEC[W].T
    sc = np.where(np.arange(N) < s1, np.float32(0.011),
                  np.where(np.arange(N) < s2, np.float32(0.5), np.float32(3.0))).astype(np.float64)
    np.testing.assert_array_equal(y, (sc * S).astype(np.float32))


def test_gemm_bf16w_oracle_one_hot_rows_pick_weight_columns():
    K, N = 64, 16
    A = np.zeros((K, K), np.uint16)
    A[np.arange(K), np.arange(K)] = 0x3F80  # bf16 1.0
    W = ol.fp8_codes(0x73, (N, K))
    y = ol.gemm_bf16w(A, W, scales=(0.25, 0.25, 0.25))
    np.testing.assert_array_equal(y, (0.25 * DEC[W].T).astype(np.float32))
