"""NVFP4 (an adjacent GGML format, ggml-common.h:211-217) through the C ABI on
the GPU, against the pinned oracle: row dequantize bit-exact at any base
alignment (the Weft encoding declares none), vec_dot and mul_mat within the
fp64 re-accumulation bar, the Q8_0 Xq workspace bit-exact.  The caller passes
the E2M1 codebook and the UE4M3 decode table as GGML's harness does
(mul_mat_runtime.cpp:579-583).  Extreme records: every scale byte (0x7F and
0xFF included) and every code."""
from __future__ import annotations

import numpy as np
import pytest

import oracle as o
from tests.test_gpu_parity import SENTINEL, acts, assert_close, check_mul_mat, run_mul_mat, weights

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n,k,w_off,y_off", [(64, 4096, 0, 0), (33, 768, 1, 1), (7, 64, 3, 2)])
def test_dequant_nvfp4(hip, n, k, w_off, y_off):
    w = weights("nvfp4", n, k)
    total = n * k
    y = hip.empty(4 * total, fill=SENTINEL, offset=4 * y_off)
    hip.call("row_dequantize_nvfp4", hip.to_dev(w, offset=w_off), hip.codebook, hip.ue4m3, y, total)
    want = o.dequantize("nvfp4", w, k).reshape(-1)
    np.testing.assert_array_equal(y.numpy(np.float32).view(np.uint32), want.view(np.uint32))


def extreme_records():
    """64 records: record r carries scale bytes 4r..4r+3, codes cycling 0..15."""
    recs = np.zeros((64, 36), np.uint8)
    recs[:, 0:4] = np.arange(256, dtype=np.uint8).reshape(64, 4)
    codes = (np.arange(64 * 64) * 7) % 16
    for r in range(64):
        c = codes[64 * r:64 * r + 64].reshape(4, 16)
        recs[r, 4:] = (c[:, :8] | (c[:, 8:] << 4)).reshape(-1)
    return recs


def test_dequant_nvfp4_extreme_records(hip):
    w = extreme_records()
    y = hip.empty(4 * 64 * 64, fill=SENTINEL)
    hip.call("row_dequantize_nvfp4", hip.to_dev(w), hip.codebook, hip.ue4m3, y, 64 * 64)
    want = o.dequantize("nvfp4", w.reshape(1, -1), 64 * 64).reshape(-1)
    np.testing.assert_array_equal(y.numpy(np.float32).view(np.uint32), want.view(np.uint32))


def test_vec_dot_nvfp4(hip):
    for k in (64, 4096, 14336):
        w = weights("nvfp4", 1, k, seed=3)
        xq = o.quantize("q8_0", acts(1, k, seed=4))
        y = hip.empty(4, fill=SENTINEL)
        hip.call("quantized_vec_dot_nvfp4_q8_0", hip.to_dev(w), hip.to_dev(xq), hip.codebook, hip.ue4m3, y, k)
        e, a = o.mul_mat_f64("nvfp4", w, xq, 1, k, 1)
        assert_close(y.numpy(np.float32).reshape(1, 1), e, a, f"vec_dot nvfp4 K={k}")


def test_vec_dot_nvfp4_extreme_records(hip):
    k = 64 * 64
    w = extreme_records().reshape(1, -1)
    x = acts(1, k, seed=8)
    x[0, 512:544] = 0.0                       # an all-zero Q8_0 block
    xq = o.quantize("q8_0", x)
    y = hip.empty(4, fill=SENTINEL)
    hip.call("quantized_vec_dot_nvfp4_q8_0", hip.to_dev(w), hip.to_dev(xq), hip.codebook, hip.ue4m3, y, k)
    e, a = o.mul_mat_f64("nvfp4", w, xq, 1, k, 1)
    assert_close(y.numpy(np.float32).reshape(1, 1), e, a, "vec_dot nvfp4 extremes")


@pytest.mark.parametrize("n,k,m", [(4096, 4096, 1), (11008, 4096, 1), (4096, 14336, 1), (300, 768, 3),
                                   (65, 1024, 5), (1, 64, 1), (17, 1024, 1), (5000, 2048, 1)])
def test_decode_nvfp4(hip, n, k, m):
    """M = 1 with K <= 4096 a multiple of 64 runs the batch-1 kernel (records
    in VGPRs), every other shape the staged GEMV."""
    w, x, xq, y = run_mul_mat(hip, "production_mul_mat_nvfp4_decode", "nvfp4", n, k, m)
    check_mul_mat("nvfp4", w, x, xq, y, n, k, m)


def test_decode_nvfp4_batch1_extreme_records(hip):
    """The batch-1 kernel on rows cycling through all 256 UE4M3 scale bytes
    and every code, against an activation with an all-zero Q8_0 block."""
    n, k = 96, 4096
    recs = extreme_records()
    w = np.stack([np.roll(recs, 3 * r, axis=0) for r in range(n)]).reshape(n, -1)
    x = acts(1, k, seed=15).copy()
    x[0, 32:64] = 0.0
    w, x, xq, y = run_mul_mat(hip, "production_mul_mat_nvfp4_decode", "nvfp4", n, k, 1, w=w, x=x)
    check_mul_mat("nvfp4", w, x, xq, y, n, k, 1)


@pytest.mark.parametrize("n,k,m", [(4096, 4096, 512), (512, 4096, 64), (144, 768, 70), (129, 256, 17),
                                   (300, 320, 40), (64, 512, 15)])
def test_prefill_nvfp4(hip, n, k, m):
    """M >= 16 with K a multiple of 256 runs the int8-MFMA GEMM (ragged
    weight and token tiles included); K = 320 and M = 15 take the GEMV."""
    w, x, xq, y = run_mul_mat(hip, "production_mul_mat_nvfp4", "nvfp4", n, k, m)
    check_mul_mat("nvfp4", w, x, xq, y, n, k, m)


def test_prefill_nvfp4_extreme_records(hip):
    """The MFMA GEMM on rows that cycle through all 256 UE4M3 scale bytes
    (0x00 and 0x7F read as zero, subnormals, 448) and every code, against
    activations with an all-zero Q8_0 block and an all-zero token."""
    n, k, m = 128, 4096, 40
    recs = extreme_records()                  # 64 records = one row of K = 4096
    w = np.stack([np.roll(recs, 5 * r, axis=0) for r in range(n)]).reshape(n, -1)
    x = acts(m, k, seed=9).copy()
    x[4, 64:96] = 0.0
    x[7] = 0.0
    w, x, xq, y = run_mul_mat(hip, "production_mul_mat_nvfp4", "nvfp4", n, k, m, w=w, x=x)
    check_mul_mat("nvfp4", w, x, xq, y, n, k, m)
