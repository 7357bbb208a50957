"""Q5_K (an adjacent GGML format, ggml-common.h:330-345) through the C ABI on
the GPU, against the pinned oracle: row dequantize bit-exact, vec_dot and
mul_mat within the fp64 re-accumulation bar, the Xq workspace bit-exact.
Extreme records: every 5-bit code 0 and 31, the 6-bit scales and mins at 63,
d = 0 with dmin != 0, and a zero activation block."""
from __future__ import annotations

import numpy as np
import pytest

import oracle as o
from tests.test_gpu_parity import SENTINEL, acts, assert_close, check_mul_mat, run_mul_mat, weights

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n,k,w_off,y_off", [(64, 4096, 0, 0), (33, 768, 2, 1), (7, 256, 6, 2)])
def test_dequant_q5_k(hip, n, k, w_off, y_off):
    w = weights("q5_k", n, k)
    total = n * k
    y = hip.empty(4 * total, fill=SENTINEL, offset=4 * y_off)
    hip.call("row_dequantize_q5_k", hip.to_dev(w, offset=w_off), y, total)
    want = o.dequantize("q5_k", w, k).reshape(-1)
    np.testing.assert_array_equal(y.numpy(np.float32).view(np.uint32), want.view(np.uint32))


def extreme_records(n_rec):
    """Random records with the codes, scales and mins pushed to their ends."""
    rng = np.random.default_rng(23)
    recs = rng.integers(0, 256, size=(n_rec, 176), dtype=np.uint8)
    recs[0, 16:176] = 0x00                    # every code 0
    recs[1, 16:176] = 0xFF                    # every code 31
    recs[2, 4:16] = 0xFF                      # scales and mins all 63
    d = (rng.standard_normal((n_rec, 2)) * 1e-3).astype(np.float16).view(np.uint8).reshape(n_rec, 4)
    recs[:, 0:4] = d
    recs[3, 0:2] = 0                          # d = 0, dmin kept
    return recs


def test_dequant_q5_k_extreme_records(hip):
    w = extreme_records(16)
    y = hip.empty(4 * 16 * 256, fill=SENTINEL)
    hip.call("row_dequantize_q5_k", hip.to_dev(w), y, 16 * 256)
    want = o.dequantize("q5_k", w.reshape(1, -1), 16 * 256).reshape(-1)
    np.testing.assert_array_equal(y.numpy(np.float32).view(np.uint32), want.view(np.uint32))


def test_vec_dot_q5_k(hip):
    for k in (256, 4096, 14336):
        w = weights("q5_k", 1, k, seed=3)
        xq = o.quantize("q8_k", acts(1, k, seed=4))
        y = hip.empty(4, fill=SENTINEL)
        hip.call("quantized_vec_dot_q5_k_q8_k", hip.to_dev(w), hip.to_dev(xq), y, k)
        e, a = o.mul_mat_f64("q5_k", w, xq, 1, k, 1)
        assert_close(y.numpy(np.float32).reshape(1, 1), e, a, f"vec_dot q5_k K={k}")


def test_vec_dot_q5_k_extreme_records(hip):
    k = 16 * 256
    w = extreme_records(16).reshape(1, -1)
    x = acts(1, k, seed=8)
    x[0, 512:768] = 0.0                       # an all-zero Q8_K block
    xq = o.quantize("q8_k", x)
    y = hip.empty(4, fill=SENTINEL)
    hip.call("quantized_vec_dot_q5_k_q8_k", hip.to_dev(w), hip.to_dev(xq), y, k)
    e, a = o.mul_mat_f64("q5_k", w, xq, 1, k, 1)
    assert_close(y.numpy(np.float32).reshape(1, 1), e, a, "vec_dot q5_k extremes")


@pytest.mark.parametrize("n,k,m", [(4096, 4096, 1), (11008, 4096, 1), (4096, 14336, 1), (300, 768, 3),
                                   (65, 1024, 5), (1, 256, 1), (17, 1024, 1), (5000, 2048, 1), (33, 768, 1)])
def test_decode_q5_k(hip, n, k, m):
    """M = 1 with K <= 4096 runs the batch-1 kernel (records in VGPRs),
    every other shape the staged GEMV."""
    w, x, xq, y = run_mul_mat(hip, "production_mul_mat_q5_k_decode", "q5_k", n, k, m)
    check_mul_mat("q5_k", w, x, xq, y, n, k, m)


def test_decode_q5_k_batch1_extreme_records(hip):
    """The batch-1 kernel on rows of 0 and 31 codes, scales and mins at 63,
    d = 0 with dmin kept, against an activation with an all-zero Q8_K block."""
    n, k = 160, 4096
    w = extreme_records(n * k // 256).reshape(n, k // 256, 176)
    w[5, :, 16:176] = 0x00
    w[9, :, 16:176] = 0xFF
    w[9, :, 4:16] = 0xFF
    w[17, :, 0:2] = 0
    w = np.ascontiguousarray(w.reshape(n, -1))
    x = acts(1, k, seed=16).copy()
    x[0, 512:768] = 0.0
    w, x, xq, y = run_mul_mat(hip, "production_mul_mat_q5_k_decode", "q5_k", n, k, 1, w=w, x=x)
    check_mul_mat("q5_k", w, x, xq, y, n, k, 1)


@pytest.mark.parametrize("n,k,m", [(4096, 4096, 512), (512, 4096, 64), (144, 1024, 70), (300, 768, 17),
                                   (129, 256, 40), (64, 512, 15)])
def test_prefill_q5_k(hip, n, k, m):
    """M >= 16 runs the int8-MFMA GEMM (odd superblock counts, ragged weight
    and token tiles included); M = 15 takes the GEMV."""
    w, x, xq, y = run_mul_mat(hip, "production_mul_mat_q5_k", "q5_k", n, k, m)
    check_mul_mat("q5_k", w, x, xq, y, n, k, m)


def test_prefill_q5_k_extreme_records(hip):
    """The MFMA GEMM on whole rows of 0 and 31 codes, scales and mins at 63,
    d = 0 with dmin kept, against activations with an all-zero Q8_K block and
    an all-zero token."""
    n, k, m = 160, 2048, 48
    w = extreme_records(n * k // 256).reshape(n, k // 256, 176)
    w[5, :, 16:176] = 0x00
    w[9, :, 16:176] = 0xFF
    w[9, :, 4:16] = 0xFF
    w[17, :, 0:2] = 0
    w[18, 2, 0:4] = 0                         # d = dmin = 0
    w = np.ascontiguousarray(w.reshape(n, -1))
    x = acts(m, k, seed=9).copy()
    x[4, 256:512] = 0.0
    x[7] = 0.0
    w, x, xq, y = run_mul_mat(hip, "production_mul_mat_q5_k", "q5_k", n, k, m, w=w, x=x)
    check_mul_mat("q5_k", w, x, xq, y, n, k, m)
