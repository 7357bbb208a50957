"""Q6_K (an adjacent GGML format, ggml-common.h:349-358) through the C ABI on
the GPU, against the pinned oracle: row dequantize bit-exact (any base
alignment: the Weft encoding declares none), vec_dot and mul_mat within the
fp64 re-accumulation bar, the Xq workspace bit-exact.  Extreme records:
scales -128 / 127, the -32 / 31 codes, d = 0, and a zero activation block."""
from __future__ import annotations

import numpy as np
import pytest

import oracle as o
from tests.test_gpu_parity import SENTINEL, acts, assert_close, check_mul_mat, run_mul_mat, weights

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n,k,w_off,y_off", [(64, 4096, 0, 0), (33, 768, 1, 1), (7, 256, 3, 2)])
def test_dequant_q6_k(hip, n, k, w_off, y_off):
    w = weights("q6_k", n, k)
    total = n * k
    y = hip.empty(4 * total, fill=SENTINEL, offset=4 * y_off)
    hip.call("row_dequantize_q6_k", hip.to_dev(w, offset=w_off), y, total)
    want = o.dequantize("q6_k", w, k).reshape(-1)
    np.testing.assert_array_equal(y.numpy(np.float32).view(np.uint32), want.view(np.uint32))


def extreme_records(n_rec):
    """Records with every code at its extremes and the widest scales."""
    rng = np.random.default_rng(17)
    recs = rng.integers(0, 256, size=(n_rec, 210), dtype=np.uint8)
    recs[0, :192] = 0x00                      # all codes 0 -> q = -32
    recs[1, :192] = 0xFF                      # all codes 63 -> q = 31
    recs[:, 192:208] = rng.choice(np.array([-128, 127, -1, 0, 1], np.int8), size=(n_rec, 16)).view(np.uint8)
    recs[2, 208:210] = 0                      # d = 0
    d = (rng.standard_normal(n_rec) * 1e-3).astype(np.float16).view(np.uint8).reshape(n_rec, 2)
    recs[3:, 208:210] = d[3:]
    return recs


def test_vec_dot_q6_k(hip):
    for k in (256, 4096, 14336):
        w = weights("q6_k", 1, k, seed=3)
        xq = o.quantize("q8_k", acts(1, k, seed=4))
        y = hip.empty(4, fill=SENTINEL)
        hip.call("quantized_vec_dot_q6_k_q8_k", hip.to_dev(w), hip.to_dev(xq), y, k)
        e, a = o.mul_mat_f64("q6_k", w, xq, 1, k, 1)
        assert_close(y.numpy(np.float32).reshape(1, 1), e, a, f"vec_dot q6_k K={k}")


def test_vec_dot_q6_k_extreme_records(hip):
    k = 16 * 256
    w = extreme_records(16).reshape(1, -1)
    x = acts(1, k, seed=8)
    x[0, 512:768] = 0.0                       # an all-zero Q8_K block
    xq = o.quantize("q8_k", x)
    y = hip.empty(4, fill=SENTINEL)
    hip.call("quantized_vec_dot_q6_k_q8_k", hip.to_dev(w), hip.to_dev(xq), y, k)
    e, a = o.mul_mat_f64("q6_k", w, xq, 1, k, 1)
    assert_close(y.numpy(np.float32).reshape(1, 1), e, a, "vec_dot q6_k extremes")


@pytest.mark.parametrize("n,k,m", [(4096, 4096, 1), (11008, 4096, 1), (4096, 14336, 1), (300, 768, 3),
                                   (65, 1024, 5), (1, 256, 1), (1, 512, 1), (17, 1024, 1), (5000, 2048, 1)])
def test_decode_q6_k(hip, n, k, m):
    """M = 1 with K <= 4096 a multiple of 512 runs the batch-1 kernel
    (records in VGPRs, odd superblocks at a 2-byte offset), every other
    shape the staged GEMV."""
    w, x, xq, y = run_mul_mat(hip, "production_mul_mat_q6_k_decode", "q6_k", n, k, m)
    check_mul_mat("q6_k", w, x, xq, y, n, k, m)


def test_decode_q6_k_batch1_extreme_records(hip):
    """The batch-1 kernel on rows of -32 and 31 codes, scales from
    {-128, 127, -1, 0, 1}, d = 0, against an activation with an all-zero
    Q8_K block."""
    n, k = 160, 4096
    rng = np.random.default_rng(31)
    w = extreme_records(n * k // 256).reshape(n, k // 256, 210)
    d = (rng.standard_normal((n, k // 256)) * 1e-2).astype(np.float16)
    w[:, :, 208:210] = d.view(np.uint8).reshape(n, k // 256, 2)
    w[5, :, :192] = 0x00
    w[9, :, :192] = 0xFF
    w[17, 3, 208:210] = 0
    w = np.ascontiguousarray(w.reshape(n, -1))
    x = acts(1, k, seed=17).copy()
    x[0, 256:512] = 0.0
    w, x, xq, y = run_mul_mat(hip, "production_mul_mat_q6_k_decode", "q6_k", n, k, 1, w=w, x=x)
    check_mul_mat("q6_k", w, x, xq, y, n, k, 1)


@pytest.mark.parametrize("n,k,m", [(4096, 4096, 512), (512, 4096, 64), (144, 1024, 70), (129, 2048, 17),
                                   (300, 768, 40), (64, 512, 15)])
def test_prefill_q6_k(hip, n, k, m):
    """M >= 16 with K a multiple of 512 runs the int8-MFMA GEMM (ragged
    weight and token tiles included); K = 768 and M = 15 take the GEMV."""
    w, x, xq, y = run_mul_mat(hip, "production_mul_mat_q6_k", "q6_k", n, k, m)
    check_mul_mat("q6_k", w, x, xq, y, n, k, m)


def test_prefill_q6_k_extreme_records(hip):
    """The MFMA GEMM on whole rows of -32 and 31 codes, scales drawn from
    {-128, 127, -1, 0, 1}, d = 0 and subnormal d, against activations with
    an all-zero Q8_K block and an all-zero token."""
    n, k, m = 160, 2048, 48
    rng = np.random.default_rng(29)
    w = extreme_records(n * k // 256).reshape(n, k // 256, 210)
    d = (rng.standard_normal((n, k // 256)) * 1e-2).astype(np.float16)
    w[:, :, 208:210] = d.view(np.uint8).reshape(n, k // 256, 2)
    w[5, :, :192] = 0x00                      # q = -32 everywhere
    w[9, :, :192] = 0xFF                      # q = 31 everywhere
    w[9, :, 192:208] = np.array(-128, np.int8).view(np.uint8)
    w[17, 3, 208:210] = 0                     # d = 0
    w[18, :, 208:210] = np.array([1, 0], np.uint8)  # smallest subnormal d
    w = np.ascontiguousarray(w.reshape(n, -1))
    x = acts(m, k, seed=9).copy()
    x[4, 256:512] = 0.0
    x[7] = 0.0
    w, x, xq, y = run_mul_mat(hip, "production_mul_mat_q6_k", "q6_k", n, k, m, w=w, x=x)
    check_mul_mat("q6_k", w, x, xq, y, n, k, m)
