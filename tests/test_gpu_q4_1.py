"""Q4_1 with its Q8_1 activation (adjacent GGML formats, ggml-common.h:187-194
and :240-249) through the C ABI on the GPU, against the pinned oracle: row
dequantize and q8_1_quantize bit-exact, vec_dot and mul_mat within the fp64
re-accumulation bar (|y - E| <= 1e-4 |E| + 4e-6 A, A counting |m s| too),
the Xq workspace bit-exact Q8_1.  The prefill runs the Q4_0 MFMA GEMM with
each block's m * s term; decode the staged GEMV."""
from __future__ import annotations

import numpy as np
import pytest

import oracle as o
from tests.test_gpu_parity import (FP16_EDGES, SENTINEL, acts, assert_close, check_mul_mat,
                                   crafted_acts_q8k, edge_rows, run_mul_mat, weights)

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n,k,w_off,y_off", [(64, 4096, 0, 0), (33, 768, 2, 1), (7, 32, 6, 2)])
def test_dequant_q4_1(hip, n, k, w_off, y_off):
    w = weights("q4_1", n, k)
    total = n * k
    y = hip.empty(4 * total, fill=SENTINEL, offset=4 * y_off)
    hip.call("row_dequantize_q4_1", hip.to_dev(w, offset=w_off), y, total)
    want = o.dequantize("q4_1", w, k).reshape(-1)
    np.testing.assert_array_equal(y.numpy(np.float32).view(np.uint32), want.view(np.uint32))


def crafted_q4_1(n, k, rng):
    rec = rng.integers(0, 256, size=(n, k // 32, 20), dtype=np.uint8)
    rec[:, :, 0:2] = rng.choice(FP16_EDGES, size=(n, k // 32)).view(np.uint8).reshape(n, k // 32, 2)
    rec[:, :, 2:4] = rng.choice(FP16_EDGES, size=(n, k // 32)).view(np.uint8).reshape(n, k // 32, 2)
    rec[5::9, :, 4:] = 0x00  # every code 0: only m contributes
    rec[6::9, :, 4:] = 0xFF  # every code 15
    return rec.reshape(n, -1)


def test_dequant_q4_1_crafted_records(hip):
    w = crafted_q4_1(16, 1024, np.random.default_rng(5))
    y = hip.empty(4 * 16 * 1024, fill=SENTINEL)
    hip.call("row_dequantize_q4_1", hip.to_dev(w), y, 16 * 1024)
    want = o.dequantize("q4_1", w, 1024).reshape(-1)
    np.testing.assert_array_equal(y.numpy(np.float32).view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("k,x_off", [(4096, 0), (2048, 1), (32, 0)])
def test_q8_1_quantize(hip, k, x_off):
    x = edge_rows(k)[0] if k >= 256 else acts(1, k, seed=9)[0]
    y = hip.empty(o.record_bytes("q8_1", k), fill=SENTINEL)
    hip.call("q8_1_quantize", hip.to_dev(x, offset=4 * x_off), y, k)
    np.testing.assert_array_equal(y.numpy(np.uint8), o.quantize("q8_1", x))


def test_q8_1_quantize_zero_and_extremes(hip):
    k = 256
    x = np.zeros(k, np.float32)
    x[32:64] = 1e30                         # d overflows fp16: inf scale
    x[64:96] = np.linspace(-1e-7, 1e-7, 32)  # subnormal fp16 d
    x[96:128] = [0.5 * (i - 16) for i in range(32)]  # .5 ties
    y = hip.empty(o.record_bytes("q8_1", k), fill=SENTINEL)
    hip.call("q8_1_quantize", hip.to_dev(x), y, k)
    np.testing.assert_array_equal(y.numpy(np.uint8), o.quantize("q8_1", x))


def test_vec_dot_q4_1(hip):
    for k in (32, 4096, 14336):
        w = weights("q4_1", 1, k, seed=3)
        xq = o.quantize("q8_1", acts(1, k, seed=4))
        y = hip.empty(4, fill=SENTINEL)
        hip.call("quantized_vec_dot_q4_1_q8_1", hip.to_dev(w), hip.to_dev(xq), y, k)
        e, a = o.mul_mat_f64("q4_1", w, xq, 1, k, 1)
        assert_close(y.numpy(np.float32).reshape(1, 1), e, a, f"vec_dot q4_1 K={k}")


@pytest.mark.parametrize("n,k,m", [(4096, 4096, 1), (11008, 4096, 1), (4096, 14336, 1), (300, 768, 3),
                                   (65, 1024, 5), (1, 32, 1), (1, 64, 1), (17, 1024, 1), (5000, 2048, 1)])
def test_decode_q4_1(hip, n, k, m):
    """M = 1 with K <= 4096 a multiple of 64 runs the batch-1 kernel (records
    in VGPRs), every other shape the staged GEMV."""
    w, x, xq, y = run_mul_mat(hip, "production_mul_mat_q4_1_decode", "q4_1", n, k, m)
    check_mul_mat("q4_1", w, x, xq, y, n, k, m)


def test_decode_q4_1_batch1_crafted_records(hip):
    rng = np.random.default_rng(81)
    n, k = 300, 4096
    w = crafted_q4_1(n, k, rng)
    x = acts(1, k, seed=14).copy()
    x[0, 64:96] = 0.0  # an all-zero Q8_1 block (d = s = 0)
    w, x, xq, y = run_mul_mat(hip, "production_mul_mat_q4_1_decode", "q4_1", n, k, 1, w=w, x=x)
    check_mul_mat("q4_1", w, x, xq, y, n, k, 1)


@pytest.mark.parametrize("n,k,m", [(4096, 4096, 512), (300, 512, 37), (129, 768, 16), (200, 1536, 70),
                                   (64, 4096, 8)])
def test_prefill_q4_1(hip, n, k, m):
    """M >= 16 and K % 256 == 0 run the MFMA GEMM; (64, 4096, 8) the GEMV."""
    w, x, xq, y = run_mul_mat(hip, "production_mul_mat_q4_1", "q4_1", n, k, m)
    check_mul_mat("q4_1", w, x, xq, y, n, k, m)


def test_prefill_q4_1_crafted_records(hip):
    rng = np.random.default_rng(79)
    n, k, m = 256, 1024, 64
    w = crafted_q4_1(n, k, rng)
    x = crafted_acts_q8k(m, k, rng)
    w, x, xq, y = run_mul_mat(hip, "production_mul_mat_q4_1", "q4_1", n, k, m, w=w, x=x)
    check_mul_mat("q4_1", w, x, xq, y, n, k, m)


def test_ggml_mul_mat_q4_1(hip):
    """GGML MUL_MAT with a Q4_1 src0: F32 src1 (quantized into the work
    buffer as Q8_1) and an already quantized Q8_1 src1."""
    from weft_amd import ggml as G
    n, k, m = 256, 1024, 40
    w = weights("q4_1", n, k)
    x = acts(m, k)
    wd, xd = hip.to_dev(w), hip.to_dev(x)
    yd = hip.empty(4 * m * n, fill=SENTINEL)
    s0 = G.tensor(G.Q4_1, (k, n), wd.ptr)
    s1 = G.tensor(G.F32, (k, m), xd.ptr)
    d = G.tensor(G.F32, (n, m), yd.ptr)
    wsize = G.mul_mat_work_size(s0, s1)
    assert wsize == o.record_bytes("q8_1", k) * m
    wdata = hip.empty(wsize, fill=SENTINEL)
    G.mul_mat(s0, s1, d, wdata.ptr, wsize)
    hip.torch.cuda.synchronize()
    assert hip.last_error() == 0
    xq = o.quantize("q8_1", x)
    e, a = o.mul_mat_f64("q4_1", w, xq, n, k, m)
    assert_close(yd.numpy(np.float32).reshape(m, n), e, a, "MUL_MAT q4_1 f32 src1")
    xqd = hip.to_dev(xq)
    yd2 = hip.empty(4 * m * n, fill=SENTINEL)
    G.mul_mat(s0, G.tensor(G.Q8_1, (k, m), xqd.ptr), G.tensor(G.F32, (n, m), yd2.ptr))
    hip.torch.cuda.synchronize()
    assert hip.last_error() == 0
    assert_close(yd2.numpy(np.float32).reshape(m, n), e, a, "MUL_MAT q4_1 q8_1 src1")
