"""IQ2_XS (an adjacent GGML format, ggml-common.h:377-383, grid :617-746)
through the C ABI on the GPU, against the pinned oracle: row dequantize
bit-exact, vec_dot and mul_mat within the fp64 re-accumulation bar, the Xq
workspace bit-exact Q8_K.  Weights are random records with a moderate fp16
d (every byte pattern is a valid record, so every grid and sign index
occurs), records with both scale nibbles at 0 and 15 and d = 0, corner
records (grid and sign indices at 0 and at their maxima, subnormal and
large d) for the MFMA GEMM and the batch-1 kernel, and records from GGML's
own quantize_iq2_xs as restated in oracle/."""
from __future__ import annotations

import functools

import numpy as np
import pytest

import oracle as o
from tests.test_gpu_parity import SENTINEL, acts, assert_close, check_mul_mat, run_mul_mat

pytestmark = pytest.mark.gpu


def weights(n, k, seed=1):
    w = o.random_records("iq2_xs", n, k, seed=seed).reshape(n, k // 256, 74)
    w[0::7, :, 66:74] = 0x00   # every scale nibble 0 (ls = 1)
    w[1::7, :, 66:74] = 0xFF   # every scale nibble 15 (ls = 31)
    w[2::11, 0, 0:2] = 0       # d = 0
    return w.reshape(n, -1)


def tables(hip):
    return [hip.grid_xs_i8x8, hip.signs_i8x8]


@pytest.mark.parametrize("n,k,w_off,y_off", [(64, 4096, 0, 0), (33, 768, 2, 1), (7, 256, 6, 2)])
def test_dequant_iq2_xs(hip, n, k, w_off, y_off):
    w = weights(n, k)
    total = n * k
    y = hip.empty(4 * total, fill=SENTINEL, offset=4 * y_off)
    hip.call("row_dequantize_iq2_xs", hip.to_dev(w, offset=w_off), *tables(hip), y, total)
    want = o.dequantize("iq2_xs", w, k).reshape(-1)
    np.testing.assert_array_equal(y.numpy(np.float32).view(np.uint32), want.view(np.uint32))


def test_vec_dot_iq2_xs(hip):
    for k in (256, 4096, 14336):
        w = weights(1, k, seed=3)
        x = acts(1, k, seed=4)
        x[0, 256:512] = 0.0  # an all-zero Q8_K block
        xq = o.quantize("q8_k", x)
        y = hip.empty(4, fill=SENTINEL)
        hip.call("quantized_vec_dot_iq2_xs_q8_k", hip.to_dev(w), hip.to_dev(xq), *tables(hip), y, k)
        e, a = o.mul_mat_f64("iq2_xs", w, xq, 1, k, 1)
        assert_close(y.numpy(np.float32).reshape(1, 1), e, a, f"vec_dot iq2_xs K={k}")


@pytest.mark.parametrize("symbol", ["production_mul_mat_iq2_xs", "production_mul_mat_iq2_xs_staged"])
@pytest.mark.parametrize("n,k,m", [(4096, 4096, 1), (4096, 14336, 1), (300, 768, 3), (65, 1024, 5),
                                   (1, 256, 1), (1, 512, 1), (17, 1024, 1), (5000, 2048, 1),
                                   (512, 4096, 64), (200, 1536, 70), (129, 1024, 17), (4096, 4096, 512)])
def test_mul_mat_iq2_xs(hip, symbol, n, k, m):
    """M >= 16 with K a multiple of 512 runs the MFMA GEMM (the IQ2 GEMM with
    per-16 scales), M = 1 with K <= 4096 a multiple of 512 the batch-1
    kernel, every other shape the staged GEMV."""
    w = weights(n, k)
    w, x, xq, y = run_mul_mat(hip, symbol, "iq2_xs", n, k, m, w=w)
    check_mul_mat("iq2_xs", w, x, xq, y, n, k, m)


@pytest.mark.parametrize("symbol", ["production_mul_mat_iq2_xs", "production_mul_mat_iq2_xs_staged"])
@pytest.mark.parametrize("n,k,m", [(4096, 4096, 1), (4096, 4096, 512), (300, 1536, 70)])
def test_mul_mat_iq2_xs_ggml_quantized(hip, symbol, n, k, m):
    """Records from GGML's own quantize_iq2_xs (unit importance) of N(0, 0.02)
    rows, through the batch-1 kernel, the MFMA GEMM and the staged GEMV."""
    w = ggml_weights(n, k)
    w, x, xq, y = run_mul_mat(hip, symbol, "iq2_xs", n, k, m, w=w)
    check_mul_mat("iq2_xs", w, x, xq, y, n, k, m)


@functools.lru_cache(maxsize=None)
def ggml_weights(n, k, seed=5):
    return o.quantize_ggml_iq2("iq2_xs", o.seeded_normal(seed, (n, k), 0.02))


def test_ggml_mul_mat_iq2_xs(hip):
    from weft_amd import ggml as G
    n, k, m = 256, 1024, 9
    w = weights(n, k)
    x = acts(m, k)
    wd, xd = hip.to_dev(w), hip.to_dev(x)
    yd = hip.empty(4 * m * n, fill=SENTINEL)
    s0 = G.tensor(G.IQ2_XS, (k, n), wd.ptr)
    s1 = G.tensor(G.F32, (k, m), xd.ptr)
    wsize = G.mul_mat_work_size(s0, s1)
    wdata = hip.empty(wsize, fill=SENTINEL)
    G.mul_mat(s0, s1, G.tensor(G.F32, (n, m), yd.ptr), wdata.ptr, wsize)
    hip.torch.cuda.synchronize()
    assert hip.last_error() == 0
    xq = o.quantize("q8_k", x)
    e, a = o.mul_mat_f64("iq2_xs", w, xq, n, k, m)
    assert_close(yd.numpy(np.float32).reshape(m, n), e, a, "MUL_MAT iq2_xs")


def extreme_weights(n, k, seed=23):
    """Records at the format's corners: every grid index and sign index at
    0 and at its maximum (qs = 0x0000 / 0xFFFF: grid entry 511, sign entry
    127), both scale nibbles 0 and 15, d = 0, the smallest subnormal d and
    d = 2^15, mixed with random records."""
    w = weights(n, k, seed=seed).reshape(n, k // 256, 74)
    rng = np.random.default_rng(seed)
    d = (rng.standard_normal((n, k // 256)) * 1e-2).astype(np.float16)
    w[:, :, 0:2] = d.view(np.uint8).reshape(n, k // 256, 2)
    w[3, :, 2:66] = 0x00                        # grid 0, sign 0 everywhere
    w[4, :, 2:66] = 0xFF                        # grid 511, sign 127 everywhere
    w[4, :, 66:74] = 0xFF
    w[5, 1, 0:2] = 0                            # d = 0
    w[6, :, 0:2] = np.array([1, 0], np.uint8)   # smallest subnormal d
    w[7, :, 0:2] = np.array([2.0 ** 15], np.float16).view(np.uint8)
    return np.ascontiguousarray(w.reshape(n, -1))


def test_prefill_iq2_xs_extreme_records(hip):
    """The MFMA GEMM (per-16 scales, sign masks from LDS, the dx dw factor
    from a bf16 outer-product MFMA) on corner records, against activations
    with an all-zero Q8_K block and an all-zero token."""
    n, k, m = 160, 2048, 48
    w = extreme_weights(n, k)
    x = acts(m, k, seed=9).copy()
    x[4, 256:512] = 0.0
    x[7] = 0.0
    w, x, xq, y = run_mul_mat(hip, "production_mul_mat_iq2_xs", "iq2_xs", n, k, m, w=w, x=x)
    check_mul_mat("iq2_xs", w, x, xq, y, n, k, m)


def test_decode_iq2_xs_batch1_extreme_records(hip):
    """The batch-1 kernel on the same corner records, against an activation
    with an all-zero Q8_K block."""
    n, k = 160, 4096
    w = extreme_weights(n, k, seed=29)
    x = acts(1, k, seed=17).copy()
    x[0, 256:512] = 0.0
    w, x, xq, y = run_mul_mat(hip, "production_mul_mat_iq2_xs", "iq2_xs", n, k, 1, w=w, x=x)
    check_mul_mat("iq2_xs", w, x, xq, y, n, k, 1)
