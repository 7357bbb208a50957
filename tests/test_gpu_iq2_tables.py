"""IQ2_XXS / IQ2_XS with caller tables other than GGML's, through the C ABI
on the GPU.  The reference's kernels take any I8X8 grid and sign table and
multiply a grid byte by its sign byte as i8 x i8 -> i8
(examples/kernels/vec_dot/iq2_xxs_q8_k.py:8-54, iq2_xs_q8_k.py:9-39); the
library's fast kernels take the signs as byte masks, which needs every sign
byte +-1 and no grid byte 0.  Each kernel checks the tables it stages and
otherwise runs the byte-product body.  Every kernel that takes IQ2 tables
is run with tables outside that precondition -- random int8 grids with 0
and negative bytes and a zero row, signs of 0, 2, -3, 127, -128 -- and with
GGML's tables carrying a single bad byte, against oracle.iq2_tables_mul_mat_f64
(pinned in tests/test_oracle.py), to the bar of the other parity tests."""
from __future__ import annotations

import numpy as np
import pytest

import oracle as o
from tests.test_gpu_parity import SENTINEL, acts, assert_close

pytestmark = pytest.mark.gpu

GRID_ROWS = {"iq2_xxs": 256, "iq2_xs": 512}
DECODE = {"iq2_xxs": "production_mul_mat_iq2_xxs_decode", "iq2_xs": "production_mul_mat_iq2_xs"}
PREFILL = {"iq2_xxs": "production_mul_mat_iq2_xxs_staged", "iq2_xs": "production_mul_mat_iq2_xs_staged"}
VEC_DOT = {"iq2_xxs": "quantized_vec_dot_iq2_xxs_q8_k", "iq2_xs": "quantized_vec_dot_iq2_xs_q8_k"}


def records(fmt, n, k, seed):
    if fmt == "iq2_xs":
        return o.random_records(fmt, n, k, seed=seed)
    return o.quantize(fmt, o.seeded_normal(seed, (n, k), 0.02))


def random_tables(fmt, seed):
    rng = np.random.default_rng(seed)
    grid = rng.integers(-128, 128, size=(GRID_ROWS[fmt], 8)).astype(np.int8)
    grid[0] = 0                         # a row of zeros
    grid[1] = -np.abs(grid[1].astype(np.int16)).clip(-128, 127).astype(np.int8)  # negated magnitudes
    grid[2, :4] = (-128, 127, 1, 0)
    signs = rng.choice(np.array([0, 1, -1, 2, -3, 127, -128], np.int8), size=(128, 8))
    return grid, signs


def ggml_tables(fmt):
    grid = (o.iq2xs_grid() if fmt == "iq2_xs" else o.iq2xxs_grid()).view(np.int8).reshape(-1, 8).copy()
    return grid, o.signs_i8x8().reshape(128, 8).copy()


def table_cases(fmt):
    g, s = ggml_tables(fmt)
    s_two = s.copy()
    s_two[17, 3] = 2                    # one sign byte other than +-1
    g_zero = g.copy()
    g_zero[5, 6] = 0                    # one grid byte 0 (a carry for the masks' negate)
    return {"random": random_tables(fmt, 81), "one_sign_2": (g, s_two), "one_grid_0": (g_zero, s)}


def run(hip, symbol, fmt, grid, signs, n, k, m, seed=83):
    w = records(fmt, n, k, seed)
    x = acts(m, k, seed=seed + 1)
    xq = hip.empty(o.record_bytes("q8_k", k) * m, fill=SENTINEL)
    y = hip.empty(4 * m * n, fill=SENTINEL)
    hip._lib.launch_log()
    hip.call(symbol, hip.to_dev(w), hip.to_dev(x), xq, hip.to_dev(grid), hip.to_dev(signs), y, n, k, m)
    launched = hip._lib.launch_log()
    want_xq = np.full((m, o.record_bytes("q8_k", k)), SENTINEL, np.uint8)
    o.quantize("q8_k", x, out=want_xq)
    np.testing.assert_array_equal(xq.numpy(np.uint8).reshape(m, -1), want_xq, err_msg="Xq differs")
    e, a = o.iq2_tables_mul_mat_f64(fmt, w, want_xq, n, k, m, grid, signs)
    assert_close(y.numpy(np.float32).reshape(m, n), e, a, f"{symbol} {fmt} caller tables")
    return launched


@pytest.mark.parametrize("case", ["random", "one_sign_2", "one_grid_0"])
@pytest.mark.parametrize("fmt", ["iq2_xxs", "iq2_xs"])
@pytest.mark.parametrize("path,n,k,m,kernel", [
    ("decode", 1000, 4096, 1, "iq2_gemv_m1_kernel"),  # batch 1, K <= 4096
    ("decode", 300, 1024, 3, "staged_gemv_kernel"),   # 1 < M < 16
    ("decode", 64, 5120, 1, "staged_gemv_kernel"),    # K > 4096
    ("prefill", 200, 1024, 64, "mfma_gemm"),          # the MFMA GEMM
])
def test_caller_tables(hip, fmt, case, path, n, k, m, kernel):
    grid, signs = table_cases(fmt)[case]
    symbol = (DECODE if path == "decode" else PREFILL)[fmt]
    launched = run(hip, symbol, fmt, grid, signs, n, k, m)
    assert any(kernel in name for name in launched), launched


@pytest.mark.parametrize("fmt", ["iq2_xxs", "iq2_xs"])
def test_vec_dot_caller_tables(hip, fmt):
    grid, signs = random_tables(fmt, 85)
    k = 4096
    w = records(fmt, 1, k, 86)
    xq = o.quantize("q8_k", acts(1, k, seed=87))
    y = hip.empty(4, fill=SENTINEL)
    hip.call(VEC_DOT[fmt], hip.to_dev(w), hip.to_dev(xq), hip.to_dev(grid), hip.to_dev(signs), y, k)
    e, a = o.iq2_tables_mul_mat_f64(fmt, w, xq, 1, k, 1, grid, signs)
    assert_close(y.numpy(np.float32).reshape(1, 1), e, a, f"vec_dot {fmt} caller tables")


@pytest.mark.parametrize("fmt", ["iq2_xxs", "iq2_xs"])
def test_ggml_tables_keep_the_mask_path_result(hip, fmt):
    """GGML's own tables give the same result as the oracle restated for
    caller tables, on every path (they take the mask path)."""
    grid, signs = ggml_tables(fmt)
    for symbol, n, k, m in ((DECODE[fmt], 500, 4096, 1), (PREFILL[fmt], 200, 1024, 64)):
        run(hip, symbol, fmt, grid, signs, n, k, m)
