"""Parity of libweft_hip against the CPU oracle, through the C ABI (GPU).

Bars (declared before any run):
  * row dequantize, Q8_0/Q8_K quantize, the Xq workspace: bit-exact, byte
    for byte, including bytes GGML leaves untouched (buffers start from the
    same sentinel fill on both sides);
  * fp32 outputs of vec_dot / mul_mat: |y - E| <= 1e-4 |E| + 4e-6 A, where E
    is the fp64 re-accumulation of the exact integer partials of the same
    quantized operands and A = sum |scale * partial| over the format's scale
    groups (oracle.within_tolerance).
Shapes are BASELINE.json's configs where the oracle finishes in seconds;
the prefill N=11008 case checks a seeded sample of output columns.
"""
from __future__ import annotations

import functools

import numpy as np
import pytest

import oracle as o

pytestmark = pytest.mark.gpu

SENTINEL = 0xA5


@functools.lru_cache(maxsize=None)
def weights(fmt: str, n: int, k: int, seed: int = 1) -> np.ndarray:
    """GGML-quantized N(0, 0.02) rows; IQ2_XXS by GGML's own quantize_iq2_xxs
    with unit importance, as the reference's repro builds its records
    (examples/repro/weft/mul_mat_runtime.cpp:762-776)."""
    w = o.seeded_normal(seed, (n, k), 0.02)
    return o.quantize_ggml_iq2(fmt, w) if fmt == "iq2_xxs" else o.quantize(fmt, w)


@functools.lru_cache(maxsize=None)
def acts(m: int, k: int, seed: int = 2) -> np.ndarray:
    return o.seeded_normal(seed, (m, k), 1.0)


def tables(hip, fmt):
    if fmt == "iq2_xxs":
        return [hip.grid_i8x8, hip.signs_i8x8]
    if fmt == "iq2_xs":
        return [hip.grid_xs_i8x8, hip.signs_i8x8]
    if fmt == "mxfp4":
        return [hip.codebook, hip.scale]
    if fmt == "nvfp4":
        return [hip.codebook, hip.ue4m3]
    return []


def assert_close(y, e, a, what):
    ok = o.within_tolerance(y, e, a)
    if not ok.all():
        bad = np.argwhere(~ok)[:5]
        rows = [(tuple(i), float(np.asarray(y)[tuple(i)]), float(e[tuple(i)]), float(a[tuple(i)]))
                for i in bad]
        raise AssertionError(f"{what}: {int((~ok).sum())} outputs outside tolerance, e.g. {rows}")


# ------------------------------------------------------------ row dequantize
DQ_SYMBOL = {"q4_0": "row_dequantize_q4_0", "q4_k": "row_dequantize_q4_k",
             "iq2_xxs": "row_dequantize_iq2_xxs", "mxfp4": "row_dequantize_mxfp4"}
DQ_TABLES = {"iq2_xxs": "iq2", "mxfp4": "mx"}


def _dequant_case(hip, fmt, n, k, w_off=0, y_off=0):
    w = weights(fmt, n, k)
    total = n * k
    wd = hip.to_dev(w, offset=w_offset_bytes(fmt, w_off))
    y = hip.empty(4 * total, fill=SENTINEL, offset=4 * y_off)
    extra = []
    if fmt == "iq2_xxs":
        extra = [hip.grid_i8x8, hip.signs_i8x8]
    elif fmt == "mxfp4":
        extra = [hip.codebook, hip.scale]
    hip.call(DQ_SYMBOL[fmt], wd, *extra, y, total)
    got = y.numpy(np.float32)
    want = o.dequantize(fmt, w, k).reshape(-1)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def w_offset_bytes(fmt, units):
    align = {"q4_0": 2, "q4_k": 2, "iq2_xxs": 2, "mxfp4": 1}[fmt]
    return units * align


def test_dequant_q4_k_config2(hip):
    """Q4_K row dequantize 11008x4096, bit-exact."""
    _dequant_case(hip, "q4_k", 11008, 4096)


@pytest.mark.parametrize("fmt", ["q4_0", "q4_k", "iq2_xxs", "mxfp4"])
@pytest.mark.parametrize("n,k", [(512, 4096), (1, 256), (37, 256)])
def test_dequant_bit_exact(hip, fmt, n, k):
    _dequant_case(hip, fmt, n, k)


@pytest.mark.parametrize("fmt", ["q4_0", "q4_k", "iq2_xxs", "mxfp4"])
def test_dequant_misaligned_pointers(hip, fmt):
    # base pointers that only meet the Encoding's own alignment
    _dequant_case(hip, fmt, 19, 512, w_off=1, y_off=1)


@pytest.mark.parametrize("fmt", ["q4_0", "q4_1", "q4_k", "q5_k", "q6_k", "mxfp4", "nvfp4"])
@pytest.mark.parametrize("n,k", [(40, 1024), (2050, 4096)])
def test_dequant_staged_chunks(hip, fmt, n, k):
    """The LDS-staged path (16-byte direct loads of 64-superblock chunks):
    a weight base 4 bytes past a 16-byte boundary, a partial last chunk
    (2.5 chunks; 512.5 chunks, more than one grid's worth, so one block
    takes a second chunk), every output written and bit-exact."""
    w = weights(fmt, n, k)
    total = n * k
    assert (w.nbytes % 16) == 0 and (total // 256) % 64 != 0
    y = hip.empty(4 * total, fill=SENTINEL)
    hip.call("row_dequantize_" + fmt, hip.to_dev(w, offset=4), *tables(hip, fmt), y, total)
    want = o.dequantize(fmt, w, k).reshape(-1)
    np.testing.assert_array_equal(y.numpy(np.float32).view(np.uint32), want.view(np.uint32))


# ---------------------------------------------------------------- quantize
def edge_rows(k: int) -> np.ndarray:
    """Known-hard blocks: exact .5 ties, all-zero, +-equal max, denormals,
    values hitting +-127, one huge outlier, negative-first maximum."""
    rows = []
    # every 32-block starts with 127, so d = 1 exactly and x.5 values tie
    r = ((np.arange(k) % 64) - 31.5).astype(np.float32)
    r[0::32] = 127.0
    rows.append(r)
    rows.append(np.zeros(k, np.float32))
    r = np.zeros(k, np.float32)
    r[3], r[7] = 5.0, -5.0
    r[300], r[301] = -5.0, 5.0
    rows.append(r)
    # tiny but normal magnitudes (fp16(d) underflows to 0; 1/d stays finite)
    rows.append(np.full(k, 1e-30, np.float32) * np.where(np.arange(k) % 2, 1, -1))
    r = np.linspace(-1.0, 1.0, k, dtype=np.float32)
    r[17] = 1e30
    rows.append(r)
    r = o.seeded_normal(9, (k,))
    r[::32] = 0
    r[0] = -3e-5
    rows.append(r)
    return np.stack(rows).astype(np.float32)


@pytest.mark.parametrize("act", ["q8_0", "q8_k"])
def test_quantize_bit_exact(hip, act):
    k = 4096
    x = np.concatenate([acts(512, k), edge_rows(k)])
    nbytes = o.record_bytes(act, k) * x.shape[0]
    xd = hip.to_dev(x)
    y = hip.empty(nbytes, fill=SENTINEL)
    hip.call("q8_0_quantize" if act == "q8_0" else "q8_K_quantize", xd, y, x.size)
    want = np.full((x.shape[0], o.record_bytes(act, k)), SENTINEL, np.uint8)
    o.quantize(act, x, out=want)
    np.testing.assert_array_equal(y.numpy(np.uint8), want.reshape(-1))


@pytest.mark.parametrize("act", ["q8_0", "q8_k"])
def test_quantize_misaligned(hip, act):
    k = 512
    x = acts(7, k)
    xd = hip.to_dev(x, offset=4)
    nbytes = o.record_bytes(act, k) * 7
    y = hip.empty(nbytes, fill=SENTINEL, offset=2 if act == "q8_0" else 4)
    hip.call("q8_0_quantize" if act == "q8_0" else "q8_K_quantize", xd, y, x.size)
    want = np.full((7, o.record_bytes(act, k)), SENTINEL, np.uint8)
    o.quantize(act, x, out=want)
    np.testing.assert_array_equal(y.numpy(np.uint8), want.reshape(-1))


# ---------------------------------------------------------------- vec_dot
VD_SYMBOL = {"q4_0": "quantized_vec_dot_q4_0_q8_0", "q4_k": "quantized_vec_dot_q4_k_q8_k",
             "iq2_xxs": "quantized_vec_dot_iq2_xxs_q8_k", "mxfp4": "quantized_vec_dot_mxfp4_q8_0"}


@pytest.mark.parametrize("fmt", ["q4_0", "q4_k", "iq2_xxs", "mxfp4"])
@pytest.mark.parametrize("k", [256, 4096, 14336])
def test_vec_dot(hip, fmt, k):
    w = weights(fmt, 1, k, seed=3)
    xq = o.quantize(o.ACT_OF[fmt], acts(1, k, seed=4))
    y = hip.empty(4, fill=SENTINEL)
    hip.call(VD_SYMBOL[fmt], hip.to_dev(w), hip.to_dev(xq), *tables(hip, fmt), y, k)
    e, a = o.mul_mat_f64(fmt, w, xq, 1, k, 1)
    assert_close(y.numpy(np.float32).reshape(1, 1), e, a, f"vec_dot {fmt}")


# ------------------------------------------------------------ decode GEMV
MM_DECODE = {"q4_0": "production_mul_mat_q4_0_decode", "q4_k": "production_mul_mat_q4_k_decode",
             "iq2_xxs": "production_mul_mat_iq2_xxs_decode", "mxfp4": "production_mul_mat_mxfp4_decode"}
MM_PREFILL = {"q4_0": "production_mul_mat_q4_0", "q4_k": "production_mul_mat_q4_k_staged",
              "iq2_xxs": "production_mul_mat_iq2_xxs_staged", "mxfp4": "production_mul_mat_mxfp4"}


def run_mul_mat(hip, symbol, fmt, n, k, m, w=None, x=None):
    w = weights(fmt, n, k) if w is None else w
    x = acts(m, k) if x is None else x
    act = o.ACT_OF[fmt]
    xq = hip.empty(o.record_bytes(act, k) * m, fill=SENTINEL)
    y = hip.empty(4 * m * n, fill=SENTINEL)
    hip.call(symbol, hip.to_dev(w), hip.to_dev(x), xq, *tables(hip, fmt), y, n, k, m)
    return w, x, xq.numpy(np.uint8).reshape(m, -1), y.numpy(np.float32).reshape(m, n)


def check_mul_mat(fmt, w, x, xq_got, y_got, n, k, m, cols=None):
    act = o.ACT_OF[fmt]
    want_xq = np.full((m, o.record_bytes(act, k)), SENTINEL, np.uint8)
    o.quantize(act, x, out=want_xq)
    np.testing.assert_array_equal(xq_got, want_xq, err_msg="Xq workspace differs")
    if cols is not None:
        w = w[cols]
        y_got = y_got[:, cols]
        n = len(cols)
    e, a = o.mul_mat_f64(fmt, w, want_xq, n, k, m)
    assert_close(y_got, e, a, f"mul_mat {fmt}")


@pytest.mark.parametrize("fmt,n,k", [
    ("q4_0", 4096, 4096),       # config 1
    ("q4_k", 11008, 4096),      # config 3, W_up
    ("q4_k", 4096, 11008),      # config 3, W_down
    ("iq2_xxs", 4096, 4096),    # config 5a
    ("mxfp4", 4096, 4096),
])
def test_decode_configs(hip, fmt, n, k):
    w, x, xq, y = run_mul_mat(hip, MM_DECODE[fmt], fmt, n, k, 1)
    check_mul_mat(fmt, w, x, xq, y, n, k, 1)


@pytest.mark.parametrize("n,k", [(300, 8192), (5000, 8192), (4100, 12288), (17, 11008)])
def test_decode_q4_k_long_rows(hip, n, k):
    # batch-1 Q4_K launch shapes: two and three 4096-column steps per row,
    # with one row per wave (N <= 16 per CU) and with two row buffers
    w, x, xq, y = run_mul_mat(hip, MM_DECODE["q4_k"], "q4_k", n, k, 1)
    check_mul_mat("q4_k", w, x, xq, y, n, k, 1)


@pytest.mark.parametrize("fmt", ["q4_0", "q4_k", "iq2_xxs", "mxfp4"])
@pytest.mark.parametrize("n,k,m", [(300, 768, 3), (65, 1024, 5), (1, 256, 1)])
def test_decode_small_shapes(hip, fmt, n, k, m):
    w, x, xq, y = run_mul_mat(hip, MM_DECODE[fmt], fmt, n, k, m)
    check_mul_mat(fmt, w, x, xq, y, n, k, m)


@pytest.mark.parametrize("fmt", ["q4_0", "q4_k", "iq2_xxs", "mxfp4"])
@pytest.mark.parametrize("m", [1, 3, 64])
def test_long_rows(hip, fmt, m):
    """K = 65536: the batch-1 and small-batch GEMVs stage the whole quantized
    activation row in LDS (about 72 KB), the prefill GEMMs stream it by
    superblock pairs."""
    n, k = 96, 65536
    w, x, xq, y = run_mul_mat(hip, MM_PREFILL[fmt] if m >= 16 else MM_DECODE[fmt], fmt, n, k, m)
    check_mul_mat(fmt, w, x, xq, y, n, k, m)


MM_ANY = {"q4_0": "production_mul_mat_q4_0", "q4_1": "production_mul_mat_q4_1",
          "mxfp4": "production_mul_mat_mxfp4", "nvfp4": "production_mul_mat_nvfp4",
          "q4_k": "production_mul_mat_q4_k_staged", "q5_k": "production_mul_mat_q5_k",
          "q6_k": "production_mul_mat_q6_k", "iq2_xxs": "production_mul_mat_iq2_xxs_staged",
          "iq2_xs": "production_mul_mat_iq2_xs_staged"}


def launch_log(hip):
    import ctypes
    buf = ctypes.create_string_buffer(4096)
    hip.lib.weft_hip_launch_log(buf, len(buf))
    return buf.value.decode()


@pytest.mark.parametrize("fmt", list(MM_ANY))
@pytest.mark.parametrize("m", [1, 3])
def test_long_row_small_batch_takes_the_gemm(hip, fmt, m):
    """K = 2^18 (a quantized activation row of ~300 KB, past a workgroup's
    LDS) below 16 activation rows: the mul_mat entry points run the
    format's prefill GEMM, which streams K, instead of the GEMVs that keep
    the row in LDS; every output against the oracle."""
    n, k = 8, 1 << 18
    x = o.seeded_normal(31, (m, k))
    w = (o.random_records(fmt, n, k, seed=32) if fmt.startswith("iq2")
         else o.quantize(fmt, o.seeded_normal(32, (n, k), 0.02)))
    was = hip.lib.weft_hip_set_launch_log(1)
    try:
        launch_log(hip)  # drop earlier names
        w_, x_, xq, y = run_mul_mat(hip, MM_ANY[fmt], fmt, n, k, m, w=w, x=x)
        names = launch_log(hip)
    finally:
        hip.lib.weft_hip_set_launch_log(was)
    assert "gemm" in names and "gemv" not in names, names
    check_mul_mat(fmt, w_, x_, xq, y, n, k, m)


@pytest.mark.parametrize("fmt", [f for f in MM_ANY if f != "iq2_xs"])  # IQ2_XS has no _decode entry
def test_long_row_decode_entry_takes_the_gemm(hip, fmt):
    """The batch-1 decode entry points with a row past the GEMV's LDS
    (K = 2^18) run the format's GEMM too."""
    n, k, m = 8, 1 << 18, 1
    x = o.seeded_normal(33, (m, k))
    w = (o.random_records(fmt, n, k, seed=34) if fmt.startswith("iq2")
         else o.quantize(fmt, o.seeded_normal(34, (n, k), 0.02)))
    was = hip.lib.weft_hip_set_launch_log(1)
    try:
        launch_log(hip)
        w_, x_, xq, y = run_mul_mat(hip, f"production_mul_mat_{fmt}_decode", fmt, n, k, m, w=w, x=x)
        names = launch_log(hip)
    finally:
        hip.lib.weft_hip_set_launch_log(was)
    assert "gemm" in names and "gemv" not in names, names
    check_mul_mat(fmt, w_, x_, xq, y, n, k, m)


VD_ANY = {"q4_0": "q8_0", "q4_1": "q8_1", "mxfp4": "q8_0", "nvfp4": "q8_0", "q4_k": "q8_k",
          "q5_k": "q8_k", "q6_k": "q8_k", "iq2_xxs": "q8_k", "iq2_xs": "q8_k"}


@pytest.mark.parametrize("fmt", list(VD_ANY))
def test_long_row_vec_dot(hip, fmt):
    """quantized_vec_dot_* with K = 2^18, the activation already quantized:
    the staged GEMV walks K in chunks its LDS holds (the first stores Y, the
    rest add), Q4_K takes its GEMM; against the oracle."""
    k = 1 << 18
    w = (o.random_records(fmt, 1, k, seed=35) if fmt.startswith("iq2")
         else o.quantize(fmt, o.seeded_normal(35, (1, k), 0.02)))
    xq = o.quantize(VD_ANY[fmt], o.seeded_normal(36, (1, k)))
    y = hip.empty(4, fill=SENTINEL)
    hip.call(f"quantized_vec_dot_{fmt}_{VD_ANY[fmt]}", hip.to_dev(w), hip.to_dev(xq), *tables(hip, fmt), y, k)
    e, a = o.mul_mat_f64(fmt, w, xq, 1, k, 1)
    assert_close(y.numpy(np.float32).reshape(1, 1), e, a, f"vec_dot {fmt} K=2^18")


@pytest.mark.parametrize("fmt", ["q4_0", "mxfp4", "q4_k"])
@pytest.mark.parametrize("m", [1, 3])
def test_long_row_chunked_gemv(hip, fmt, m):
    """A row past the GEMV's LDS whose weights the GEMM cannot take (a base
    2 bytes past 4-byte alignment; the GEMMs' direct loads need 4): the
    GEMV (the staged one, Q4_K's own) walks K in chunks, one activation row
    at a time; Xq and every output against the oracle."""
    n, k = 8, 1 << 18
    w = o.quantize(fmt, o.seeded_normal(37, (n, k), 0.02))
    x = o.seeded_normal(38, (m, k))
    xq = hip.empty(o.record_bytes(o.ACT_OF[fmt], k) * m, fill=SENTINEL)
    y = hip.empty(4 * m * n, fill=SENTINEL)
    was = hip.lib.weft_hip_set_launch_log(1)
    try:
        launch_log(hip)
        hip.call(MM_DECODE[fmt], hip.to_dev(w, offset=2), hip.to_dev(x), xq, *tables(hip, fmt), y, n, k, m)
        names = launch_log(hip)
    finally:
        hip.lib.weft_hip_set_launch_log(was)
    assert "gemm" not in names and names.count("gemv_kernel") >= 2 * m, names
    check_mul_mat(fmt, w, x, xq.numpy(np.uint8).reshape(m, -1), y.numpy(np.float32).reshape(m, n), n, k, m)


@pytest.mark.parametrize("k,launches", [(76864, 1), (76928, 2)])
def test_staged_row_lds_boundary(hip, k, launches):
    """The staged GEMV's LDS edge for Q4_0 (16 wave windows of 4640 bytes,
    3 KB of tables and a Q8_0 row of 1.125 K bytes in 160 KB): K = 76864 is
    the longest row one pass holds, K = 76928 takes two chunks (76800 +
    128); weights 2 bytes past 4-byte alignment keep the GEMM out.  Both
    against the oracle."""
    fmt, n, m = "q4_0", 8, 1
    w = o.quantize(fmt, o.seeded_normal(39, (n, k), 0.02))
    x = o.seeded_normal(40, (m, k))
    xq = hip.empty(o.record_bytes(o.ACT_OF[fmt], k) * m, fill=SENTINEL)
    y = hip.empty(4 * m * n, fill=SENTINEL)
    was = hip.lib.weft_hip_set_launch_log(1)
    try:
        launch_log(hip)
        hip.call(MM_DECODE[fmt], hip.to_dev(w, offset=2), hip.to_dev(x), xq, y, n, k, m)
        names = launch_log(hip)
    finally:
        hip.lib.weft_hip_set_launch_log(was)
    assert names.count("staged_gemv_kernel") == launches, names
    check_mul_mat(fmt, w, x, xq.numpy(np.uint8).reshape(m, -1), y.numpy(np.float32).reshape(m, n), n, k, m)


@pytest.mark.parametrize("fmt", ["q4_0", "q4_k", "iq2_xxs", "mxfp4"])
def test_prefill_entry_points(hip, fmt):
    n, k, m = 512, 4096, 64
    w, x, xq, y = run_mul_mat(hip, MM_PREFILL[fmt], fmt, n, k, m)
    check_mul_mat(fmt, w, x, xq, y, n, k, m)


@pytest.mark.parametrize("fmt", ["q4_k", "q4_0", "mxfp4", "iq2_xxs"])
@pytest.mark.parametrize("n,k,m", [(300, 512, 37), (129, 768, 16), (128, 256, 65), (200, 1536, 70)])
def test_prefill_ragged_tiles(hip, fmt, n, k, m):
    # shapes that leave partial 64 x 128 MFMA tiles on both axes, an odd
    # number of 256-value stages (K = 768) for the stage-parity waves, and an
    # odd number of stage pairs (K = 1536) for the two LDS ring slots; IQ2_XXS
    # at K = 768 / 256 takes the GEMV path (its GEMM stages superblock pairs)
    w, x, xq, y = run_mul_mat(hip, MM_PREFILL[fmt], fmt, n, k, m)
    check_mul_mat(fmt, w, x, xq, y, n, k, m)


@pytest.mark.parametrize("fmt", ["q4_0", "mxfp4", "iq2_xxs"])
def test_prefill_misaligned_weights_fall_back(hip, fmt):
    # W at a 2-byte offset is valid for these records but not for the MFMA
    # path's 4-byte direct loads: the call must take the GEMV path and agree
    n, k, m = 96, 512, 20
    w, x = weights(fmt, n, k), acts(m, k)
    act = o.ACT_OF[fmt]
    xq = hip.empty(o.record_bytes(act, k) * m, fill=SENTINEL)
    y = hip.empty(4 * m * n, fill=SENTINEL)
    hip.call(MM_PREFILL[fmt], hip.to_dev(w, offset=2), hip.to_dev(x), xq, *tables(hip, fmt), y, n, k, m)
    check_mul_mat(fmt, w, x, xq.numpy(np.uint8).reshape(m, -1), y.numpy(np.float32).reshape(m, n), n, k, m)


def test_prefill_q4_k_config4_n4096(hip):
    """BASELINE config 4 (N=4096): 512 tokens x 4096, full check."""
    n = k = 4096
    m = 512
    w, x, xq, y = run_mul_mat(hip, "production_mul_mat_q4_k_staged", "q4_k", n, k, m)
    check_mul_mat("q4_k", w, x, xq, y, n, k, m)


def test_prefill_q4_k_config4_n11008(hip):
    """BASELINE config 4 (N=11008): 512 tokens x 11008, every output."""
    n, k, m = 11008, 4096, 512
    w, x, xq, y = run_mul_mat(hip, "production_mul_mat_q4_k_staged", "q4_k", n, k, m)
    check_mul_mat("q4_k", w, x, xq, y, n, k, m)


@pytest.mark.parametrize("n,k,m", [(32900, 768, 70), (16500, 1536, 130)])
def test_prefill_q4_k_several_tiles_per_workgroup(hip, n, k, m):
    # more 64 x 128 tiles than a launch has workgroups (one per CU), so each
    # workgroup walks several: partial last token and weight tiles, an odd
    # superblock count (K = 768) and an odd pair count (K = 1536) across the
    # tile boundaries of the ring
    w, x, xq, y = run_mul_mat(hip, "production_mul_mat_q4_k_staged", "q4_k", n, k, m)
    check_mul_mat("q4_k", w, x, xq, y, n, k, m)


@pytest.mark.parametrize("fmt", ["mxfp4", "q4_0", "iq2_xxs"])
def test_prefill_config5b(hip, fmt):
    """BASELINE config 5b (MXFP4, 512 x 4096 x 4096; Q4_0 and IQ2_XXS at the
    same shape): every output."""
    n = k = 4096
    m = 512
    w, x, xq, y = run_mul_mat(hip, MM_PREFILL[fmt], fmt, n, k, m)
    check_mul_mat(fmt, w, x, xq, y, n, k, m)


@pytest.mark.parametrize("symbol,fmt", [("production_mul_mat_q4_k", "q4_k"),
                                        ("production_mul_mat_iq2_xxs", "iq2_xxs")])
def test_prefill_unstaged_entry_points(hip, symbol, fmt):
    """The reference's unstaged mul_mat symbols (mul_mat/q4_k.py,
    mul_mat/iq2_xxs.py) share the staged kernels; one call each."""
    n, k, m = 384, 2048, 80
    w, x, xq, y = run_mul_mat(hip, symbol, fmt, n, k, m)
    check_mul_mat(fmt, w, x, xq, y, n, k, m)


# ------------------------------------------------ crafted records, prefill
FP16_EDGES = np.array([0x0000, 0x8000, 0x0001, 0x03FF, 0x0400, 0x7BFF, 0xFBFF, 0x3C00, 0x2E66, 0xB1A0],
                      np.uint16)  # zeros, subnormals, smallest normal, +-max, ordinary values


def crafted_q4_k(n, k, rng):
    rec = rng.integers(0, 256, size=(n, k // 256, 144), dtype=np.uint8)
    d = rng.choice(FP16_EDGES, size=(n, k // 256))
    dmin = rng.choice(FP16_EDGES, size=(n, k // 256))
    rec[:, :, 0:2] = d.view(np.uint8).reshape(n, k // 256, 2)
    rec[:, :, 2:4] = dmin.view(np.uint8).reshape(n, k // 256, 2)
    rec[0::7, :, 4:16] = 0xFF  # every sub-block: sc = m = 63
    rec[3::11, :, 16:] = 0xFF  # every nibble 15
    return rec.reshape(n, -1)


def crafted_q4_0(n, k, rng):
    rec = rng.integers(0, 256, size=(n, k // 32, 18), dtype=np.uint8)
    rec[:, :, 0:2] = rng.choice(FP16_EDGES, size=(n, k // 32)).view(np.uint8).reshape(n, k // 32, 2)
    rec[5::9, :, 2:] = 0x00  # q - 8 = -8 everywhere
    return rec.reshape(n, -1)


def crafted_iq2_xxs(n, k, rng):
    rec = rng.integers(0, 256, size=(n, k // 256, 66), dtype=np.uint8)
    rec[:, :, 0:2] = rng.choice(FP16_EDGES, size=(n, k // 256)).view(np.uint8).reshape(n, k // 256, 2)
    words = rec[:, :, 2:].copy().view(np.uint32)  # (n, nsb, 16): pairs of (grid idx, signs | scale << 28)
    words[:, :, 1::2] |= np.uint32(0xF0000000)  # s = 15 in every group ...
    words[2::5, :, 1::2] &= np.uint32(0x0FFFFFFF)  # ... except some rows with s = 0
    rec[:, :, 2:] = words.view(np.uint8).reshape(n, k // 256, 64)
    return rec.reshape(n, -1)


def crafted_acts_q8k(m, k, rng):
    x = o.seeded_normal(int(rng.integers(1 << 30)), (m, k))
    x[:, 256:512] = 0.0            # an all-zero Q8_K block in every row
    x[1, :] = 0.0                  # an all-zero row
    x[2, ::256] = 1e4              # a dominant first element per superblock
    x[3, 7::256] = -127.0          # a negative maximum
    return x


@pytest.mark.parametrize("n,k", [(1, 512), (17, 1024), (300, 2048), (5000, 4096), (4097, 4096)])
def test_decode_iq2_xxs_batch1(hip, n, k):
    """The batch-1 IQ2_XXS kernel (records in VGPRs, K <= 4096 with an even
    superblock count): one row, rows past a wave's share, idle lanes for
    K < 4096, a row count that leaves the last workgroup short; crafted
    records (d at the fp16 edges, s = 15 and s = 0) against activations with
    a zero block."""
    rng = np.random.default_rng(n + k)
    w = crafted_iq2_xxs(n, k, rng)
    x = acts(1, k, seed=13).copy()
    x[0, 256:512] = 0.0
    w, x, xq, y = run_mul_mat(hip, MM_DECODE["iq2_xxs"], "iq2_xxs", n, k, 1, w=w, x=x)
    check_mul_mat("iq2_xxs", w, x, xq, y, n, k, 1)


@pytest.mark.parametrize("fmt,make", [("q4_k", crafted_q4_k), ("q4_0", crafted_q4_0),
                                      ("iq2_xxs", crafted_iq2_xxs)])
def test_prefill_crafted_records(hip, fmt, make):
    """The MFMA prefill GEMMs on records no quantizer emits: d / dmin zero,
    negative zero, subnormal, the smallest normal and +-65504; Q4_K sub-blocks
    with sc = m = 63 and all-15 nibbles; Q4_0 blocks of q - 8 = -8; IQ2_XXS
    groups with scale 15 and 0; activations with all-zero Q8_K blocks and
    rows, a dominant element and a negative maximum."""
    rng = np.random.default_rng(77)
    n, k, m = 256, 1024, 64
    w = make(n, k, rng)
    x = crafted_acts_q8k(m, k, rng)
    print(f"crafted prefill {fmt}", flush=True)
    w, x, xq, y = run_mul_mat(hip, MM_PREFILL[fmt], fmt, n, k, m, w=w, x=x)
    check_mul_mat(fmt, w, x, xq, y, n, k, m)


def test_prefill_mxfp4_crafted_scales(hip):
    """MXFP4 prefill on the block-scaled MFMA with every nibble and a wide
    spread of E8M0 exponents (2..200, whole rows at both ends), not just the
    few a quantizer emits; products stay inside fp32's range."""
    n, k, m = 256, 1024, 64
    rng = np.random.default_rng(21)
    rec = rng.integers(0, 256, size=(n, k // 32, 17), dtype=np.uint8)
    rec[:, :, 0] = rng.integers(2, 201, size=(n, k // 32), dtype=np.uint8)
    rec[0, :, 0] = 200
    rec[1, :, 0] = 2  # 2^-126: the smallest normal block scale
    w = rec.reshape(n, -1)
    x = acts(m, k)
    xq = hip.empty(o.record_bytes("q8_0", k) * m, fill=SENTINEL)
    y = hip.empty(4 * m * n, fill=SENTINEL)
    hip.call("production_mul_mat_mxfp4", hip.to_dev(w), hip.to_dev(x), xq, hip.codebook, hip.scale, y,
             n, k, m)
    check_mul_mat("mxfp4", w, x, xq.numpy(np.uint8).reshape(m, -1), y.numpy(np.float32).reshape(m, n),
                  n, k, m)


@pytest.mark.parametrize("symbol,m", [("production_mul_mat_mxfp4", 64), ("production_mul_mat_mxfp4_decode", 1)])
def test_mxfp4_caller_tables_are_used(hip, symbol, m):
    """A scale table that is not GGML's (every entry doubled) is honoured:
    the prefill takes the table-driven int8-MFMA GEMM and the result is
    exactly twice GGML's."""
    n, k = 256, 1024
    w, x = weights("mxfp4", n, k), acts(m, k)
    with np.errstate(over="ignore"):  # entry 255 (2^127) doubles to inf
        scale2 = hip.to_dev(2.0 * o.e8m0_half_table())
    xq = hip.empty(o.record_bytes("q8_0", k) * m, fill=SENTINEL)
    y = hip.empty(4 * m * n, fill=SENTINEL)
    hip.call(symbol, hip.to_dev(w), hip.to_dev(x), xq, hip.codebook, scale2, y, n, k, m)
    want_xq = np.full((m, o.record_bytes("q8_0", k)), SENTINEL, np.uint8)
    o.quantize("q8_0", x, out=want_xq)
    np.testing.assert_array_equal(xq.numpy(np.uint8).reshape(m, -1), want_xq)
    e, a = o.mul_mat_f64("mxfp4", w, want_xq, n, k, m)
    assert_close(y.numpy(np.float32).reshape(m, n), 2.0 * e, 2.0 * a, "mxfp4 with doubled scale table")


@pytest.mark.parametrize("fmt,symbol,m", [
    ("mxfp4", "production_mul_mat_mxfp4_decode", 1), ("mxfp4", "production_mul_mat_mxfp4", 64),
    ("nvfp4", "production_mul_mat_nvfp4_decode", 1), ("nvfp4", "production_mul_mat_nvfp4", 64)])
def test_fp4_caller_codebook_is_used(hip, fmt, symbol, m):
    """A codebook that is not GGML's (kvalues_mxfp4 negated) is honoured:
    the batch-1 kernels look it up with v_perm instead of converting the
    nibbles as E2M1 codes, the prefill takes its table-driven body, and the
    result is exactly minus GGML's."""
    n, k = 256, 1024
    w, x = weights(fmt, n, k), acts(m, k)
    neg = hip.to_dev((-o.kvalues_mxfp4().astype(np.int16)).astype(np.int8))
    tab = hip.scale if fmt == "mxfp4" else hip.ue4m3
    xq = hip.empty(o.record_bytes("q8_0", k) * m, fill=SENTINEL)
    y = hip.empty(4 * m * n, fill=SENTINEL)
    hip.call(symbol, hip.to_dev(w), hip.to_dev(x), xq, neg, tab, y, n, k, m)
    want_xq = np.full((m, o.record_bytes("q8_0", k)), SENTINEL, np.uint8)
    o.quantize("q8_0", x, out=want_xq)
    np.testing.assert_array_equal(xq.numpy(np.uint8).reshape(m, -1), want_xq)
    e, a = o.mul_mat_f64(fmt, w, want_xq, n, k, m)
    assert_close(y.numpy(np.float32).reshape(m, n), -e, a, f"{fmt} with a negated codebook")


# ------------------------------------------------------------ error paths
def test_invalid_shape_reports_error_and_launches_nothing(hip):
    y = hip.empty(16, fill=SENTINEL)
    w = hip.empty(4096)
    x = hip.empty(4096)
    xq = hip.empty(4096)
    hip.lib.production_mul_mat_q4_k_decode(w.ptr, x.ptr, xq.ptr, y.ptr, 1, 100, 1)
    hip.torch.cuda.synchronize()
    assert hip.last_error() != 0
    assert hip.last_error() == 0  # cleared once read
    assert (y.numpy(np.uint8) == SENTINEL).all()
