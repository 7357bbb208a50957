"""GGML MUL_MAT through libweft_hip's weft_ggml_mul_mat on the GPU, against the
oracle's GGML MUL_MAT (ggml-cpu/ggml-cpu.c:1245-1443) applied plane by plane.

Bars: the work buffer holds each src1 row quantized bit-exactly as GGML's
wdata would; dst within |y - E| <= 1e-4 |E| + 4e-6 A (oracle.within_tolerance)
of the fp64 re-accumulation for the src0 plane that broadcast selects
(i02 = i12 / r2, i03 = i13 / r3); bytes between strided dst rows untouched.
Cases: contiguous 2D at decode and prefill batch sizes, padded rows on every
operand (aligned, and 2-byte pads that take the unaligned kernels), src0
broadcast over src1 planes, batched planes that collapse into one GEMM, and a
src1 already quantized to the vec_dot type."""
from __future__ import annotations

import numpy as np
import pytest

import oracle as o
from weft_amd import ggml as G

pytestmark = pytest.mark.gpu

TYPE = {"q4_0": G.Q4_0, "q4_k": G.Q4_K, "iq2_xxs": G.IQ2_XXS, "mxfp4": G.MXFP4, "q6_k": G.Q6_K,
        "q5_k": G.Q5_K, "nvfp4": G.NVFP4, "q4_1": G.Q4_1, "iq2_xs": G.IQ2_XS}
VDT = {"q4_0": G.Q8_0, "mxfp4": G.Q8_0, "q4_k": G.Q8_K, "iq2_xxs": G.Q8_K, "q6_k": G.Q8_K,
       "q5_k": G.Q8_K, "nvfp4": G.Q8_0, "q4_1": G.Q8_1, "iq2_xs": G.Q8_K}
FMTS = list(TYPE)
NAN = 0x7FC00001  # a quiet NaN the kernels never produce


def make_weights(fmt, n, k, seed):
    """GGML-quantized N(0, 0.02) rows (the IQ2 formats by GGML's own
    quantize_iq2_xxs / quantize_iq2_xs, unit importance)."""
    x = o.seeded_normal(seed, (n, k), 0.02)
    if fmt in ("iq2_xs", "iq2_xxs"):
        return o.quantize_ggml_iq2(fmt, x)
    return o.quantize(fmt, x)


def run(hip, fmt, k, n, m, planes0=(1, 1), planes1=(1, 1), pad_w=0, pad_x=0, pad_y=0,
        prequant=False, seed=7):
    hip.torch.cuda.synchronize()
    ne02, ne03 = planes0
    ne12, ne13 = planes1
    rb = o.record_bytes(fmt, k)
    act = o.ACT_OF[fmt]
    rq = o.record_bytes(act, k)
    # src0: ne03 x ne02 planes of n rows, each row followed by pad_w bytes
    w = np.stack([make_weights(fmt, n, k, seed + p) for p in range(ne02 * ne03)]).reshape(ne03, ne02, n, rb)
    w_host = np.full((ne03, ne02, n, rb + pad_w), 0x5A, np.uint8)
    w_host[..., :rb] = w
    x = o.seeded_normal(seed + 100, (ne13, ne12, m, k))
    if prequant:
        src1_host = np.stack([o.quantize(act, x[i3, i2]) for i3 in range(ne13)
                              for i2 in range(ne12)]).reshape(ne13, ne12, m, rq)
        nb1 = [G.type_size(VDT[fmt]), rq, rq * m, rq * m * ne12]
        t1 = VDT[fmt]
    else:
        src1_host = np.zeros((ne13, ne12, m, k + pad_x), np.float32)
        src1_host[..., :k] = x
        row = 4 * (k + pad_x)
        nb1 = [4, row, row * m, row * m * ne12]
        t1 = G.F32
    y_row = 4 * (n + pad_y)
    wd = hip.to_dev(w_host)
    xd = hip.to_dev(src1_host)
    yd = hip.empty(y_row * m * ne12 * ne13)
    yd.t[:yd.nbytes].view(hip.torch.int32).fill_(NAN)
    nb0 = [G.type_size(TYPE[fmt]), rb + pad_w, (rb + pad_w) * n, (rb + pad_w) * n * ne02]
    s0 = G.tensor(TYPE[fmt], (k, n, ne02, ne03), wd.ptr, nb0)
    s1 = G.tensor(t1, (k, m, ne12, ne13), xd.ptr, nb1)
    d = G.tensor(G.F32, (n, m, ne12, ne13), yd.ptr, [4, y_row, y_row * m, y_row * m * ne12])
    wsize = G.mul_mat_work_size(s0, s1)
    assert wsize == (0 if prequant else rq * m * ne12 * ne13)
    wdata = hip.empty(max(wsize, 4), fill=0xA5)
    print(f"ggml mul_mat {fmt} k={k} n={n} m={m} planes0={planes0} planes1={planes1} "
          f"pads={pad_w},{pad_x},{pad_y} prequant={prequant}", flush=True)
    G.mul_mat(s0, s1, d, wdata.ptr, wsize)
    hip.torch.cuda.synchronize()
    assert hip.last_error() == 0
    y = yd.numpy(np.float32).reshape(ne13, ne12, m, n + pad_y)
    wq = wdata.numpy(np.uint8)[:wsize].reshape(ne13, ne12, m, rq) if wsize else None
    r2, r3 = ne12 // ne02, ne13 // ne03
    for i3 in range(ne13):
        for i2 in range(ne12):
            xq = o.quantize(act, x[i3, i2])
            if wq is not None:
                np.testing.assert_array_equal(wq[i3, i2], xq, err_msg=f"wdata plane {i2},{i3}")
            e, a = o.mul_mat_f64(fmt, w[i3 // r3, i2 // r2], xq, n, k, m)
            ok = o.within_tolerance(y[i3, i2, :, :n], e, a)
            assert ok.all(), f"plane {i2},{i3}: {int((~ok).sum())} outputs outside tolerance"
    if pad_y:
        assert (y[..., n:].view(np.int32) == NAN).all(), "dst padding written"


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("m", [1, 3, 40])
def test_contiguous(hip, fmt, m):
    run(hip, fmt, 1024, 256, m)


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("m", [1, 40])
def test_padded_rows(hip, fmt, m):
    # 16-byte pads keep the aligned kernels (GEMM / 16-byte GEMV paths)
    run(hip, fmt, 512, 200, m, pad_w=16, pad_x=12, pad_y=8)


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("m", [1, 24])
def test_unaligned_row_pads(hip, fmt, m):
    # a 2-byte (1-byte for MXFP4) weight-row pad: rows keep only the Encoding
    # alignment, so the GEMV kernels take every size
    run(hip, fmt, 512, 96, m, pad_w=1 if fmt in ("mxfp4", "q6_k", "nvfp4") else 2, pad_x=1, pad_y=3)


@pytest.mark.parametrize("fmt", FMTS)
def test_broadcast_over_planes(hip, fmt):
    run(hip, fmt, 512, 64, 3, planes0=(2, 1), planes1=(4, 2))


@pytest.mark.parametrize("fmt", FMTS)
def test_batched_planes_collapse(hip, fmt):
    run(hip, fmt, 512, 160, 20, planes1=(3, 1))


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("m", [1, 33])
def test_prequantized_src1(hip, fmt, m):
    run(hip, fmt, 512, 128, m, planes1=(2, 1), prequant=True)


# ---------------------------------------------------------------- MUL_MAT_ID
def run_id(hip, fmt, k, n, n_as, n_ids, ne11, n_tok, ids, pad_w=0, pad_x=0, prequant=False, seed=11):
    """ids: (n_tok, n_ids) int32 expert choices; entries outside [0, n_as)
    must leave their dst rows untouched."""
    hip.torch.cuda.synchronize()
    rb = o.record_bytes(fmt, k)
    act = o.ACT_OF[fmt]
    rq = o.record_bytes(act, k)
    w = np.stack([make_weights(fmt, n, k, seed + e) for e in range(n_as)])
    w_host = np.full((n_as, n, rb + pad_w), 0x5A, np.uint8)
    w_host[..., :rb] = w
    x = o.seeded_normal(seed + 500, (n_tok, ne11, k))
    xq = np.stack([o.quantize(act, x[t]) for t in range(n_tok)])  # (n_tok, ne11, rq)
    if prequant:
        xd = hip.to_dev(xq)
        s1 = G.tensor(VDT[fmt], (k, ne11, n_tok), xd.ptr)
    else:
        xp = np.zeros((n_tok, ne11, k + pad_x), np.float32)
        xp[..., :k] = x
        xd = hip.to_dev(xp)
        row = 4 * (k + pad_x)
        s1 = G.tensor(G.F32, (k, ne11, n_tok), xd.ptr, [4, row, row * ne11, row * ne11 * n_tok])
    wd = hip.to_dev(w_host)
    idd = hip.to_dev(np.ascontiguousarray(ids, dtype=np.int32))
    yd = hip.empty(4 * n * n_ids * n_tok)
    yd.t[:yd.nbytes].view(hip.torch.int32).fill_(NAN)
    s0 = G.tensor(TYPE[fmt], (k, n, n_as), wd.ptr,
                  [G.type_size(TYPE[fmt]), rb + pad_w, (rb + pad_w) * n, (rb + pad_w) * n * n_as])
    it = G.tensor(G.I32, (n_ids, n_tok), idd.ptr)
    d = G.tensor(G.F32, (n, n_ids, n_tok), yd.ptr)
    wsize = G.mul_mat_id_work_size(s0, s1, it)
    wdata = hip.empty(wsize, fill=0xA5)
    print(f"ggml mul_mat_id {fmt} k={k} n={n} n_as={n_as} n_ids={n_ids} ne11={ne11} "
          f"n_tok={n_tok} pad_w={pad_w} pad_x={pad_x} prequant={prequant}", flush=True)
    G.mul_mat_id(s0, s1, it, d, wdata.ptr, wsize)
    hip.torch.cuda.synchronize()
    assert hip.last_error() == 0
    y = yd.numpy(np.float32).reshape(n_tok, n_ids, n)
    wq = None if prequant else wdata.numpy(np.uint8)[:n_tok * ne11 * rq].reshape(n_tok, ne11, rq)
    for t in range(n_tok):
        for s in range(n_ids):
            e = int(ids[t, s])
            if not 0 <= e < n_as:
                assert (y[t, s].view(np.int32) == NAN).all(), f"pair {t},{s} with id {e} written"
                continue
            want_e, want_a = o.mul_mat_f64(fmt, w[e], xq[t, s % ne11][None], n, k, 1)
            ok = o.within_tolerance(y[t, s][None], want_e, want_a)
            assert ok.all(), f"pair {t},{s} expert {e}: {int((~ok).sum())} outside tolerance"
        if wq is not None:
            for r in range(ne11):
                if 0 <= int(ids[t, r]) < n_as:  # the row's writer pair ran
                    np.testing.assert_array_equal(wq[t, r], xq[t, r], err_msg=f"wdata row {t},{r}")


@pytest.mark.parametrize("fmt", FMTS)
def test_mul_mat_id_decode(hip, fmt):
    # one token, 4 of 8 experts, the activation broadcast to every slot
    run_id(hip, fmt, 1024, 256, 8, 4, 1, 1, np.array([[5, 0, 7, 2]]))


@pytest.mark.parametrize("fmt", FMTS)
def test_mul_mat_id_tokens_and_invalid_ids(hip, fmt):
    rng = np.random.default_rng(3)
    ids = rng.integers(0, 6, size=(7, 2))
    ids[2, 1] = -1
    ids[5, 0] = 6
    run_id(hip, fmt, 512, 96, 6, 2, 2, 7, ids)


@pytest.mark.parametrize("fmt", FMTS)
def test_mul_mat_id_prequantized_and_strided(hip, fmt):
    ids = np.array([[1, 3, 0], [2, 2, 1]])
    run_id(hip, fmt, 512, 64, 4, 3, 1, 2, ids, pad_w=1 if fmt in ("mxfp4", "q6_k", "nvfp4") else 2, prequant=True)


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("ne11", [1, 4])
@pytest.mark.parametrize("prequant", [False, True])
def test_mul_mat_id_grouped_gemm(hip, fmt, ne11, prequant):
    """Many pairs per expert: the device groups the pairs by expert and the
    grouped MFMA GEMMs run them (ragged tiles, one expert unused, invalid ids
    skipped).  A pre-quantized Q8_0 / Q8_1 src1 takes the pair GEMV (the
    Q4_0 / MXFP4 / NVFP4 / Q4_1 GEMMs read a planar activation quantized from
    F32); the launch log shows which ran."""
    from weft_amd import _lib
    rng = np.random.default_rng(5)
    n_tok, n_ids, n_as = 70, 4, 8
    ids = rng.integers(0, n_as - 1, size=(n_tok, n_ids))  # expert 7 never chosen
    ids[3, 2] = -1
    ids[40, 0] = n_as
    _lib.launch_log()
    run_id(hip, fmt, 1024, 300, n_as, n_ids, ne11, n_tok, ids, pad_w=16,
           pad_x=0 if prequant else 4, prequant=prequant)
    launched = _lib.launch_log()
    gemv = prequant and o.ACT_OF[fmt] in ("q8_0", "q8_1")
    assert any("gemm" in name for name in launched) != gemv, launched


@pytest.mark.parametrize("fmt,prequant", [(f, False) for f in FMTS] +
                         [(f, True) for f in ("q4_k", "q6_k", "iq2_xxs")])
def test_mul_mat_id_rows_past_the_pair_gemv(hip, fmt, prequant):
    """Four pairs with K = 2^18 (a quantized row of ~300 KB, past the pair
    GEMV's LDS): the grouped MFMA GEMM takes them whatever the pair count."""
    from weft_amd import _lib
    _lib.launch_log()
    run_id(hip, fmt, 1 << 18, 8, 3, 2, 1, 2, np.array([[2, 0], [0, 1]]), prequant=prequant)
    launched = _lib.launch_log()
    assert any("gemm" in name for name in launched) and not any("gemv" in name for name in launched), launched


@pytest.mark.parametrize("k", [8192, 11008])
def test_mul_mat_id_decode_long_rows(hip, k):
    # batch-1 pairs with rows of two / three 4096-column steps: the
    # split-step GEMV with its per-row partial sums, pair by pair
    run_id(hip, "q4_k", k, 160, 4, 2, 1, 1, np.array([[3, 1]]))
