"""MXFP4 x Q8_0 on every E8M0 exponent, against GGML's own fp32 order (GPU).

GGML combines a block as d = fp16(dx) * e8m0_half(e), then sumf += d * I
(ggml-cpu/quants.c:265-273).  Near the ends of the exponent range that order
decides the result: d can be a rounded subnormal (e small), d or d * I can
overflow to inf (e large, or e = 255 whose 2^127 has no E8M0 block-scale
encoding), and inf * 0 is NaN.  The block-scaled MFMA prefill, the GEMV and
the grouped MUL_MAT_ID GEMM must reproduce those results.

Inputs: every row carries one block at exponent e = row (0..255) among
blocks at moderate exponents, a few rows have small exponents throughout
(subnormal d), and the activation has a large-scale token (d * I overflows
for high e), a tiny-scale token (fp16 subnormal dx), a token whose fp16 dx
is inf, and an all-zero token.

Bar: outputs are non-finite exactly where GGML's are (same NaN-ness, same
sign of inf).  Finite outputs satisfy |y - g| <= 1e-4 |g| + 4e-6 A, g being
GGML's fp32 result (the oracle's restatement of its order) and A the fp64
sum of |scale * partial| (oracle.mul_mat_f64): the per-block terms are then
GGML's and only their summation order differs.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle as o
from weft_amd import ggml as G

SENTINEL = 0xA5


def crafted_weights(n: int, k: int, seed: int = 31) -> np.ndarray:
    rng = np.random.default_rng(seed)
    nb = k // 32
    rec = rng.integers(0, 256, size=(n, nb, 17), dtype=np.uint8)
    rec[:, :, 0] = rng.integers(100, 151, size=(n, nb), dtype=np.uint8)
    rows = np.arange(n)
    rec[rows, rows % nb, 0] = (rows % 256).astype(np.uint8)  # every exponent once per 256 rows
    for r in range(min(n, 8)):  # small exponents throughout: subnormal d
        rec[r, :, 0] = (3 * r + np.arange(nb) % 3).astype(np.uint8)
    rec[9, :, 0] = 255
    rec[9, :, 1:] = 0  # e = 255 blocks with I = 0: inf * 0 where dx overflows ...
    rec[10, :, 0] = 255  # ... and e = 255 blocks with random nibbles
    return rec.reshape(n, -1)


def crafted_acts(m: int, k: int, seed: int = 32) -> np.ndarray:
    x = o.seeded_normal(seed, (m, k))
    x[0] *= 1e4    # dx ~ 300: d * I overflows for e >= ~228
    x[1] *= 1e-5   # dx ~ 3e-7: an fp16 subnormal
    x[2] *= 3e6    # amax / 127 > 65504: fp16 dx = inf
    x[3] = 0.0     # dx = 0
    return x.astype(np.float32)


def check_ggml(y, w, xq, n, k, m, what, mixed=True):
    g = o.mul_mat_q("mxfp4", w, xq, n, k, m)
    _, a = o.mul_mat_f64("mxfp4", w, xq, n, k, m)
    y = np.asarray(y, np.float32).reshape(m, n)
    fin = np.isfinite(g)
    if mixed:
        assert fin.sum() > 0 and (~fin).sum() > 0, "inputs must produce finite and non-finite outputs"
    bad = np.isfinite(y) != fin
    assert not bad.any(), f"{what}: finiteness differs at {np.argwhere(bad)[:5].tolist()}"
    nf = ~fin
    bad = nf & (np.isnan(y) != np.isnan(g))
    assert not bad.any(), (f"{what}: NaN / inf pattern differs at (token, row, gpu, ggml) "
                           f"{[(int(i), int(j), float(y[i, j]), float(g[i, j])) for i, j in np.argwhere(bad)[:8]]}")
    inf = nf & ~np.isnan(g)
    assert (np.sign(y[inf]) == np.sign(g[inf])).all(), f"{what}: sign of inf differs"
    yd, gd = y[fin].astype(np.float64), g[fin].astype(np.float64)
    ok = np.abs(yd - gd) <= 1e-4 * np.abs(gd) + 4e-6 * a[fin]
    if not ok.all():
        idx = np.argwhere(fin)[~ok][:5]
        raise AssertionError(f"{what}: {int((~ok).sum())} finite outputs off, e.g. "
                             f"{[(tuple(i), float(y[tuple(i)]), float(g[tuple(i)])) for i in idx]}")


def q80(x):
    return o.quantize("q8_0", x)


def test_inputs_cover_every_exponent():
    w = crafted_weights(256, 1024).reshape(256, 32, 17)
    assert set(np.unique(w[:, :, 0]).tolist()) == set(range(256))
    xq = q80(crafted_acts(64, 1024)).reshape(64, 32, 34)
    d = o.fp16_to_fp32(xq[:, :, :2].copy().view(np.uint16)[..., 0])
    assert np.isinf(d[2]).any() and (d[3] == 0).all()
    assert ((d[1] > 0) & (d[1] < 2.0 ** -14)).any()  # fp16 subnormal dx


@pytest.mark.gpu
@pytest.mark.parametrize("n,k,m", [(256, 1024, 64), (300, 1536, 70)])
def test_prefill_every_exponent(hip, n, k, m):
    """production_mul_mat_mxfp4: the block-scaled MFMA GEMM (tiles whose
    exponents leave the exactly reproduced range run at unit scale and are
    combined in GGML's order)."""
    w, x = crafted_weights(n, k), crafted_acts(m, k)
    xq = hip.empty(o.record_bytes("q8_0", k) * m, fill=SENTINEL)
    y = hip.empty(4 * m * n, fill=SENTINEL)
    print(f"mxfp4 prefill exponents n={n} k={k} m={m}", flush=True)
    hip.call("production_mul_mat_mxfp4", hip.to_dev(w), hip.to_dev(x), xq, hip.codebook, hip.scale, y,
             n, k, m)
    want_xq = q80(x)
    np.testing.assert_array_equal(xq.numpy(np.uint8).reshape(m, -1), want_xq)
    check_ggml(y.numpy(np.float32), w, want_xq, n, k, m, "prefill")


@pytest.mark.gpu
@pytest.mark.parametrize("m", [4, 3])
def test_decode_every_exponent(hip, m):
    """production_mul_mat_mxfp4_decode (the table-driven GEMV)."""
    n, k = 256, 1024
    w, x = crafted_weights(n, k), crafted_acts(4, k)[:m]
    xq = hip.empty(o.record_bytes("q8_0", k) * m, fill=SENTINEL)
    y = hip.empty(4 * m * n, fill=SENTINEL)
    print(f"mxfp4 decode exponents m={m}", flush=True)
    hip.call("production_mul_mat_mxfp4_decode", hip.to_dev(w), hip.to_dev(x), xq, hip.codebook, hip.scale,
             y, n, k, m)
    check_ggml(y.numpy(np.float32), w, q80(x), n, k, m, "decode")


@pytest.mark.gpu
def test_vec_dot_every_exponent(hip):
    """quantized_vec_dot_mxfp4_q8_0 over one row holding all 256 exponents,
    against each of the four extreme tokens."""
    k = 256 * 32
    rng = np.random.default_rng(33)
    rec = rng.integers(0, 256, size=(k // 32, 17), dtype=np.uint8)
    rec[:, 0] = np.arange(256, dtype=np.uint8)
    w = rec.reshape(1, -1)
    xs = crafted_acts(4, k, seed=34)
    got, want = [], []
    for t in range(4):
        xq = q80(xs[t:t + 1])
        y = hip.empty(4, fill=SENTINEL)
        hip.call("quantized_vec_dot_mxfp4_q8_0", hip.to_dev(w), hip.to_dev(xq), hip.codebook, hip.scale, y, k)
        got.append(y.numpy(np.float32)[0])
        want.append(o.vec_dot("mxfp4", w, xq, k))
    g, y = np.array(want, np.float32), np.array(got, np.float32)
    assert (np.isfinite(g) == np.isfinite(y)).all() and (np.isnan(g) == np.isnan(y)).all()
    fin = np.isfinite(g)
    assert np.allclose(y[fin], g[fin], rtol=1e-4, atol=0), (y, g)


@pytest.mark.gpu
def test_grouped_mul_mat_id_every_exponent(hip):
    """GGML MUL_MAT_ID with enough pairs per expert for the grouped
    block-scaled GEMM, each expert holding every exponent."""
    k, n, n_as, n_ids, n_tok = 1024, 256, 3, 2, 64
    rb, rq = o.record_bytes("mxfp4", k), o.record_bytes("q8_0", k)
    w = np.stack([crafted_weights(n, k, seed=40 + e) for e in range(n_as)])
    x = crafted_acts(n_tok, k, seed=41)
    ids = np.stack([np.arange(n_tok) % n_as, (np.arange(n_tok) + 1) % n_as], axis=1).astype(np.int32)
    wd, xd, idd = hip.to_dev(w), hip.to_dev(x[:, None, :].copy()), hip.to_dev(ids)
    yd = hip.empty(4 * n * n_ids * n_tok, fill=SENTINEL)
    s0 = G.tensor(G.MXFP4, (k, n, n_as), wd.ptr, [G.type_size(G.MXFP4), rb, rb * n, rb * n * n_as])
    s1 = G.tensor(G.F32, (k, 1, n_tok), xd.ptr, [4, 4 * k, 4 * k, 4 * k * n_tok])
    it = G.tensor(G.I32, (n_ids, n_tok), idd.ptr)
    d = G.tensor(G.F32, (n, n_ids, n_tok), yd.ptr)
    wsize = G.mul_mat_id_work_size(s0, s1, it)
    wdata = hip.empty(wsize, fill=SENTINEL)
    print("mxfp4 grouped mul_mat_id exponents", flush=True)
    G.mul_mat_id(s0, s1, it, d, wdata.ptr, wsize)
    hip.torch.cuda.synchronize()
    assert hip.last_error() == 0
    y = yd.numpy(np.float32).reshape(n_tok, n_ids, n)
    xq = q80(x)
    for e in range(n_as):
        for s in range(n_ids):
            toks = np.nonzero(ids[:, s] == e)[0]
            check_ggml(y[toks, s], w[e], xq[toks], n, k, len(toks), f"expert {e} slot {s}", mixed=False)
    assert rq * n_tok <= wsize
