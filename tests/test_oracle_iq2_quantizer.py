"""GGML's IQ2_XXS / IQ2_XS weight quantizers as restated in oracle/
(quantize_iq2_xxs / quantize_iq2_xs, ggml-quants.c:3580-3602, over
quantize_row_iq2_xxs_impl :3222-3398 and quantize_row_iq2_xs_impl
:3400-3578, with iq2xs_init_impl's search tables :2781-3186).

GGML itself cannot be built here (ggml-impl.h includes gguf.h, which the
reference does not vendor), so the quantizers' bytes are not compared with
GGML's; they are pinned by:
  * the search tables against a brute-force restatement of their definition
    (every one of the 43692 2-bit points, both grids);
  * known answers: inputs that lie exactly on the grid (every grid entry,
    random even-parity signs, one scale per superblock) come back with those
    signs, nearly all as those grid entries (GGML's search misses a few,
    explained in the test), and fully recovered superblocks with d = a / 31
    and the top scale code;
  * the record invariants and the reconstruction error of N(0, 0.02) rows.
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

import oracle as o

GOLDEN = json.loads((Path(__file__).parent / "golden" / "ggml_tables.json").read_text())
LEVEL = {0x08: 0, 0x19: 1, 0x2B: 2}  # grid byte -> 2-bit level l (value 2l + 1 in the search)


def grid_levels(fmt: str) -> np.ndarray:
    """(entries, 8) levels of the GGML grid fixture (ggml-common.h text)."""
    key = "iq2xxs_grid" if fmt == "iq2_xxs" else "iq2xs_grid"
    g = np.array([int(h, 16) for h in GOLDEN[key]], np.uint64).view(np.uint8).reshape(-1, 8)
    return np.vectorize(LEVEL.__getitem__)(g).astype(np.int64)


def point_codes(levels: np.ndarray) -> np.ndarray:
    return (levels << (2 * np.arange(8))).sum(-1)


@pytest.mark.parametrize("fmt", ["iq2_xxs", "iq2_xs"])
def test_search_tables_brute_force(fmt):
    """iq2xs_init_impl: a grid point maps to its index; every other point
    lists the grid entries at the two smallest squared distances present
    (on the odd integers 2l + 1), in order of (distance, index)."""
    gl = grid_levels(fmt)
    codes = point_codes(gl)
    on_grid = {int(c): j for j, c in enumerate(codes)}
    gpos = 2 * gl + 1
    u = np.arange(43692)
    upos = 2 * ((u[:, None] >> (2 * np.arange(8))[None, :]) & 3) + 1
    buf = np.zeros(512, np.uint16)
    lib = o.lib()
    xs = int(fmt == "iq2_xs")
    for c0 in range(0, u.size, 4096):
        pos = upos[c0:c0 + 4096]
        d2 = ((pos[:, None, :] - gpos[None, :, :]) ** 2).sum(-1)
        keys = np.sort(d2 * 4096 + np.arange(gl.shape[0])[None, :], axis=1)
        dist, idx = keys // 4096, keys % 4096
        second = np.where(dist > dist[:, :1], dist, 1 << 30).min(axis=1)
        count = (dist <= second[:, None]).sum(axis=1)
        for r in range(pos.shape[0]):
            p = c0 + r
            n = lib.wo_iq2_neighbours(xs, p, buf.ctypes.data)
            if p in on_grid:
                assert o.iq2_grid_index(fmt, p) == on_grid[p] and n == 0
                continue
            assert o.iq2_grid_index(fmt, p) == -1
            assert n == count[r] and np.array_equal(buf[:n], idx[r, :n]), p


def exact_superblocks(fmt: str, seed: int):
    """Rows whose every 8-chunk is a grid entry (each entry of the grid once)
    with an even-parity sign pattern, at one scale a per superblock."""
    rng = np.random.default_rng(seed)
    gl = grid_levels(fmt)
    n = gl.shape[0]                  # 256 or 512 chunks: 8 or 16 superblocks
    order = rng.permutation(n)
    signs7 = rng.integers(0, 128, size=n)
    neg = (signs7[:, None] >> np.arange(7)) & 1
    neg = np.concatenate([neg, neg.sum(1, keepdims=True) & 1], axis=1)  # bit 7: parity
    nsb = n // 32
    a = np.repeat(rng.uniform(1e-3, 5e-2, size=nsb), 32)  # one scale per superblock
    x = (np.where(neg == 1, -1.0, 1.0) * (2 * gl[order] + 1) * a[:, None]).astype(np.float32)
    return x.reshape(1, -1), order, signs7, a


@pytest.mark.parametrize("fmt,seed", [("iq2_xxs", 3), ("iq2_xxs", 4), ("iq2_xs", 3), ("iq2_xs", 4)])
def test_quantizer_recovers_exact_grid_points(fmt, seed):
    """Every sign pattern comes back; almost every chunk comes back as its
    grid entry.  GGML's level search does not reach every exact point: it
    tries 13 (IQ2_XS: 19) scales around 5 / eff_max, eff_max = 3 x the scale
    make_qp_quants fits with levels up to 4, and a group of mostly 1s and 3s
    with a single 5 is fitted with levels 1, 3, 4, so no tried scale maps
    the 3s to level 1 (ggml-quants.c:3282-3305).  Superblocks whose chunks
    all came back carry d = fp16(a / 31) and scale code 15 in every group."""
    x, order, signs7, a = exact_superblocks(fmt, seed=seed)
    rec = o.quantize_ggml_iq2(fmt, x).reshape(-1, 66 if fmt == "iq2_xxs" else 74)
    d = o.fp16_to_fp32(rec[:, 0:2].copy().view(np.uint16).reshape(-1))
    want_d = o.fp16_to_fp32(o.fp32_to_fp16(a[::32] / 31))  # a: one value per chunk
    if fmt == "iq2_xxs":
        words = rec[:, 2:66].copy().view(np.uint32).reshape(-1, 8, 2)  # (superblock, group, word)
        idx = (words[..., 0:1] >> (8 * np.arange(4))) & 0xFF          # (sb, g, chunk)
        sg = (words[..., 1:2] >> (7 * np.arange(4))) & 0x7F
        sc = words[..., 1] >> 28
    else:
        qs = rec[:, 2:66].copy().view(np.uint16).reshape(-1, 16, 2)    # (sb, 16-group, chunk)
        idx, sg = qs & 511, qs >> 9
        sc = np.stack([rec[:, 66:74] & 15, rec[:, 66:74] >> 4], axis=-1).reshape(-1, 16)
    assert np.array_equal(sg.reshape(-1), signs7)
    hit = (idx.reshape(-1) == order).reshape(len(d), 32)
    assert hit.mean() >= 0.95, hit.mean()  # a lane, sign or layout mistake misses nearly all
    whole = hit.all(axis=1)
    assert whole.sum() >= len(d) // 2
    assert np.allclose(d[whole], want_d[whole], rtol=2e-3)
    assert np.all(sc[whole] == 15)


@pytest.mark.parametrize("fmt", ["iq2_xxs", "iq2_xs"])
def test_quantizer_records_and_error(fmt):
    x = o.seeded_normal(17, (24, 1024), 0.02)
    w = o.quantize_ggml_iq2(fmt, x)
    assert np.array_equal(w, o.quantize_ggml_iq2(fmt, x, np.ones_like(x)))  # None = importance 1
    y = o.dequantize(fmt, w, 1024)
    rel = np.sqrt(((y - x) ** 2).sum() / (x ** 2).sum())
    assert rel < 0.36, rel
    if fmt == "iq2_xxs":  # GGML's search does better than the nearest-grid generator
        y2 = o.dequantize(fmt, o.quantize(fmt, x), 1024)
        assert rel < np.sqrt(((y2 - x) ** 2).sum() / (x ** 2).sum())
    # a zero superblock: d = 0 and no payload
    z = np.zeros((1, 256), np.float32)
    assert not o.quantize_ggml_iq2(fmt, z).any()
    # importance changes the search
    imp = np.random.default_rng(1).uniform(0.1, 4.0, size=x.shape).astype(np.float32)
    assert not np.array_equal(w, o.quantize_ggml_iq2(fmt, x, imp))


@pytest.mark.parametrize("fmt,f", [("iq2_xs", 15), ("iq2_xxs", 16)])
def test_reference_repro_record(fmt, f):
    """The reference repro's weight record (mul_mat_runtime.cpp:762-776:
    x_i = ((19 i + 7 F) % 127 - 63) / 13, importance 1, F the format's
    1-based index in kQuantizedWeightTypes): a valid record that
    reconstructs the row."""
    i = np.arange(256)
    x = (((i * 19 + f * 7) % 127 - 63) / 13.0).astype(np.float32).reshape(1, 256)
    w = o.quantize_ggml_iq2(fmt, x)
    y = o.dequantize(fmt, w, 256)
    assert np.isfinite(y).all()
    assert np.sqrt(((y - x) ** 2).sum() / (x ** 2).sum()) < 0.5
