"""bench.py's GPU legs build their inputs without oracle/: the lookup tables
it passes to the kernels must equal the oracle's (pinned against GGML's
tables), and its synthetic records must have the formats' sizes (CPU)."""
from __future__ import annotations

import numpy as np
import pytest

import bench
import oracle as o


def test_bench_tables_are_ggmls():
    t = bench.ggml_tables()
    assert np.array_equal(t["iq2_xxs"][0].view(np.uint8), o.iq2xxs_grid())
    assert np.array_equal(t["iq2_xs"][0].view(np.uint8), o.iq2xs_grid())
    assert np.array_equal(t["iq2_xxs"][1], o.signs_i8x8()) and np.array_equal(t["iq2_xs"][1], o.signs_i8x8())
    assert np.array_equal(t["mxfp4"][0], o.kvalues_mxfp4()) and np.array_equal(t["nvfp4"][0], o.kvalues_mxfp4())
    assert np.array_equal(t["mxfp4"][1].view(np.uint32), o.e8m0_half_table().view(np.uint32))
    assert np.array_equal(t["nvfp4"][1].view(np.uint32), o.ue4m3_table().view(np.uint32))


@pytest.mark.parametrize("fmt", sorted({c[1] for c in bench.CASES.values()}))
def test_synthetic_records(fmt):
    w = bench.synthetic_weights(fmt, 3, 512)
    assert w.shape == (3, o.record_bytes(fmt, 512)) and bench.record_bytes(fmt, 512) == w.shape[1]
    if fmt == "mxfp4":
        e = w.reshape(3, -1, 17)[:, :, 0]
        assert ((e >= 26) & (e <= 224)).all()  # exponents the block-scaled MFMA takes directly


def test_bench_seeded_normal_is_the_oracles():
    assert np.array_equal(bench.seeded_normal(7, (3, 5), 0.5), o.seeded_normal(7, (3, 5), 0.5))
