"""Seeded random shapes through every format's mul_mat entry point (GPU).

Each case draws N in [1, 3000), K a multiple of the format's K step (1-12
steps) and either a prefill batch (M in [16, 300): the MFMA GEMMs, with
ragged row and token tiles and odd superblock / pair counts) or a small
batch (M in [1, 16): the batch-1 kernels and the staged GEMV), and checks
Xq byte for byte and every output against the oracle's fp64
re-accumulation (oracle.within_tolerance).  A wider sweep of this kind
found a K = 256 Q5_K output whose superblock halves cancel to 1/19000 of
their size, which fixed the tolerance's magnitude to be summed over scale
groups.  IQ2 weights are random records (every byte pattern is valid), so
the kernels see every grid and sign index.  A second set sends random
batch-1 shapes through the `*_decode` entry points, where the
register-resident kernels run (N up to 12000, K up to their row limits).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle as o
from tests.test_gpu_parity import check_mul_mat, run_mul_mat

pytestmark = pytest.mark.gpu

SYMBOL = {"q4_0": "production_mul_mat_q4_0", "q4_1": "production_mul_mat_q4_1",
          "mxfp4": "production_mul_mat_mxfp4", "nvfp4": "production_mul_mat_nvfp4",
          "q4_k": "production_mul_mat_q4_k_staged", "q5_k": "production_mul_mat_q5_k",
          "q6_k": "production_mul_mat_q6_k", "iq2_xxs": "production_mul_mat_iq2_xxs_staged",
          "iq2_xs": "production_mul_mat_iq2_xs_staged"}


def _cases():
    rng = np.random.default_rng(20261202)
    out = []
    for fmt in SYMBOL:
        step = 512 if fmt.startswith("iq2") else 256  # the IQ2 GEMMs take pairs of superblocks
        for kind, (mlo, mhi) in (("prefill", (16, 300)), ("small", (1, 16))):
            for _ in range(2):
                n = int(rng.integers(1, 3000))
                k = int(rng.integers(1, 13)) * step
                m = int(rng.integers(mlo, mhi))
                out.append(pytest.param(fmt, n, k, m, int(rng.integers(1 << 30)),
                                        id=f"{fmt}-{kind}-n{n}-k{k}-m{m}"))
    return out


@pytest.mark.parametrize("fmt,n,k,m,seed", _cases())
def test_random_shape(hip, fmt, n, k, m, seed):
    x = o.seeded_normal(seed, (m, k))
    if fmt.startswith("iq2"):
        w = o.random_records(fmt, n, k, seed=seed + 1)
    else:
        w = o.quantize(fmt, o.seeded_normal(seed + 1, (n, k), 0.02))
    print(f"{fmt} n={n} k={k} m={m}", flush=True)
    w_, x_, xq, y = run_mul_mat(hip, SYMBOL[fmt], fmt, n, k, m, w=w, x=x)
    check_mul_mat(fmt, w_, x_, xq, y, n, k, m)


def _decode_cases():
    """Batch-1 shapes for the register-resident decode kernels: N anywhere
    in [1, 12000) (partial workgroups and waves), K up to 16 steps of the
    format's K granule (Q4_K: 48 superblocks, its split-step kernel)."""
    rng = np.random.default_rng(20261203)
    out = []
    for fmt in SYMBOL:
        if fmt == "iq2_xs":
            continue  # IQ2_XS has no _decode entry; its mul_mat entry is swept above
        step = {"q4_0": 64, "q4_1": 64, "mxfp4": 64, "nvfp4": 64, "q4_k": 256, "q5_k": 256,
                "q6_k": 512, "iq2_xxs": 512}[fmt]
        top = 48 * 256 // step if fmt == "q4_k" else 4096 // step
        for _ in range(3):
            n = int(rng.integers(1, 12000))
            k = int(rng.integers(1, top + 1)) * step
            out.append(pytest.param(fmt, n, k, int(rng.integers(1 << 30)), id=f"{fmt}-n{n}-k{k}"))
    return out


@pytest.mark.parametrize("fmt,n,k,seed", _decode_cases())
def test_random_decode_shape(hip, fmt, n, k, seed):
    x = o.seeded_normal(seed, (1, k))
    if fmt.startswith("iq2"):
        w = o.random_records(fmt, n, k, seed=seed + 1)
    else:
        w = o.quantize(fmt, o.seeded_normal(seed + 1, (n, k), 0.02))
    print(f"decode {fmt} n={n} k={k}", flush=True)
    w_, x_, xq, y = run_mul_mat(hip, f"production_mul_mat_{fmt}_decode", fmt, n, k, 1, w=w, x=x)
    check_mul_mat(fmt, w_, x_, xq, y, n, k, 1)
