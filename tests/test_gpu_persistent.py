"""production_mul_mat_q4_k_persistent and its artifact-phase functions on the
GPU, through the C ABI (examples/kernels/mul_mat/q4_k_persistent.py:10-31;
harness examples/repro/weft/mul_mat_runtime.cpp:338-347 and :807-808, which
packs with (N, K) and calls with (M, K, N)).

Bars (declared before any run): the packed weight is byte-for-byte the
oracle's 16-row interleave; Xq is bit-exact Q8_K of X; Y is within the fp64
re-accumulation tolerance (|y - E| <= 1e-4 |E| + 4e-6 A) of the row-major
records the packed bytes came from.  For M >= 16 the GEMM reads the same
bytes in the same order as production_mul_mat_q4_k_staged, so the two
outputs must be bit-identical.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle as o
from tests.test_gpu_parity import crafted_acts_q8k, crafted_q4_k

pytestmark = pytest.mark.gpu

SYM = "production_mul_mat_q4_k_persistent"
SENTINEL = 0xA5


def pack(hip, w, n, k):
    size_fn = getattr(hip.lib, SYM + "_W_packed_size")
    size_fn.restype = ctypes.c_size_t
    size_fn.argtypes = [ctypes.c_size_t, ctypes.c_size_t]
    size = size_fn(n, k)
    assert size == w.nbytes
    dst = hip.empty(size, fill=SENTINEL)
    hip.call(SYM + "_W_pack", hip.to_dev(w), dst, n, k)
    return dst


def run(hip, w, x, n, k, m):
    wi = pack(hip, w, n, k)
    xq = hip.empty(o.record_bytes("q8_k", k) * m, fill=SENTINEL)
    y = hip.empty(4 * m * n, fill=SENTINEL)
    print(f"{SYM} n={n} k={k} m={m}", flush=True)
    hip.call(SYM, wi, hip.to_dev(x), xq, y, m, k, n)
    return wi, xq.numpy(np.uint8).reshape(m, -1), y.numpy(np.float32).reshape(m, n)


def check(w, x, xq, y, n, k, m):
    # GGML leaves an all-zero block's bsums unwritten: quantize over the sentinel
    want_xq = np.full((m, o.record_bytes("q8_k", k)), SENTINEL, np.uint8)
    o.quantize("q8_k", x, out=want_xq)
    np.testing.assert_array_equal(xq, want_xq, err_msg="Xq workspace differs")
    e, a = o.mul_mat_f64("q4_k", w, want_xq, n, k, m)
    ok = o.within_tolerance(y, e, a)
    assert ok.all(), f"{int((~ok).sum())} outputs outside tolerance, e.g. {np.argwhere(~ok)[:4].tolist()}"


@pytest.mark.parametrize("n,k,m", [
    (4096, 4096, 512),    # config 4 at N = 4096
    (144, 768, 70),       # partial weight tile (N % 128 = 16) and token tile, odd superblocks
    (48, 11008, 17),      # long rows, one partial cohort tile
    (256, 256, 16),       # one superblock, one token tile
    (64, 1024, 1),        # decode: the interleaved GEMV
    (32, 512, 5),         # a few rows: one GEMV per row
])
def test_persistent_matches_fp64(hip, n, k, m):
    w = o.quantize("q4_k", o.seeded_normal(3, (n, k), 0.02))
    x = o.seeded_normal(4, (m, k))
    wi, xq, y = run(hip, w, x, n, k, m)
    np.testing.assert_array_equal(wi.numpy(np.uint8), o.interleave_rows(w, n, k))
    check(w, x, xq, y, n, k, m)


@pytest.mark.parametrize("n,k,m", [(4096, 4096, 512), (144, 768, 70), (32784, 768, 70)])
def test_persistent_gemm_equals_row_major_gemm(hip, n, k, m):
    w = o.quantize("q4_k", o.seeded_normal(5, (n, k), 0.02))
    x = o.seeded_normal(6, (m, k))
    _, _, y = run(hip, w, x, n, k, m)
    xq2 = hip.empty(o.record_bytes("q8_k", k) * m, fill=SENTINEL)
    y2 = hip.empty(4 * m * n, fill=SENTINEL)
    hip.call("production_mul_mat_q4_k_staged", hip.to_dev(w), hip.to_dev(x), xq2, y2, n, k, m)
    np.testing.assert_array_equal(y, y2.numpy(np.float32).reshape(m, n))


def test_persistent_crafted_records(hip):
    """The interleaved GEMM on records no quantizer emits (zero, subnormal,
    extreme d / dmin, sc = m = 63, all-15 nibbles) against activations with
    all-zero Q8_K blocks and rows."""
    rng = np.random.default_rng(78)
    n, k, m = 256, 1024, 64
    w = crafted_q4_k(n, k, rng)
    x = crafted_acts_q8k(m, k, rng)
    _, xq, y = run(hip, w, x, n, k, m)
    check(w, x, xq, y, n, k, m)


def test_persistent_rejects_partial_cohorts(hip):
    lib = hip.lib
    w = hip.empty(24 * 144 * 2)
    x = hip.empty(4 * 512 * 2)
    xq = hip.empty(292 * 2 * 2)
    y = hip.empty(4 * 24 * 2)
    getattr(lib, SYM)(w.ptr, x.ptr, xq.ptr, y.ptr, 2, 512, 24)  # N = 24: not whole cohorts
    assert hip.last_error() != 0
    assert hip.last_error() == 0
    getattr(lib, SYM)(w.ptr, x.ptr, xq.ptr, y.ptr, 2, 500, 16)  # K not whole superblocks
    assert hip.last_error() != 0
    assert hip.last_error() == 0
