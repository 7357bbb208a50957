"""Q4K_I[16] artifact functions and q4_k_q8_k_gemv{,_groups4,_contract} on the
GPU, through the C ABI (examples/kernels/gemv/q4_k.py:8-26; repro
examples/repro/weft/q4_k_gemv_runtime.cpp).

Bars (declared before any run): the device pack is byte-for-byte the oracle's
interleave (itself pinned against the reference emitter's record address in
test_oracle.py); the gemv's fp32 outputs satisfy the fp64 re-accumulation
tolerance of oracle.within_tolerance (|y - E| <= 1e-4 |E| + 4e-6 A) on the
row-major records the packed bytes came from.  Shapes: the reference
harness's M = 14336, K = 4096, long rows (K = 11008, an odd number of
superblocks per wave), and small ones.
"""
from __future__ import annotations

import ctypes
import functools

import numpy as np
import pytest

import oracle as o

pytestmark = pytest.mark.gpu

VARIANTS = ("q4_k_q8_k_gemv", "q4_k_q8_k_gemv_groups4", "q4_k_q8_k_gemv_contract")


@functools.lru_cache(maxsize=None)
def case(m: int, k: int, seed: int = 31):
    w = o.quantize("q4_k", o.seeded_normal(seed, (m, k), 0.02))
    x = o.quantize("q8_k", o.seeded_normal(seed + 1, (1, k)))
    return w, x


def packed_size(hip, sym, m, k):
    fn = getattr(hip.lib, sym + "_W_packed_size")
    fn.restype = ctypes.c_size_t
    fn.argtypes = [ctypes.c_size_t, ctypes.c_size_t]
    return fn(m, k)


def pack(hip, sym, w, m, k):
    size = packed_size(hip, sym, m, k)
    assert size == w.nbytes
    src = hip.to_dev(w)
    dst = hip.empty(size, fill=0xA5)
    fn = getattr(hip.lib, sym + "_W_pack")
    fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_size_t]
    fn.restype = None
    fn(src.ptr, dst.ptr, m, k)
    hip.torch.cuda.synchronize()
    hip._lib.check(sym + "_W_pack")
    return dst


@pytest.mark.parametrize("m,k", [(14336, 4096), (64, 256), (48, 11008)])
def test_pack_is_the_interleave(hip, m, k):
    w, _ = case(m, k)
    dst = pack(hip, "q4_k_q8_k_gemv", w, m, k)
    np.testing.assert_array_equal(dst.numpy(np.uint8), o.interleave_rows(w, m, k))


@pytest.mark.parametrize("sym", VARIANTS)
@pytest.mark.parametrize("m,k", [(14336, 4096), (4096, 11008), (16, 256), (32, 768), (160, 1280)])
def test_gemv_matches_fp64_reaccumulation(hip, sym, m, k):
    w, x = case(m, k)
    wi = pack(hip, sym, w, m, k)
    xd = hip.to_dev(x)
    y = hip.empty(4 * m, fill=0xA5)
    hip.call(sym, wi, xd, y, m, k)
    got = y.numpy(np.float32)
    e, a = o.mul_mat_f64("q4_k", w, x.reshape(1, -1), m, k, 1)
    ok = o.within_tolerance(got, e.reshape(-1), a.reshape(-1))
    assert ok.all(), f"{int((~ok).sum())} rows outside tolerance"


def test_gemv_edge_records(hip):
    """Zero d, zero dmin, all-zero activation superblock, largest scales."""
    m, k = 32, 1024
    w, x = case(m, k, seed=77)
    w = w.copy().reshape(m, k // 256, 144)
    w[3, 1, 0:2] = 0           # d = 0: the scale term vanishes
    w[5, 2, 2:4] = 0           # dmin = 0: the min term vanishes
    w[7, 0, 4:16] = 0xFF       # every 6-bit scale and min at 63
    w = w.reshape(-1)
    x = x.copy().reshape(k // 256, 292)
    x[2, :260] = 0             # an all-zero Q8_K record (d = 0, qs = 0)
    x = x.reshape(-1)
    wi = pack(hip, "q4_k_q8_k_gemv", w, m, k)
    y = hip.empty(4 * m, fill=0xA5)
    hip.call("q4_k_q8_k_gemv", wi, hip.to_dev(x), y, m, k)
    e, a = o.mul_mat_f64("q4_k", w, x.reshape(1, -1), m, k, 1)
    assert o.within_tolerance(y.numpy(np.float32), e.reshape(-1), a.reshape(-1)).all()


def test_gemv_rejects_partial_cohorts_and_records(hip):
    lib = hip.lib
    w = hip.empty(24 * 144 * 2)
    x = hip.empty(292 * 2)
    y = hip.empty(4 * 24)
    lib.q4_k_q8_k_gemv(w.ptr, x.ptr, y.ptr, 24, 512)  # 24 rows: not whole cohorts
    assert hip.last_error() != 0
    assert hip.last_error() == 0
    lib.q4_k_q8_k_gemv(w.ptr, x.ptr, y.ptr, 16, 500)  # K not whole superblocks
    assert hip.last_error() != 0
    assert hip.last_error() == 0


def test_gemv_through_the_runtime(hip):
    import torch
    from weft_amd import kernels as K
    from weft_amd.runtime import Buffer, jit

    m, k = 256, 4096
    w, x = case(m, k)
    wi = pack(hip, "q4_k_q8_k_gemv", w, m, k)
    W = Buffer(wi.t[wi.offset:wi.offset + wi.nbytes], shape=(m, k), encoding="Q4K_I[16]")
    X = Buffer(torch.from_numpy(x).to(hip.dev), shape=(k,), encoding="Q8_K")
    y_t = torch.zeros(m, dtype=torch.float32, device=hip.dev)
    jit(K.q4_k_q8_k_gemv)(W, X, y_t)
    e, a = o.mul_mat_f64("q4_k", w, x.reshape(1, -1), m, k, 1)
    assert o.within_tolerance(y_t.cpu().numpy(), e.reshape(-1), a.reshape(-1)).all()
