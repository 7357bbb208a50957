"""CPU oracle for the quantized mul_mat path -- TEST INFRASTRUCTURE ONLY.

numpy-facing ctypes wrapper of ``oracle/libweft_oracle.so`` (built from
``oracle/weft_oracle.c`` by ``oracle/Makefile``), a plain-C restatement of the
GGML CPU functions the reference Weft repo checks its kernels against
(``source/c/ggml/llama.cpp/ggml/src/ggml-quants.c``,
``ggml-cpu/quants.c``).  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg import this package, and only as the checker
or the timed CPU baseline; the product library ``libweft_hip`` never calls it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libweft_oracle.so"

Q4_0, Q4_K, IQ2_XXS, MXFP4, Q6_K, Q5_K, NVFP4, Q4_1, IQ2_XS = 0, 1, 2, 3, 4, 5, 6, 7, 8
FORMATS = {"q4_0": Q4_0, "q4_k": Q4_K, "iq2_xxs": IQ2_XXS, "mxfp4": MXFP4, "q6_k": Q6_K, "q5_k": Q5_K,
           "nvfp4": NVFP4, "q4_1": Q4_1, "iq2_xs": IQ2_XS}

# (elements per record, bytes per record)
RECORD = {
    "q4_0": (32, 18), "mxfp4": (32, 17), "q8_0": (32, 34),
    "q4_k": (256, 144), "q8_k": (256, 292), "iq2_xxs": (256, 66), "q6_k": (256, 210),
    "q5_k": (256, 176), "nvfp4": (64, 36), "q4_1": (32, 20), "q8_1": (32, 36), "iq2_xs": (256, 74),
}
ACT_OF = {"q4_0": "q8_0", "mxfp4": "q8_0", "q4_k": "q8_k", "iq2_xxs": "q8_k", "q6_k": "q8_k", "q5_k": "q8_k",
          "nvfp4": "q8_0", "q4_1": "q8_1", "iq2_xs": "q8_k"}


def build() -> Path:
    """Compile the oracle library with its Makefile (gcc)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


_lib = None
NATIVE_PATH = HERE / "libweft_oracle_native.so"
BUILD_FLAGS = "-O3 -march=x86-64-v3 -ffp-contract=off -fopenmp"
NATIVE_FLAGS = "-O3 -march=native -ffp-contract=off -fopenmp"


def use_native() -> str:
    """Switch this process to the oracle built for the running machine's own
    ISA (``make native``, built here if missing) and return its flags; on a
    failed build keep the portable library and return its flags."""
    global _lib
    try:
        subprocess.run(["make", "-s", "-C", str(HERE), "native"], check=True,
                       stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL)
        l = ctypes.CDLL(str(NATIVE_PATH))
    except (OSError, subprocess.CalledProcessError):
        lib()
        return BUILD_FLAGS
    _declare(l)
    _lib = l
    return NATIVE_FLAGS


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = ctypes.CDLL(str(LIB_PATH))
        _declare(_lib)
    return _lib


_P = ctypes.c_void_p
_I64 = ctypes.c_int64


def _declare(l: ctypes.CDLL) -> None:
    sig = {
        "wo_fp16_to_fp32": ([ctypes.c_uint16], ctypes.c_float),
        "wo_fp32_to_fp16": ([ctypes.c_float], ctypes.c_uint16),
        "wo_e8m0_to_fp32_half": ([ctypes.c_uint8], ctypes.c_float),
        "wo_fp16_to_fp32_array": ([_P, _P, _I64], None),
        "wo_fp32_to_fp16_array": ([_P, _P, _I64], None),
        "wo_iq2xxs_grid": ([_P], None), "wo_ksigns_iq2xs": ([_P], None), "wo_iq2xs_grid": ([_P], None),
        "wo_signs_i8x8": ([_P], None), "wo_kvalues_mxfp4": ([_P], None),
        "wo_e8m0_half_table": ([_P], None),
        "wo_ue4m3_to_fp32": ([ctypes.c_uint8], ctypes.c_float),
        "wo_fp32_to_ue4m3": ([ctypes.c_float], ctypes.c_uint8),
        "wo_ue4m3_table": ([_P], None),
        "wo_weight_row_bytes": ([ctypes.c_int, _I64], ctypes.c_size_t),
        "wo_act_row_bytes": ([ctypes.c_int, _I64], ctypes.c_size_t),
        "wo_mul_mat": ([ctypes.c_int, _P, _P, _P, _P, _I64, _I64, _I64, ctypes.c_int], None),
        "wo_mul_mat_q": ([ctypes.c_int, _P, _P, _P, _I64, _I64, _I64, ctypes.c_int], None),
        "wo_mul_mat_f64": ([ctypes.c_int, _P, _P, _P, _P, _I64, _I64, _I64, ctypes.c_int], None),
        "wo_int_partials": ([ctypes.c_int, _P, _P, _I64, _P], _I64),
        "wo_max_threads": ([], ctypes.c_int),
        "wo_mul_mat_ggml": ([ctypes.c_int, _P, _P, _P, _P, _I64, _I64, _I64, ctypes.c_int], None),
        "wo_evict": ([_P, ctypes.c_size_t], None),
        "wo_quantize_row_iq2_xxs_ggml": ([_P, _P, _I64, _P], None),
        "wo_quantize_row_iq2_xs_ggml": ([_P, _P, _I64, _P], None),
        "wo_iq2_grid_index": ([ctypes.c_int, ctypes.c_int], ctypes.c_int),
        "wo_iq2_neighbours": ([ctypes.c_int, ctypes.c_int, _P], ctypes.c_int),
    }
    for fmt in ("q4_0", "q4_K", "mxfp4", "iq2_xxs", "q6_K", "q5_K", "nvfp4", "q8_0", "q8_K", "q4_1", "q8_1"):
        sig[f"wo_quantize_row_{fmt}"] = ([_P, _P, _I64], None)
    for fmt in ("q4_0", "q4_K", "mxfp4", "iq2_xxs", "q6_K", "q5_K", "nvfp4", "q4_1", "iq2_xs"):
        sig[f"wo_dequantize_row_{fmt}"] = ([_P, _P, _I64], None)
    for name in ("q4_0_q8_0", "q4_K_q8_K", "iq2_xxs_q8_K", "mxfp4_q8_0", "q6_K_q8_K", "q5_K_q8_K",
                 "nvfp4_q8_0", "q4_1_q8_1", "iq2_xs_q8_K"):
        sig[f"wo_vec_dot_{name}"] = ([_P, _P, _I64], ctypes.c_float)
    for name, (args, res) in sig.items():
        fn = getattr(l, name)
        fn.argtypes = args
        fn.restype = res


def _ptr(a: np.ndarray) -> int:
    assert a.flags.c_contiguous
    return a.ctypes.data


def record_bytes(fmt: str, k: int) -> int:
    elems, nbytes = RECORD[fmt]
    if k % elems:
        raise ValueError(f"{fmt} needs K to be a multiple of {elems}")
    return k // elems * nbytes


# ---------------------------------------------------------------- conversions
def fp16_to_fp32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().wo_fp16_to_fp32_array(_ptr(h), _ptr(out), h.size)
    return out


def fp32_to_fp16(f: np.ndarray) -> np.ndarray:
    f = np.ascontiguousarray(f, dtype=np.float32)
    out = np.empty(f.shape, np.uint16)
    lib().wo_fp32_to_fp16_array(_ptr(f), _ptr(out), f.size)
    return out


def e8m0_half(e: int) -> float:
    return lib().wo_e8m0_to_fp32_half(e)


# --------------------------------------------------------------------- tables
def iq2xxs_grid() -> np.ndarray:
    out = np.empty(2048, np.uint8)
    lib().wo_iq2xxs_grid(_ptr(out))
    return out


def iq2xs_grid() -> np.ndarray:
    """iq2xs_grid (ggml-common.h:617-746) as 512 x 8 bytes."""
    out = np.empty(4096, np.uint8)
    lib().wo_iq2xs_grid(_ptr(out))
    return out


def ksigns_iq2xs() -> np.ndarray:
    out = np.empty(128, np.uint8)
    lib().wo_ksigns_iq2xs(_ptr(out))
    return out


def signs_i8x8() -> np.ndarray:
    out = np.empty(1024, np.int8)
    lib().wo_signs_i8x8(_ptr(out))
    return out


def kvalues_mxfp4() -> np.ndarray:
    out = np.empty(16, np.int8)
    lib().wo_kvalues_mxfp4(_ptr(out))
    return out


def e8m0_half_table() -> np.ndarray:
    out = np.empty(256, np.float32)
    lib().wo_e8m0_half_table(_ptr(out))
    return out


def ue4m3_table() -> np.ndarray:
    """ggml_ue4m3_to_fp32 of every byte (NVFP4 sub-block scales)."""
    out = np.empty(256, np.float32)
    lib().wo_ue4m3_table(_ptr(out))
    return out


# ----------------------------------------------------------------- quantizers
def quantize(fmt: str, x: np.ndarray, out: np.ndarray | None = None) -> np.ndarray:
    """Quantize rows of fp32 ``x`` (..., K) into ``fmt`` records (uint8)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    k = x.shape[-1]
    rows = x.size // k if k else 0
    rb = record_bytes(fmt, k)
    if out is None:
        out = np.zeros(x.shape[:-1] + (rb,), np.uint8)
    if fmt == "iq2_xs":
        raise ValueError("no IQ2_XS weight quantizer: tests use random_records('iq2_xs', ...)")
    name = {"q4_0": "q4_0", "q4_k": "q4_K", "mxfp4": "mxfp4", "iq2_xxs": "iq2_xxs",
            "q6_k": "q6_K", "q5_k": "q5_K", "nvfp4": "nvfp4", "q8_0": "q8_0", "q8_k": "q8_K",
            "q4_1": "q4_1", "q8_1": "q8_1"}[fmt]
    fn = getattr(lib(), f"wo_quantize_row_{name}")
    # one call over all rows: records never straddle rows
    fn(_ptr(x), _ptr(out), rows * k)
    return out


def quantize_ggml_iq2(fmt: str, x: np.ndarray, importance: np.ndarray | None = None) -> np.ndarray:
    """GGML's own IQ2_XXS / IQ2_XS weight quantizer (quantize_iq2_xxs /
    quantize_iq2_xs, ggml-quants.c:3580-3602) on rows of fp32 ``x`` (..., K),
    with an importance matrix of x's shape (None: all ones, as the
    reference's repro passes, examples/repro/weft/mul_mat_runtime.cpp:762-776)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    k = x.shape[-1]
    out = np.zeros(x.shape[:-1] + (record_bytes(fmt, k),), np.uint8)
    qw = None
    if importance is not None:
        qw = np.ascontiguousarray(np.broadcast_to(importance, x.shape), dtype=np.float32)
    fn = {"iq2_xxs": lib().wo_quantize_row_iq2_xxs_ggml, "iq2_xs": lib().wo_quantize_row_iq2_xs_ggml}[fmt]
    fn(_ptr(x), _ptr(out), x.size, None if qw is None else _ptr(qw))
    return out


def iq2_grid_index(fmt: str, u: int) -> int:
    """The grid entry of 2-bit point u in GGML's quantizer map (-1: off the grid)."""
    return lib().wo_iq2_grid_index(int(fmt == "iq2_xs"), u)


def iq2_neighbours(fmt: str, u: int) -> list[int]:
    """The neighbour list iq2xs_init_impl builds for off-grid point u."""
    out = np.zeros(512, np.uint16)
    n = lib().wo_iq2_neighbours(int(fmt == "iq2_xs"), u, _ptr(out))
    return [int(v) for v in out[:n]]


def dequantize(fmt: str, w: np.ndarray, k: int) -> np.ndarray:
    """Dequantize ``w`` (..., row_bytes) of ``fmt`` into fp32 (..., k)."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    rb = record_bytes(fmt, k)
    rows = w.size // rb if rb else 0
    out = np.empty(w.shape[:-1] + (k,), np.float32)
    name = {"q4_0": "q4_0", "q4_k": "q4_K", "mxfp4": "mxfp4", "iq2_xxs": "iq2_xxs", "q6_k": "q6_K", "q5_k": "q5_K",
            "nvfp4": "nvfp4", "q4_1": "q4_1", "iq2_xs": "iq2_xs"}[fmt]
    getattr(lib(), f"wo_dequantize_row_{name}")(_ptr(w), _ptr(out), rows * k)
    return out


_VEC_DOT = {"q4_0": "q4_0_q8_0", "q4_k": "q4_K_q8_K", "iq2_xxs": "iq2_xxs_q8_K",
            "mxfp4": "mxfp4_q8_0", "q6_k": "q6_K_q8_K", "q5_k": "q5_K_q8_K", "nvfp4": "nvfp4_q8_0",
            "q4_1": "q4_1_q8_1", "iq2_xs": "iq2_xs_q8_K"}


def vec_dot(fmt: str, w: np.ndarray, x: np.ndarray, k: int) -> float:
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.uint8)
    return float(getattr(lib(), f"wo_vec_dot_{_VEC_DOT[fmt]}")(_ptr(w), _ptr(x), k))


def mul_mat(fmt: str, W: np.ndarray, X: np.ndarray, n: int, k: int, m: int,
            threads: int = 0, xq: np.ndarray | None = None):
    """GGML MUL_MAT: returns (Xq, Y) with Y (m, n) fp32."""
    W = np.ascontiguousarray(W, dtype=np.uint8)
    X = np.ascontiguousarray(X, dtype=np.float32)
    if xq is None:
        xq = np.zeros((m, record_bytes(ACT_OF[fmt], k)), np.uint8)
    y = np.empty((m, n), np.float32)
    lib().wo_mul_mat(FORMATS[fmt], _ptr(W), _ptr(X), _ptr(xq), _ptr(y), n, k, m, threads)
    return xq, y


def mul_mat_ggml(fmt: str, W: np.ndarray, X: np.ndarray, n: int, k: int, m: int,
                 threads: int = 0, xq: np.ndarray | None = None, y: np.ndarray | None = None):
    """GGML MUL_MAT with GGML's thread schedule (quantize split by blocks,
    chunked rows from a shared counter): returns (Xq, Y)."""
    W = np.ascontiguousarray(W, dtype=np.uint8)
    X = np.ascontiguousarray(X, dtype=np.float32)
    if xq is None:
        xq = np.zeros((m, record_bytes(ACT_OF[fmt], k)), np.uint8)
    if y is None:
        y = np.empty((m, n), np.float32)
    lib().wo_mul_mat_ggml(FORMATS[fmt], _ptr(W), _ptr(X), _ptr(xq), _ptr(y), n, k, m, threads)
    return xq, y


def evict(buf: np.ndarray) -> None:
    lib().wo_evict(_ptr(buf), buf.nbytes)


def mul_mat_q(fmt: str, W: np.ndarray, Xq: np.ndarray, n: int, k: int, m: int,
              threads: int = 0) -> np.ndarray:
    W = np.ascontiguousarray(W, dtype=np.uint8)
    Xq = np.ascontiguousarray(Xq, dtype=np.uint8)
    y = np.empty((m, n), np.float32)
    lib().wo_mul_mat_q(FORMATS[fmt], _ptr(W), _ptr(Xq), _ptr(y), n, k, m, threads)
    return y


def mul_mat_f64(fmt: str, W: np.ndarray, Xq: np.ndarray, n: int, k: int, m: int,
                threads: int = 0):
    """fp64 re-accumulation of the exact integer partials: (E, A)."""
    W = np.ascontiguousarray(W, dtype=np.uint8)
    Xq = np.ascontiguousarray(Xq, dtype=np.uint8)
    e = np.empty((m, n), np.float64)
    a = np.empty((m, n), np.float64)
    lib().wo_mul_mat_f64(FORMATS[fmt], _ptr(W), _ptr(Xq), _ptr(e), _ptr(a), n, k, m, threads)
    return e, a


def int_partials(fmt: str, w: np.ndarray, x: np.ndarray, k: int) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.uint8)
    out = np.empty(9 * (k // 32) + 16, np.int32)
    n = lib().wo_int_partials(FORMATS[fmt], _ptr(w), _ptr(x), k, _ptr(out))
    return out[:n].copy()


def interleave_rows(w: np.ndarray, n: int, k: int, rows: int = 16) -> np.ndarray:
    """The derived layout Q4K_I[rows] of an n x k Q4_K matrix
    (examples/formats/ggml.py:286-290): each ``rows``-row cohort is written
    byte-major per record (doc/dsl/encoding-and-artifacts.md:209), cohort
    superblock j at ((c * nsb) + j) * 144 * rows, byte b of row r at
    16 b + r (lib/Target/Emission/Memory.cpp:984-991)."""
    nsb = k // 256
    if n % rows or k % 256:
        raise ValueError("Q4K_I needs whole row cohorts and whole superblocks")
    src = np.ascontiguousarray(w, dtype=np.uint8).reshape(n // rows, rows, nsb, 144)
    return np.ascontiguousarray(src.transpose(0, 2, 3, 1)).reshape(-1)


def random_records(fmt: str, n: int, k: int, seed: int = 0) -> np.ndarray:
    """Rows of records with random payload bytes and a moderate fp16 scale
    (every byte pattern of these formats is a valid record).  The input
    generator for IQ2_XS, whose GGML quantizer (an importance-weighted grid
    search) is not restated here."""
    rng = np.random.default_rng(seed)
    nrec = k // RECORD[fmt][0]
    rec = rng.integers(0, 256, size=(n, nrec, RECORD[fmt][1]), dtype=np.uint8)
    d = fp32_to_fp16(rng.uniform(1e-4, 2e-3, size=(n, nrec)).astype(np.float32))
    rec[:, :, 0:2] = d.view(np.uint8).reshape(n, nrec, 2)
    return rec.reshape(n, -1)


def iq2_tables_mul_mat_f64(fmt: str, W: np.ndarray, Xq: np.ndarray, n: int, k: int, m: int,
                           grid: np.ndarray, signs: np.ndarray):
    """fp64 re-accumulation (E, A) of IQ2_XXS / IQ2_XS rows against Q8_K rows
    with CALLER tables, as the reference's kernels state it for any I8X8
    grid and sign table: each weight byte is grid * sign as i8 x i8 -> i8,
    wrapping modulo 256 (examples/kernels/vec_dot/iq2_xxs_q8_k.py:25-45,
    examples/functions/quantization.py:71-83: equal element types are not
    promoted, python/weft/frontend/compiler.py:1276-1292); those bytes are
    dotted with the Q8_K bytes in int32 per grid entry pair of one scale
    (IQ2_XXS: a 32-group with 2 s + 1, s = the group word's top 4 bits;
    IQ2_XS: a 16-element half with 2 s + 1 from its scale nibble), then
    fp16 d * Q8_K d * 0.125 per superblock.  GGML's generic vec_dots
    (ggml-cpu/quants.c:855-946) are the same function on GGML's tables.
    Numpy, small shapes (tests only).  E = sum of the scale-group terms, A =
    sum of their magnitudes (oracle.within_tolerance), as wo_mul_mat_f64."""
    xs = fmt == "iq2_xs"
    rec = 74 if xs else 66
    nsb = k // 256
    g8 = np.asarray(grid, np.int8).reshape(-1, 8)
    s8 = np.asarray(signs, np.int8).reshape(128, 8)
    Wr = np.ascontiguousarray(W, np.uint8).reshape(n, nsb, rec)
    Xr = np.ascontiguousarray(Xq, np.uint8).reshape(m, nsb, 292)
    dw = fp16_to_fp32(Wr[:, :, 0:2].copy().view(np.uint16)[..., 0]).astype(np.float64)    # (n, nsb)
    dx = Xr[:, :, 0:4].copy().view(np.float32)[..., 0].astype(np.float64)              # (m, nsb)
    xq = Xr[:, :, 4:260].view(np.int8).astype(np.int64).reshape(m, nsb, 16, 16)        # 16 halves of 16
    words = Wr[:, :, 2:66].copy().view(np.uint16).astype(np.int64)                     # (n, nsb, 32)
    if xs:
        gi = words & 511                                                                # entry e: elements 8e..
        si = words >> 9
        sc = Wr[:, :, 66:74].astype(np.int64)
        ls = np.stack([sc & 15, sc >> 4], axis=-1).reshape(n, nsb, 16)                  # per 16-half
    else:
        w4 = words.reshape(n, nsb, 8, 4)
        idx = w4[..., 0] | (w4[..., 1] << 16)
        meta = w4[..., 2] | (w4[..., 3] << 16)
        gi = np.stack([(idx >> (8 * l)) & 255 for l in range(4)], axis=-1).reshape(n, nsb, 32)
        si = np.stack([(meta >> (7 * l)) & 127 for l in range(4)], axis=-1).reshape(n, nsb, 32)
        ls = np.repeat(meta >> 28, 2, axis=-1)                                          # per 16-half
    # i8 x i8 -> i8 (wraps), then widened: (n, nsb, 32 entries, 8)
    wb = (g8[gi].astype(np.int16) * s8[si].astype(np.int16)).astype(np.int8).astype(np.int64)
    wb = wb.reshape(n, nsb, 16, 16)
    # integer sums per 16-element half: (m, n, nsb, 16)
    part = np.einsum("msjt,nsjt->mnsj", xq, wb)
    term = part * (2 * ls[None] + 1)
    if not xs:  # one scale per 32-group: the two halves' integer sum times 2 s + 1
        term = (part[..., 0::2] + part[..., 1::2]) * (2 * ls[None, ..., 0::2] + 1)
    t = 0.125 * dw[None, :, :, None] * dx[:, None, :, None] * term                      # (m, n, nsb, groups)
    e = np.zeros((m, n))
    a = np.zeros((m, n))
    for b in range(nsb):  # wo_mul_mat_f64's order: superblocks, then their scale groups
        for g in range(t.shape[3]):
            e += t[:, :, b, g]
            a += np.abs(t[:, :, b, g])
    return e, a


def max_threads() -> int:
    return int(lib().wo_max_threads())


# Tolerance for fp32 outputs against the fp64 re-accumulation E with
# magnitude A = sum_b |scale_b * P_b| over the format's scale groups (a
# 32- or 16-element block or sub-block, the K-quants' min terms apart):
# relative 1e-4 of |E| plus 4e-6 of A (about 64 fp32 ulps of the magnitude:
# room for the fp32 rounding of up to ~90 group terms in any summation
# order).  Every partial sum a kernel rounds to fp32 is a sum of whole scale
# groups, so |partial| <= A: a K-quant superblock's two halves can each be
# hundreds of times its total (the min terms of x's halves cancel), which a
# per-superblock A would not bound.
REL_TOL = 1e-4
MAG_TOL = 4e-6


def within_tolerance(y: np.ndarray, e: np.ndarray, a: np.ndarray) -> np.ndarray:
    y = np.asarray(y, np.float64)
    return np.isfinite(y) & (np.abs(y - e) <= REL_TOL * np.abs(e) + MAG_TOL * a)


def seeded_normal(seed: int, shape, sigma: float = 1.0) -> np.ndarray:
    """Counter-based seeded N(0, sigma^2) fp32 (numpy PCG64 + Box-Muller)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    return (rng.standard_normal(size=shape, dtype=np.float64) * sigma).astype(np.float32)
