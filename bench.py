#!/usr/bin/env python3
"""Benchmark of the quantized mul_mat hot path on one MI355X.

Headline (BASELINE.json metric "Q4_K mul_mat: decode GB/s (% of 8 TB/s) +
prefill TOPS (% int8 MFMA peak)"): one step = one production_mul_mat_q4_k_decode
call on config 3's W_up shape (N=11008, K=4096, M=1), Q8_K activation quantize
included, exactly as the reference's timed mul_mat (weft-kernel-performance.csv:59).
``value`` is the algorithmic HBM bytes of the call (encoded W + fp32 X + Xq
write + fp32 Y = 25,427,520 B) divided by the measured time per call, in GB/s.

Inputs are seeded synthetic data, resident in HBM before timing: weight
records of random payload bytes with their scale fields at the magnitudes
GGML's quantizers give an N(0, 0.02^2) matrix (the kernels' time does not
depend on the values), activations ~ N(0, 1), pre-quantized activations by
the library's own q8_K_quantize.  Only the CPU baseline below uses oracle/.  Every case rotates its weights
over enough copies (> 2 x the 256 MB Infinity Cache) that each call reads
them from HBM; the write-bound row dequantize rotates its outputs as well
(``one_output_us``: the same calls into one output buffer).  Each case is
timed three ways on the library's stream:
  * ``us``: windows of K back-to-back calls, each window between two HIP
    events; the per-call time of the median window of 10 (``us_min`` /
    ``us_max``: the fastest and slowest window), the headline;
  * ``cold_us``: BASELINE.md's protocol -- 512 MiB written to flush the
    caches, then one call between two events; median of 20;
  * ``graph_us``: the same back-to-back calls replayed from a captured HIP
    graph (launch cost of a serving loop that captures its steps).
Floors measured in the same run: an empty launch back to back, one
streaming-read launch of the same bytes, and for the write-bound row
dequantize one streaming-write launch of its output bytes (library
probes); for the
prefill shapes, the vendor's plain int8 GEMM (hipBLASLt through
torch._int_mm) of the same M x N x K.  ``kernels`` lists what one call
launched (the library's launch log).

CPU baseline: oracle/'s restatement of GGML's MUL_MAT (quantize_row_q8_K_ref
+ ggml_vec_dot_q4_K_q8_K_generic) on the same decode call, built on the host
that runs it with -march=native, with GGML's thread schedule over every host
thread (``value``), and single-threaded under the reference's kernel
protocol: one warmup, a 64 MiB eviction before each of 10 timed calls,
median (doc/experiments/protocol.md:46-55).

Output: one JSON line.  ``adjacent`` (the formats beside the north star, in
brief) comes before ``configs`` (BASELINE.json's configs 1-5b in full), so
the end of the line, which is what a log tail keeps, holds the BASELINE
configs.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0   # dense int8 MFMA
FP8_PEAK_TOPS = 5000.0    # dense fp8 MFMA: the rate of an fp4 x fp8 f8f6f4 product
FP4_PEAK_TOPS = 10100.0   # dense fp4 / fp6 MFMA
MALL_BYTES = 256 << 20
FLUSH_BYTES = 512 << 20

# name: (symbol, format, N, K, M, bound)
CASES = {
    "q4_k_decode_w_up": ("production_mul_mat_q4_k_decode", "q4_k", 11008, 4096, 1, "hbm"),
    "q4_k_decode_w_down": ("production_mul_mat_q4_k_decode", "q4_k", 4096, 11008, 1, "hbm"),
    "q4_0_decode": ("production_mul_mat_q4_0_decode", "q4_0", 4096, 4096, 1, "hbm"),
    "iq2_xxs_decode": ("production_mul_mat_iq2_xxs_decode", "iq2_xxs", 4096, 4096, 1, "hbm"),
    "mxfp4_decode": ("production_mul_mat_mxfp4_decode", "mxfp4", 4096, 4096, 1, "hbm"),
    "q4_k_dequant": ("row_dequantize_q4_k", "q4_k", 11008, 4096, 0, "hbm"),
    # Q4K_I[16] GEMV at the reference harness's shape (q4_k_gemv_runtime.cpp:77-78);
    # N is the row count M of that ABI, the activation is pre-quantized Q8_K
    "q4_k_gemv_interleaved": ("q4_k_q8_k_gemv", "q4_k", 14336, 4096, -1, "hbm"),
    "q4_k_prefill_n4096": ("production_mul_mat_q4_k_staged", "q4_k", 4096, 4096, 512, "mfma"),
    "q4_k_prefill_n11008": ("production_mul_mat_q4_k_staged", "q4_k", 11008, 4096, 512, "mfma"),
    "mxfp4_prefill": ("production_mul_mat_mxfp4", "mxfp4", 4096, 4096, 512, "mfma"),
    "q4_0_prefill": ("production_mul_mat_q4_0", "q4_0", 4096, 4096, 512, "mfma"),
    "iq2_xxs_prefill": ("production_mul_mat_iq2_xxs_staged", "iq2_xxs", 4096, 4096, 512, "mfma"),
    # adjacent formats at the W_up shape (ggml-common.h:330-358, :211-217)
    "q6_k_decode": ("production_mul_mat_q6_k_decode", "q6_k", 11008, 4096, 1, "hbm"),
    "q6_k_prefill": ("production_mul_mat_q6_k", "q6_k", 4096, 4096, 512, "mfma"),
    "q5_k_decode": ("production_mul_mat_q5_k_decode", "q5_k", 11008, 4096, 1, "hbm"),
    "q5_k_prefill": ("production_mul_mat_q5_k", "q5_k", 4096, 4096, 512, "mfma"),
    "nvfp4_decode": ("production_mul_mat_nvfp4_decode", "nvfp4", 11008, 4096, 1, "hbm"),
    "nvfp4_prefill": ("production_mul_mat_nvfp4", "nvfp4", 4096, 4096, 512, "mfma"),
    "q4_1_decode": ("production_mul_mat_q4_1_decode", "q4_1", 11008, 4096, 1, "hbm"),
    "q4_1_prefill": ("production_mul_mat_q4_1", "q4_1", 4096, 4096, 512, "mfma"),
    "iq2_xs_decode": ("production_mul_mat_iq2_xs", "iq2_xs", 4096, 4096, 1, "hbm"),
    "iq2_xs_prefill": ("production_mul_mat_iq2_xs_staged", "iq2_xs", 4096, 4096, 512, "mfma"),
    # GGML MUL_MAT_ID (MoE) prefill at a Mixtral-8x7B FFN shape: 8 experts of
    # 14336 x 4096 Q4_K, 2 experts per token, 512 tokens (the grouped GEMM)
    "q4_k_moe_prefill": ("weft_ggml_mul_mat_id", "q4_k", 14336, 4096, 512, "mfma"),
    # GGML MUL_MAT with src1 already in Q8_K: the Q4_K GEMM alone, no quantize pass
    # the same prefill from the persisted Q4K_I[16] interleave (packed outside the timing)
    "q4_k_persistent_prefill_n4096": ("production_mul_mat_q4_k_persistent", "q4_k", 4096, 4096, 512, "mfma"),
    "q4_k_prefill_n4096_q8k_src1": ("weft_ggml_mul_mat", "q4_k", 4096, 4096, 512, "mfma"),
    "q4_k_prefill_n11008_q8k_src1": ("weft_ggml_mul_mat", "q4_k", 11008, 4096, 512, "mfma"),
}
MOE_EXPERTS, MOE_USED = 8, 2
HEADLINE = "q4_k_decode_w_up"
# BASELINE.json configs (label: case), reported in full and last
BASELINE_CASES = {
    "1_q4_0_decode": "q4_0_decode",
    "2_q4_k_dequant": "q4_k_dequant",
    "3_q4_k_decode_w_up": "q4_k_decode_w_up",
    "3_q4_k_decode_w_down": "q4_k_decode_w_down",
    "4_q4_k_prefill_n4096": "q4_k_prefill_n4096",
    "4_q4_k_prefill_n11008": "q4_k_prefill_n11008",
    "5a_iq2_xxs_decode": "iq2_xxs_decode",
    "5b_mxfp4_prefill": "mxfp4_prefill",
}
WINDOWS = 10  # timed windows per case; the median window is reported


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50, help="calls per timed window")
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--cpu-seconds", type=float, default=10.0,
                   help="wall-clock budget of the all-threads CPU baseline sample")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--no-extra", action="store_true",
                   help="skip the cold / graph timings and the floors")
    p.add_argument("--cases", default="all",
                   help="comma-separated secondary cases to run (default all; 'none' for "
                        "the headline only): " + ",".join(c for c in CASES if c != HEADLINE))
    p.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                   help="also run one plain device-to-device copy of MIB MiB, the known-size "
                        "kernel that HBM byte counters are scaled against")
    return p.parse_args()


# (elements, bytes) per record of the GGML formats (ggml-common.h block structs)
RECORD = {"q4_0": (32, 18), "q4_1": (32, 20), "mxfp4": (32, 17), "q8_0": (32, 34), "q8_1": (32, 36),
          "q4_k": (256, 144), "q5_k": (256, 176), "q6_k": (256, 210), "q8_k": (256, 292),
          "iq2_xxs": (256, 66), "iq2_xs": (256, 74), "nvfp4": (64, 36)}
ACT_OF = {"q4_0": "q8_0", "mxfp4": "q8_0", "nvfp4": "q8_0", "q4_1": "q8_1"}  # others: Q8_K


def record_bytes(fmt: str, k: int) -> int:
    elems, nbytes = RECORD[fmt]
    return k // elems * nbytes


def seeded_normal(seed: int, shape, sigma: float = 1.0) -> np.ndarray:
    rng = np.random.Generator(np.random.PCG64(seed))
    return (rng.standard_normal(size=shape, dtype=np.float64) * sigma).astype(np.float32)


def synthetic_weights(fmt: str, n: int, k: int, seed: int = 1) -> np.ndarray:
    """n rows of fmt records: random payload bytes, and the scale fields at
    the magnitudes GGML's quantizers give an N(0, 0.02) matrix (every byte
    pattern is a valid record of these formats, and the kernels' time does
    not depend on the values; MXFP4 exponents stay in the range the
    block-scaled MFMA takes directly)."""
    rng = np.random.default_rng(seed)
    elems, nbytes = RECORD[fmt]
    nrec = k // elems
    rec = rng.integers(0, 256, size=(n, nrec, nbytes), dtype=np.uint8)

    def f16(lo, hi, at):
        v = rng.uniform(lo, hi, size=(n, nrec)).astype(np.float16)
        rec[:, :, at:at + 2] = v.view(np.uint8).reshape(n, nrec, 2)

    if fmt in ("q4_0", "iq2_xxs", "iq2_xs"):
        f16(2e-3, 8e-3, 0)
    elif fmt == "q4_1":
        f16(4e-3, 8e-3, 0)
        f16(-6e-2, -3e-2, 2)
    elif fmt in ("q4_k", "q5_k"):
        f16(1e-4, 3e-4, 0)
        f16(1e-4, 3e-4, 2)
    elif fmt == "q6_k":
        f16(2e-5, 6e-5, 208)
    elif fmt == "mxfp4":
        rec[:, :, 0] = rng.integers(118, 123, size=(n, nrec), dtype=np.uint8)
    elif fmt == "nvfp4":
        rec[:, :, 0:4] = rng.integers(0x20, 0x40, size=(n, nrec, 4), dtype=np.uint8)
    return rec.reshape(n, -1)


def ggml_tables() -> dict:
    """The lookup tables the ABI passes to IQ2_XXS / IQ2_XS / MXFP4 / NVFP4
    kernels: grids from the GGML table fixture (ggml-common.h's text), the
    rest from their definitions."""
    with open(os.path.join(ROOT, "tests", "golden", "ggml_tables.json")) as f:
        t = json.load(f)
    grid = np.array([int(h, 16) for h in t["iq2xxs_grid"]], np.uint64).view(np.int8)
    grid_xs = np.array([int(h, 16) for h in t["iq2xs_grid"]], np.uint64).view(np.int8)
    ks = np.array(t["ksigns_iq2xs"], np.int64)
    signs = np.where((ks[:, None] >> np.arange(8)[None, :]) & 1, -1, 1).astype(np.int8).reshape(-1)
    kv = np.array(t["kvalues_mxfp4"], np.int8)
    e = np.arange(256, dtype=np.uint32)
    e8m0 = np.where(e < 2, np.uint32(0x00200000) << e, (e - 1) << 23).astype(np.uint32).view(np.float32)
    c = np.arange(256)
    ex, mant = (c >> 3) & 15, c & 7
    ue4m3 = np.where(ex == 0, mant / 1024.0, (8 + mant) * np.ldexp(1.0, ex.astype(np.int32) - 11)).astype(np.float32)
    ue4m3[[0, 0x7F]] = 0.0
    return {"iq2_xxs": [grid, signs], "iq2_xs": [grid_xs, signs], "mxfp4": [kv, e8m0], "nvfp4": [kv, ue4m3]}


def profiled_traffic(name: str):
    """HBM bytes per launch measured by the FETCH_SIZE / WRITE_SIZE counter
    runs recorded in profiles/<name>.md (scaled against a known-size copy),
    or None when no such profile is committed."""
    path = os.path.join(ROOT, "profiles", name + ".md")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def cpu_model() -> str:
    """The host CPU's identity as /proc/cpuinfo gives it (model name, family,
    model and stepping, clock, whether AVX-512 is present)."""
    fields = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if not line.strip():
                    break  # the first processor's block
                key, _, val = line.partition(":")
                fields[key.strip()] = val.strip()
    except OSError:
        return platform.processor() or "unknown"
    name = fields.get("model name", platform.processor() or "unknown")
    ident = "/".join(fields.get(k, "?") for k in ("cpu family", "model", "stepping"))
    avx512 = "avx512f" in fields.get("flags", "").split()
    mhz = fields.get("cpu MHz")
    return f"{name} (family/model/stepping {ident}{', ' + mhz + ' MHz' if mhz else ''}, avx512f {'yes' if avx512 else 'no'})"


class Bench:
    def __init__(self):
        import torch

        from weft_amd import _lib
        self.torch = torch
        self.lib = _lib.load()
        self._lib = _lib
        self.dev = torch.device("cuda:0")
        self.stream = torch.cuda.current_stream()
        _lib.set_stream(self.stream.cuda_stream)
        self.tables = {fmt: [self.dev_copy(a) for a in arrs] for fmt, arrs in ggml_tables().items()}
        self.flush_buf = None

    def dev_copy(self, a: np.ndarray):
        return self.torch.from_numpy(np.ascontiguousarray(a)).to(self.dev)

    def q8k(self, x: np.ndarray):
        """Q8_K records of the rows of x, by the library's q8_K_quantize."""
        m, k = x.shape
        xd = self.dev_copy(x)
        out = self.torch.empty(record_bytes("q8_k", k) * m, dtype=self.torch.uint8, device=self.dev)
        self.lib.q8_K_quantize(xd.data_ptr(), out.data_ptr(), m * k)
        self.torch.cuda.synchronize()
        self._lib.check("q8_K_quantize")
        return out

    def events(self):
        return (self.torch.cuda.Event(enable_timing=True), self.torch.cuda.Event(enable_timing=True))

    def time_calls(self, launch, steps, warmup, windows=WINDOWS):
        """launch(i) enqueues call i.  After `warmup` calls, `windows` windows
        of `steps` back-to-back calls, each between two HIP events on the
        library's stream with a synchronize on both sides; returns the
        seconds per call of the median, fastest and slowest window."""
        torch = self.torch
        for i in range(warmup):
            launch(i)
        torch.cuda.synchronize()
        self._lib.check("warmup")
        per, i = [], warmup
        for _ in range(windows):
            start, end = self.events()
            torch.cuda.synchronize()
            start.record(self.stream)
            for _ in range(steps):
                launch(i)
                i += 1
            end.record(self.stream)
            torch.cuda.synchronize()
            per.append(start.elapsed_time(end) / 1e3 / steps)
        self._lib.check("timed region")
        return statistics.median(per), min(per), max(per)

    def time_cold(self, launch, reps=20):
        """Median seconds of one call after the caches are flushed by writing
        FLUSH_BYTES (BASELINE.md's headline protocol)."""
        torch = self.torch
        if self.flush_buf is None:
            self.flush_buf = torch.empty(FLUSH_BYTES // 4, dtype=torch.float32, device=self.dev)
        times = []
        for i in range(reps):
            self.flush_buf.fill_(float(i))
            start, end = self.events()
            start.record(self.stream)
            launch(i)
            end.record(self.stream)
            torch.cuda.synchronize()
            times.append(start.elapsed_time(end) / 1e3)
        self._lib.check("cold calls")
        return statistics.median(times)

    def time_graph(self, launch, calls=20, replays=5):
        """Seconds per call when `calls` back-to-back calls are replayed from
        one captured HIP graph."""
        torch = self.torch
        side = torch.cuda.Stream()
        side.wait_stream(self.stream)
        g = torch.cuda.CUDAGraph()
        try:
            with torch.cuda.stream(side):
                self._lib.set_stream(side.cuda_stream)
                with torch.cuda.graph(g, stream=side):
                    for i in range(calls):
                        launch(i)
        finally:
            self._lib.set_stream(self.stream.cuda_stream)
        self._lib.check("graph capture")
        g.replay()
        torch.cuda.synchronize()
        start, end = self.events()
        start.record(self.stream)
        for _ in range(replays):
            g.replay()
        end.record(self.stream)
        torch.cuda.synchronize()
        self._lib.check("graph replay")
        return start.elapsed_time(end) / 1e3 / (calls * replays)

    def floors(self, nbytes_list, sweep_bytes, write_list=()):
        """Per-launch floors on this stream: an empty kernel back to back, and
        the fastest single streaming-read launch of each byte count.  For
        sweep_bytes the read probe is swept over every shape it has (threads
        per workgroup, 16-byte loads in flight per lane, nontemporal or not,
        grid-stride or one contiguous chunk per workgroup) and grid size; the
        other byte counts try the five best shapes of that sweep.  The best
        shape is then timed like a case (median of the windows).  For each
        of write_list (a write-bound case's output bytes) the write probe is
        swept the same way (1, 2 or 4 stores in flight per lane)."""
        torch = self.torch
        lib = self.lib
        out = {"empty_launch_us": round(self.time_calls(lambda i: lib.weft_hip_probe_empty(), 100, 20)[0] * 1e6, 3)}
        sink = torch.empty(1 << 16, dtype=torch.int32, device=self.dev)
        shapes = [(t, u, f) for t in (256, 512, 1024) for u in (1, 2, 4, 8, 16) for f in (0, 1, 2, 3)]
        grids = (256, 512, 1024, 2048)
        reads, ranked = {}, None
        for nbytes in sorted(nbytes_list, key=lambda nb: nb != sweep_bytes):
            n16 = (nbytes + 15) // 16 * 16
            copies = max(2, int(np.ceil(2 * MALL_BYTES / n16)) + 1)
            bufs = [torch.zeros(n16, dtype=torch.uint8, device=self.dev) for _ in range(copies)]
            tried = []
            for shape in (shapes if ranked is None else ranked[:5]):
                for grid in grids:
                    t, u, f = shape
                    sec = self.time_calls(lambda i: lib.weft_hip_probe_read_shape(
                        bufs[i % copies].data_ptr(), n16, sink.data_ptr(), grid, t, u, f), 20, 5, windows=3)[0]
                    tried.append((sec, shape, grid))
            tried.sort()
            if ranked is None:
                ranked = list(dict.fromkeys(shape for _, shape, _ in tried))
            _, (t, u, f), grid = tried[0]
            sec = self.time_calls(lambda i: lib.weft_hip_probe_read_shape(
                bufs[i % copies].data_ptr(), n16, sink.data_ptr(), grid, t, u, f), 50, 10)[0]
            reads[str(nbytes)] = {"us": round(sec * 1e6, 3), "GBs": round(nbytes / sec / 1e9, 1),
                                  "grid": grid, "threads": t, "unroll": u, "nontemporal": bool(f & 1),
                                  "blocked": bool(f & 2), "launch_shapes_tried": len(tried)}
            del bufs
            torch.cuda.empty_cache()
        out["stream_read"] = reads
        writes = {}
        for nbytes in write_list:
            n16 = (nbytes + 15) // 16 * 16
            copies = max(2, int(np.ceil(2 * MALL_BYTES / n16)) + 1)
            bufs = [torch.empty(n16, dtype=torch.uint8, device=self.dev) for _ in range(copies)]
            tried = []
            for t in (256, 512, 1024):
                for u in (1, 2, 4):
                    for f in (0, 1, 2, 3):
                        for grid in grids:
                            sec = self.time_calls(lambda i: lib.weft_hip_probe_write_shape(
                                bufs[i % copies].data_ptr(), n16, grid, t, u, f), 10, 3, windows=3)[0]
                            tried.append((sec, (t, u, f), grid))
            tried.sort()
            _, (t, u, f), grid = tried[0]
            sec = self.time_calls(lambda i: lib.weft_hip_probe_write_shape(
                bufs[i % copies].data_ptr(), n16, grid, t, u, f), 20, 5)[0]
            writes[str(nbytes)] = {"us": round(sec * 1e6, 3), "GBs": round(nbytes / sec / 1e9, 1),
                                   "grid": grid, "threads": t, "unroll": u, "nontemporal": bool(f & 1),
                                   "blocked": bool(f & 2), "launch_shapes_tried": len(tried)}
            del bufs
            torch.cuda.empty_cache()
        out["stream_write"] = writes
        out["mfma_valu_ns_per_mfma"] = self.mfma_probe()
        return out

    def mfma_probe(self):
        """ns per v_mfma_i32_32x32x32_i8 per SIMD with V independent VALU
        instructions issued after each MFMA, at 1 and 2 waves per SIMD
        (library probe weft_hip_probe_mfma): how much VALU work hides beside
        the matrix pipe.  The prefill GEMMs issue 9-38 VALU per MFMA."""
        torch = self.torch
        sink = torch.empty(1 << 18, dtype=torch.int32, device=self.dev)
        iters = 2000
        res = {}
        for waves in (1, 2):
            for v in (0, 4, 8, 12, 16):
                sec = self.time_calls(lambda i: self.lib.weft_hip_probe_mfma(v, waves, iters, sink.data_ptr()),
                                      3, 2, windows=3)[0]
                res[f"w{waves}_v{v}"] = round(sec * 1e9 / (2 * iters * waves), 2)
        return res

    def vendor_int8_gemm(self, m, n, k):
        """hipBLASLt's plain int8 GEMM (torch._int_mm) of the same shape:
        seconds per call, back to back."""
        torch = self.torch
        a = torch.randint(-127, 128, (m, k), dtype=torch.int8, device=self.dev)
        b = torch.randint(-127, 128, (n, k), dtype=torch.int8, device=self.dev).t()
        try:
            for _ in range(3):
                torch._int_mm(a, b)
            torch.cuda.synchronize()
            per = []
            for _ in range(WINDOWS):
                start, end = self.events()
                start.record(self.stream)
                for _ in range(20):
                    torch._int_mm(a, b)
                end.record(self.stream)
                torch.cuda.synchronize()
                per.append(start.elapsed_time(end) / 1e3 / 20)
            return statistics.median(per)
        except RuntimeError:
            return None


def run_case(b: Bench, name: str, steps: int, warmup: int, extra: bool) -> dict:
    """Time one case; returns its figures (algorithmic bytes / ops, rate, roofline fraction)."""
    sym, fmt, n, k, m, bound = CASES[name]
    w = synthetic_weights(fmt, n, k)
    torch = b.torch
    copies = max(2, int(np.ceil(2 * MALL_BYTES / w.nbytes)) + 1)
    fn = getattr(b.lib, sym)
    if sym == "weft_ggml_mul_mat_id":
        # expert matrices copied from one quantized matrix (the timing does
        # not depend on the values); the expert set itself is rotated
        from weft_amd import ggml as G
        bank = b.dev_copy(np.concatenate([w] * MOE_EXPERTS))
        copies = max(2, int(np.ceil(2 * MALL_BYTES / bank.numel())) + 1)
        wd = [bank] + [bank.clone() for _ in range(copies - 1)]
        rng = np.random.default_rng(3)
        ids_h = np.stack([rng.choice(MOE_EXPERTS, MOE_USED, replace=False) for _ in range(m)]).astype(np.int32)
        ids = b.dev_copy(ids_h)
        x = b.dev_copy(seeded_normal(2, (m, k)))
        y = torch.empty(m * MOE_USED * n, dtype=torch.float32, device=b.dev)
        s1 = G.tensor(G.F32, (k, 1, m), x.data_ptr())
        it = G.tensor(G.I32, (MOE_USED, m), ids.data_ptr())
        d = G.tensor(G.F32, (n, MOE_USED, m), y.data_ptr())
        s0s = [G.tensor(G.Q4_K, (k, n, MOE_EXPERTS), t.data_ptr()) for t in wd]
        wsize = G.mul_mat_id_work_size(s0s[0], s1, it)
        work = torch.empty(wsize, dtype=torch.uint8, device=b.dev)

        def launch(i):
            G.mul_mat_id(s0s[i % copies], s1, it, d, work.data_ptr(), wsize)

        nbytes = MOE_EXPERTS * w.nbytes + 4 * m * k + record_bytes("q8_k", k) * m + 4 * m * MOE_USED * n
        m *= MOE_USED  # products: one per (token, expert) pair
    elif sym == "weft_ggml_mul_mat":
        from weft_amd import ggml as G
        wd = [b.dev_copy(w) for _ in range(copies)]
        xq = b.q8k(seeded_normal(2, (m, k)))
        y = torch.empty(m * n, dtype=torch.float32, device=b.dev)
        s0s = [G.tensor(G.Q4_K, (k, n), t.data_ptr()) for t in wd]
        s1 = G.tensor(G.Q8_K, (k, m), xq.data_ptr())
        d = G.tensor(G.F32, (n, m), y.data_ptr())

        def launch(i):
            G.mul_mat(s0s[i % copies], s1, d)

        nbytes = w.nbytes + xq.numel() + 4 * m * n
    else:
        wd = [b.dev_copy(w) for _ in range(copies)]
        if m == 0:  # row dequantize of the whole matrix
            # write-bound: the outputs rotate too, past the Infinity Cache,
            # so that no call writes into lines a previous call left cached
            ycopies = max(2, int(np.ceil(2 * MALL_BYTES / (4 * n * k))) + 1)
            ys = [torch.empty(n * k, dtype=torch.float32, device=b.dev) for _ in range(ycopies)]
            y = ys[0]

            def launch(i):
                fn(wd[i % copies].data_ptr(), ys[i % ycopies].data_ptr(), n * k)

            def launch_one_output(i):
                fn(wd[i % copies].data_ptr(), y.data_ptr(), n * k)

            nbytes = w.nbytes + 4 * n * k
        elif m < 0:  # GEMV over the Q4K_I[16] layout: pack every copy once, outside the timing
            packed = [torch.empty_like(t) for t in wd]
            pack = getattr(b.lib, sym + "_W_pack")
            for src, dst in zip(wd, packed):
                pack(src.data_ptr(), dst.data_ptr(), n, k)
            torch.cuda.synchronize()
            b._lib.check(sym + "_W_pack")
            wd = packed
            xq = b.q8k(seeded_normal(2, (1, k)))
            y = torch.empty(n, dtype=torch.float32, device=b.dev)

            def launch(i):
                fn(wd[i % copies].data_ptr(), xq.data_ptr(), y.data_ptr(), n, k)

            nbytes = w.nbytes + xq.numel() + 4 * n
        elif sym.endswith("_persistent"):  # Q4K_I[16] weights, shapes in the artifact's order M, K, N
            packed = [torch.empty_like(t) for t in wd]
            pack = getattr(b.lib, sym + "_W_pack")
            for src, dst in zip(wd, packed):
                pack(src.data_ptr(), dst.data_ptr(), n, k)
            torch.cuda.synchronize()
            b._lib.check(sym + "_W_pack")
            wd = packed
            x = b.dev_copy(seeded_normal(2, (m, k)))
            xq = torch.empty(record_bytes("q8_k", k) * m, dtype=torch.uint8, device=b.dev)
            y = torch.empty(m * n, dtype=torch.float32, device=b.dev)

            def launch(i):
                fn(wd[i % copies].data_ptr(), x.data_ptr(), xq.data_ptr(), y.data_ptr(), m, k, n)

            nbytes = w.nbytes + 4 * m * k + xq.numel() + 4 * m * n
        else:
            act = ACT_OF.get(fmt, "q8_k")
            x = b.dev_copy(seeded_normal(2, (m, k)))
            xq = torch.empty(record_bytes(act, k) * m, dtype=torch.uint8, device=b.dev)
            y = torch.empty(m * n, dtype=torch.float32, device=b.dev)
            tabs = [t.data_ptr() for t in b.tables.get(fmt, [])]

            def launch(i):
                fn(wd[i % copies].data_ptr(), x.data_ptr(), xq.data_ptr(), *tabs, y.data_ptr(), n, k, m)

            nbytes = w.nbytes + 4 * m * k + xq.numel() + 4 * m * n
    warmup = max(3, warmup if bound == "hbm" else warmup // 4)
    b._lib.launch_log()
    launch(0)
    torch.cuda.synchronize()
    log = b._lib.launch_log()
    kernels = [f"{k} x{log.count(k)}" if log.count(k) > 1 else k for k in dict.fromkeys(log)]
    sec, lo, hi = b.time_calls(launch, steps, warmup)
    out = {"symbol": sym, "N": n, "K": k, "M": max(m, 1) if m < 0 else m, "us": round(sec * 1e6, 3),
           "us_min": round(lo * 1e6, 3), "us_max": round(hi * 1e6, 3),
           "algorithmic_bytes": int(nbytes), "GBs": round(nbytes / sec / 1e9, 2),
           "weight_copies_rotated": copies, "kernels": kernels}
    if m == 0:
        out["write_bytes"] = 4 * n * k  # the fp32 rows written
        out["output_copies_rotated"] = ycopies
        # the same calls writing one output buffer (180 MB at config 2, part
        # of which the Infinity Cache keeps between calls)
        out["one_output_us"] = round(b.time_calls(launch_one_output, steps, warmup)[0] * 1e6, 3)
    if extra:
        out["cold_us"] = round(b.time_cold(launch) * 1e6, 3)
        out["graph_us"] = round(b.time_graph(launch) * 1e6, 3)
    if bound == "hbm":
        out["frac_hbm_peak"] = round(nbytes / sec / 1e9 / HBM_PEAK_GBS, 4)
    else:
        ops = 2.0 * m * n * k
        tops = ops / sec / 1e12
        out.update({"ops": int(ops), "TOPS": round(tops, 2)})
        if fmt == "mxfp4":
            # fp4 weights x fp8 activation planes on the block-scaled MFMA
            out["frac_fp8_rate"] = round(tops / FP8_PEAK_TOPS, 4)
            out["frac_fp4_peak"] = round(tops / FP4_PEAK_TOPS, 4)
        else:
            out["frac_int8_peak"] = round(tops / INT8_PEAK_TOPS, 4)
        if extra and sym != "weft_ggml_mul_mat_id":
            vs = b.vendor_int8_gemm(m, n, k)
            if vs is not None:
                out["vendor_int8_gemm_us"] = round(vs * 1e6, 3)
                out["vendor_int8_gemm_TOPS"] = round(ops / vs / 1e12, 2)
    del wd
    torch.cuda.empty_cache()
    return out


def cpu_baseline(n, k, budget_s):
    """GGML's MUL_MAT restated in oracle/ on the headline call: all threads
    with GGML's schedule for ~budget_s, then one thread under the reference's
    kernel protocol."""
    import oracle as o
    build = o.use_native()
    w = o.quantize("q4_k", o.seeded_normal(1, (n, k), 0.02))
    x = o.seeded_normal(2, (1, k))
    nbytes = w.nbytes + 4 * k + (k // 256) * 292 + 4 * n
    threads = o.max_threads()
    xq = np.zeros((1, o.record_bytes("q8_k", k)), np.uint8)
    y = np.empty((1, n), np.float32)
    o.mul_mat_ggml("q4_k", w, x, n, k, 1, threads=threads, xq=xq, y=y)  # warmup
    reps, t0 = 0, time.perf_counter()
    while True:
        o.mul_mat_ggml("q4_k", w, x, n, k, 1, threads=threads, xq=xq, y=y)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s or reps >= 100000:
            break
    per = el / reps
    # single thread: 1 warmup, 64 MiB eviction before each of 10 timed calls, median
    evict = np.zeros(64 << 20, np.uint8)
    o.mul_mat_ggml("q4_k", w, x, n, k, 1, threads=1, xq=xq, y=y)
    singles = []
    for _ in range(10):
        o.evict(evict)
        t = time.perf_counter()
        o.mul_mat_ggml("q4_k", w, x, n, k, 1, threads=1, xq=xq, y=y)
        singles.append(time.perf_counter() - t)
    one = statistics.median(singles)
    return {"value": round(nbytes / per / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{reps} full decode calls (N={n}, K={k}, M=1) in {el:.1f} s, {per * 1e3:.3f} ms/call, "
                      f"GGML's MUL_MAT thread schedule over {threads} host threads",
            "single_thread": {"us": round(one * 1e6, 1), "GBs": round(nbytes / one / 1e9, 3),
                              "protocol": "1 warmup, 64 MiB eviction before each of 10 calls, median"},
            "cpu_model": cpu_model(), "nproc": os.cpu_count(), "build": "gcc " + build}


def brief(case: dict) -> dict:
    """The figures of an adjacent-format case kept in the output line."""
    keep = ("us", "GBs", "TOPS", "frac_hbm_peak", "frac_int8_peak", "vs_read_floor")
    return {k: case[k] for k in keep if k in case}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; multi-GPU figures are not part of it "
                                   "(--gpus must be 1)", "n_gpus": args.gpus}))
        sys.exit(2)
    b = Bench()
    steps, warmup = args.steps, args.warmup
    extra = not args.no_extra

    head = run_case(b, HEADLINE, steps, warmup, extra)
    sec = head["us"] / 1e6
    gbs = head["GBs"]
    if args.cases == "all":
        names = [c for c in CASES if c != HEADLINE]
    elif args.cases == "none":
        names = []
    else:
        names = [c for c in args.cases.split(",") if c]
    results = {HEADLINE: head}
    results.update({name: run_case(b, name, steps, warmup, extra) for name in names})
    floors = None
    if extra:
        byte_counts = sorted({v["algorithmic_bytes"] for v in results.values() if v.get("frac_hbm_peak")})
        write_counts = sorted({v["write_bytes"] for v in results.values() if v.get("write_bytes")})
        floors = b.floors(byte_counts, head["algorithmic_bytes"], write_counts)
        for v in results.values():
            read = floors["stream_read"].get(str(v["algorithmic_bytes"])) if v.get("frac_hbm_peak") else None
            if read is not None:
                v["read_floor_us"] = read["us"]
                v["vs_read_floor"] = round(v["us"] / read["us"], 3)
            write = floors["stream_write"].get(str(v.get("write_bytes")))
            if write is not None:
                v["write_floor_us"] = write["us"]
                v["vs_write_floor"] = round(v["us"] / write["us"], 3)
    if args.calibrate_copy:
        nb = args.calibrate_copy << 20
        src = b.torch.empty(nb, dtype=b.torch.uint8, device=b.dev)
        dst = b.torch.empty_like(src)
        b.torch.cuda.synchronize()
        dst.copy_(src)
        b.torch.cuda.synchronize()
    cpu = None
    if not args.no_cpu:
        # a reported baseline only: a failure here must not lose the GPU line
        try:
            cpu = cpu_baseline(11008, 4096, args.cpu_seconds)
        except Exception as e:  # noqa: BLE001
            cpu = {"value": None, "unit": "GB/s", "error": f"{type(e).__name__}: {e}"[:300]}

    roofline = {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": profiled_traffic("q4k_decode_w_up"),
                "algorithmic_bytes": head["algorithmic_bytes"],
                "kernel": head["kernels"][0] if len(head["kernels"]) == 1 else ",".join(head["kernels"])}
    if floors is not None:
        read = floors["stream_read"][str(head["algorithmic_bytes"])]
        roofline["floor"] = {"empty_launch_us": floors["empty_launch_us"], "stream_read_us": read["us"],
                             "stream_read_frac": round(read["GBs"] / HBM_PEAK_GBS, 4),
                             "kernel_vs_read": round(head["us"] / read["us"], 3)}
    labels = {case: label for label, case in BASELINE_CASES.items()}
    line = {
        "metric": "Q4_K mul_mat: decode GB/s (% of 8 TB/s) + prefill TOPS (% int8 MFMA peak)",
        "value": gbs,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(sec * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (weight records of random payload bytes with scale fields at the magnitudes "
                "an N(0,0.02) matrix quantizes to; seeded N(0,1) activations)",
        "config": {"workload": "production_mul_mat_q4_k_decode, config 3 W_up: N=11008 K=4096 "
                               "M=1, Q8_K activation quantize inside the timed call",
                   "N": 11008, "K": 4096, "M": 1,
                   "weight_copies_rotated": head["weight_copies_rotated"],
                   "timing": f"median of {WINDOWS} windows of {steps} back-to-back calls (HIP events)"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "floors": None if floors is None else {
            "empty_launch_us": floors["empty_launch_us"],
            "stream_read_headline": floors["stream_read"][str(head["algorithmic_bytes"])],
            "stream_read_us": {k: v["us"] for k, v in floors["stream_read"].items()},
            "stream_write": floors["stream_write"],
            "mfma_valu_ns_per_mfma": floors["mfma_valu_ns_per_mfma"]},
        "adjacent": {name: brief(v) for name, v in results.items() if name not in labels},
        "configs": {labels[name]: results[name] for name in CASES if name in labels and name in results},
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
