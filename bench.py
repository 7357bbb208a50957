#!/usr/bin/env python3
"""Benchmark of the quantized mul_mat hot path on one MI355X.

Headline (BASELINE.json metric "Q4_K mul_mat: decode GB/s (% of 8 TB/s) +
prefill TOPS (% int8 MFMA peak)"): one step = one production_mul_mat_q4_k_decode
call on config 3's W_up shape (N=11008, K=4096, M=1), Q8_K activation quantize
included, exactly as the reference's timed mul_mat (weft-kernel-performance.csv:59).
``value`` is the algorithmic HBM bytes of the call (encoded W + fp32 X + Xq
write + fp32 Y = 25,427,520 B) divided by the measured time per call, in GB/s.

Inputs are seeded synthetic data (W ~ N(0, 0.02^2) quantized with the GGML
Q4_K reference quantizer restated in oracle/, X ~ N(0, 1)) resident in HBM
before timing.  W is rotated over enough copies (> 2 x the 256 MB Infinity
Cache) that every call streams its weights from HBM.  The timed region is K
back-to-back calls on one stream between two HIP events, bracketed by device
synchronisation.  Secondary lines time W_down (4096 x 11008) and the Q4_K
prefill entry point (config 4, M=512).

The CPU baseline is oracle/'s restatement of GGML's generic MUL_MAT path
(quantize_row_q8_K_ref + ggml_vec_dot_q4_K_q8_K_generic, rows over OpenMP
threads), timed on this host on the same decode workload.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
MALL_BYTES = 256 << 20


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--cpu-seconds", type=float, default=10.0,
                   help="wall-clock budget of the CPU baseline sample")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--no-prefill", action="store_true")
    p.add_argument("--no-wdown", action="store_true")
    p.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                   help="also run one plain device-to-device copy of MIB MiB, the known-size "
                        "kernel that HBM byte counters are scaled against")
    return p.parse_args()


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


def algorithmic_bytes(n, k, m, w_bytes):
    xq = m * (k // 256) * 292
    return w_bytes + 4 * m * k + xq + 4 * m * n


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

    def dev_copy(self, a: np.ndarray):
        return self.torch.from_numpy(np.ascontiguousarray(a)).to(self.dev)

    def time_calls(self, launch, steps, warmup):
        """launch(i) enqueues call i; returns seconds per call over `steps`."""
        torch = self.torch
        for i in range(warmup):
            launch(i)
        torch.cuda.synchronize()
        self._lib.check("warmup")
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record(self.stream)
        for i in range(steps):
            launch(warmup + i)
        end.record(self.stream)
        torch.cuda.synchronize()
        self._lib.check("timed region")
        return start.elapsed_time(end) / 1e3 / steps


def q4k_weights(n, k, seed):
    import oracle as o
    return o.quantize("q4_k", o.seeded_normal(seed, (n, k), 0.02))


def decode_case(b, n, k, steps, warmup):
    import oracle as o
    w = q4k_weights(n, k, 1)
    copies = max(2, int(np.ceil(2 * MALL_BYTES / w.nbytes)) + 1)
    wd = [b.dev_copy(w) for _ in range(copies)]
    x = b.dev_copy(o.seeded_normal(2, (1, k)))
    xq = b.torch.empty((k // 256) * 292, dtype=b.torch.uint8, device=b.dev)
    y = b.torch.empty(n, dtype=b.torch.float32, device=b.dev)
    fn = b.lib.production_mul_mat_q4_k_decode

    def launch(i):
        fn(wd[i % copies].data_ptr(), x.data_ptr(), xq.data_ptr(), y.data_ptr(), n, k, 1)

    sec = b.time_calls(launch, steps, warmup)
    nbytes = algorithmic_bytes(n, k, 1, w.nbytes)
    del wd
    b.torch.cuda.empty_cache()
    return sec, nbytes, copies


def prefill_case(b, n, k, m, steps, warmup):
    import oracle as o
    w = b.dev_copy(q4k_weights(n, k, 1))
    x = b.dev_copy(o.seeded_normal(2, (m, k)))
    xq = b.torch.empty(m * (k // 256) * 292, dtype=b.torch.uint8, device=b.dev)
    y = b.torch.empty(m * n, dtype=b.torch.float32, device=b.dev)
    fn = b.lib.production_mul_mat_q4_k_staged

    def launch(i):
        fn(w.data_ptr(), x.data_ptr(), xq.data_ptr(), y.data_ptr(), n, k, m)

    sec = b.time_calls(launch, steps, warmup)
    return sec, 2.0 * m * n * k


def cpu_baseline(n, k, budget_s):
    import oracle as o
    w = q4k_weights(n, k, 1)
    x = o.seeded_normal(2, (1, k))
    threads = o.max_threads()
    o.mul_mat("q4_k", w, x, n, k, 1, threads=threads)  # warmup
    reps, t0 = 0, time.perf_counter()
    while True:
        o.mul_mat("q4_k", w, x, n, k, 1, threads=threads)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s or reps >= 100000:
            break
    per = el / reps
    gbs = algorithmic_bytes(n, k, 1, w.nbytes) / per / 1e9
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{reps} full decode calls (N={n}, K={k}, M=1) in {el:.1f} s, "
                      f"{per * 1e3:.3f} ms/call, OpenMP over {threads} host threads"}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    b = Bench()
    steps, warmup = args.steps, args.warmup

    sec, nbytes, copies = decode_case(b, 11008, 4096, steps, warmup)
    gbs = nbytes / sec / 1e9
    sec_dn = nbytes_dn = None
    if not args.no_wdown:
        sec_dn, nbytes_dn, _ = decode_case(b, 4096, 11008, steps, warmup)
    if args.calibrate_copy:
        n = args.calibrate_copy << 20
        src = b.torch.empty(n, dtype=b.torch.uint8, device=b.dev)
        dst = b.torch.empty_like(src)
        b.torch.cuda.synchronize()
        dst.copy_(src)
        b.torch.cuda.synchronize()
    prefill = {}
    if not args.no_prefill:
        for n in (4096, 11008):
            psec, ops = prefill_case(b, n, 4096, 512, max(3, steps // 20), 2)
            tops = ops / psec / 1e12
            prefill[f"N{n}"] = {"us": round(psec * 1e6, 2), "TOPS": round(tops, 3),
                                "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 5)}
    cpu = None if args.no_cpu else cpu_baseline(11008, 4096, args.cpu_seconds)

    line = {
        "metric": "Q4_K mul_mat: decode GB/s (% of 8 TB/s) + prefill TOPS (% int8 MFMA peak)",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(sec * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded N(0,0.02) weights quantized by the oracle's GGML Q4_K "
                "quantizer, N(0,1) activations)",
        "config": {"workload": "production_mul_mat_q4_k_decode, config 3 W_up: N=11008 K=4096 "
                               "M=1, Q8_K activation quantize inside the timed call",
                   "N": 11008, "K": 4096, "M": 1, "weight_copies_rotated": copies},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": profiled_traffic("q4k_decode_w_up"),
                     "algorithmic_bytes": nbytes},
        "cpu_baseline": cpu,
        "w_down": None if sec_dn is None else {
            "N": 4096, "K": 11008, "us": round(sec_dn * 1e6, 3),
            "GBs": round(nbytes_dn / sec_dn / 1e9, 2)},
        "prefill_q4_k_M512_K4096": prefill,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
