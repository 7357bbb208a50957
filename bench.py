#!/usr/bin/env python3
"""Benchmark of the quantized mul_mat hot path on one MI355X.

Headline (BASELINE.json metric "Q4_K mul_mat: decode GB/s (% of 8 TB/s) +
prefill TOPS (% int8 MFMA peak)"): one step = one production_mul_mat_q4_k_decode
call on config 3's W_up shape (N=11008, K=4096, M=1), Q8_K activation quantize
included, exactly as the reference's timed mul_mat (weft-kernel-performance.csv:59).
``value`` is the algorithmic HBM bytes of the call (encoded W + fp32 X + Xq
write + fp32 Y = 25,427,520 B) divided by the measured time per call, in GB/s.

Inputs are seeded synthetic data (weights ~ N(0, 0.02^2) quantized with the
GGML reference quantizers restated in oracle/, activations ~ N(0, 1)) resident
in HBM before timing.  For the HBM-bound decode cases the weights are rotated
over enough copies (> 2 x the 256 MB Infinity Cache) that every call streams
them from HBM.  A timed region is K back-to-back calls on the library's stream
between two HIP events, bracketed by device synchronisation.

Secondary figures (the other BASELINE.json configs) ride in the same JSON
line under ``configs``: W_down decode, the Q4_0 / IQ2_XXS / MXFP4 decode GEMVs,
the Q4_K row dequantize, and the prefill mul_mats (Q4_K config 4 at N=4096 and
N=11008, MXFP4 config 5b, Q4_0 and IQ2_XXS at the same shape), the latter
against the int8 MFMA peak, plus the derived Q4K_I[16] GEMV and GGML's
MUL_MAT_ID at a Mixtral-8x7B expert shape (ops counted per (token, expert)
pair).

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
    # adjacent format Q6_K (ggml-common.h:349-358) at the W_up shape; its
    # prefill entry runs the GEMV kernel (no MFMA form yet)
    "q6_k_decode": ("production_mul_mat_q6_k_decode", "q6_k", 11008, 4096, 1, "hbm"),
    "q6_k_prefill": ("production_mul_mat_q6_k", "q6_k", 4096, 4096, 512, "mfma"),
    # adjacent format Q5_K (ggml-common.h:330-345), decode at the W_up shape
    "q5_k_decode": ("production_mul_mat_q5_k_decode", "q5_k", 11008, 4096, 1, "hbm"),
    # adjacent format NVFP4 (ggml-common.h:211-217) at the W_up shape
    "nvfp4_decode": ("production_mul_mat_nvfp4_decode", "nvfp4", 11008, 4096, 1, "hbm"),
    # GGML MUL_MAT_ID (MoE) prefill at a Mixtral-8x7B FFN shape: 8 experts of
    # 14336 x 4096 Q4_K, 2 experts per token, 512 tokens (the grouped GEMM)
    "q4_k_moe_prefill": ("weft_ggml_mul_mat_id", "q4_k", 14336, 4096, 512, "mfma"),
}
MOE_EXPERTS, MOE_USED = 8, 2
HEADLINE = "q4_k_decode_w_up"


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--cpu-seconds", type=float, default=10.0,
                   help="wall-clock budget of the CPU baseline sample")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--cases", default="all",
                   help="comma-separated secondary cases to run (default all; 'none' for "
                        "the headline only): " + ",".join(c for c in CASES if c != HEADLINE))
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


class Bench:
    def __init__(self):
        import torch

        import oracle as o
        from weft_amd import _lib
        self.torch = torch
        self.lib = _lib.load()
        self._lib = _lib
        self.dev = torch.device("cuda:0")
        self.stream = torch.cuda.current_stream()
        _lib.set_stream(self.stream.cuda_stream)
        self.tables = {
            "iq2_xxs": [self.dev_copy(o.iq2xxs_grid().view(np.int8)), self.dev_copy(o.signs_i8x8())],
            "mxfp4": [self.dev_copy(o.kvalues_mxfp4()), self.dev_copy(o.e8m0_half_table())],
            "nvfp4": [self.dev_copy(o.kvalues_mxfp4()), self.dev_copy(o.ue4m3_table())],
        }

    def dev_copy(self, a: np.ndarray):
        return self.torch.from_numpy(np.ascontiguousarray(a)).to(self.dev)

    def time_calls(self, launch, steps, warmup):
        """launch(i) enqueues call i; returns seconds per call over `steps`,
        from two HIP events on the stream the library launches on."""
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


def run_case(b: Bench, name: str, steps: int, warmup: int) -> dict:
    """Time one case; returns its figures (algorithmic bytes / ops, rate, roofline fraction)."""
    import oracle as o
    sym, fmt, n, k, m, bound = CASES[name]
    w = o.quantize(fmt, o.seeded_normal(1, (n, k), 0.02))
    torch = b.torch
    copies = 1
    if bound == "hbm":  # stream the weights from HBM on every call
        copies = max(2, int(np.ceil(2 * MALL_BYTES / w.nbytes)) + 1)
    wd = [b.dev_copy(w) for _ in range(copies)]
    fn = getattr(b.lib, sym)
    if m == 0:  # row dequantize of the whole matrix
        y = torch.empty(n * k, dtype=torch.float32, device=b.dev)

        def launch(i):
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
        xq = b.dev_copy(o.quantize("q8_k", o.seeded_normal(2, (1, k))))
        y = torch.empty(n, dtype=torch.float32, device=b.dev)

        def launch(i):
            fn(wd[i % copies].data_ptr(), xq.data_ptr(), y.data_ptr(), n, k)

        nbytes = w.nbytes + xq.numel() + 4 * n
    elif sym == "weft_ggml_mul_mat_id":
        # one quantized expert matrix copied MOE_EXPERTS times (the timing
        # does not depend on the values); seeded top-MOE_USED choices per token
        from weft_amd import ggml as G
        experts = b.dev_copy(np.concatenate([w] * MOE_EXPERTS))
        del wd
        wd = [experts]
        rng = np.random.default_rng(3)
        ids_h = np.stack([rng.choice(MOE_EXPERTS, MOE_USED, replace=False) for _ in range(m)]).astype(np.int32)
        ids = b.dev_copy(ids_h)
        x = b.dev_copy(o.seeded_normal(2, (m, k)))
        y = torch.empty(m * MOE_USED * n, dtype=torch.float32, device=b.dev)
        s0 = G.tensor(G.Q4_K, (k, n, MOE_EXPERTS), experts.data_ptr())
        s1 = G.tensor(G.F32, (k, 1, m), x.data_ptr())
        it = G.tensor(G.I32, (MOE_USED, m), ids.data_ptr())
        d = G.tensor(G.F32, (n, MOE_USED, m), y.data_ptr())
        wsize = G.mul_mat_id_work_size(s0, s1, it)
        work = torch.empty(wsize, dtype=torch.uint8, device=b.dev)

        def launch(i):
            G.mul_mat_id(s0, s1, it, d, work.data_ptr(), wsize)

        nbytes = MOE_EXPERTS * w.nbytes + 4 * m * k + o.record_bytes("q8_k", k) * m + 4 * m * MOE_USED * n
        m *= MOE_USED  # products: one per (token, expert) pair
    else:
        act = o.ACT_OF[fmt]
        x = b.dev_copy(o.seeded_normal(2, (m, k)))
        xq = torch.empty(o.record_bytes(act, k) * m, dtype=torch.uint8, device=b.dev)
        y = torch.empty(m * n, dtype=torch.float32, device=b.dev)
        tabs = [t.data_ptr() for t in b.tables.get(fmt, [])]

        def launch(i):
            fn(wd[i % copies].data_ptr(), x.data_ptr(), xq.data_ptr(), *tabs, y.data_ptr(), n, k, m)

        nbytes = w.nbytes + 4 * m * k + xq.numel() + 4 * m * n
    if bound == "mfma":
        steps, warmup = max(3, steps // 20), 3
    sec = b.time_calls(launch, steps, warmup)
    del wd
    torch.cuda.empty_cache()
    out = {"symbol": sym, "N": n, "K": k, "M": max(m, 1) if m < 0 else m, "us": round(sec * 1e6, 3),
           "algorithmic_bytes": int(nbytes), "GBs": round(nbytes / sec / 1e9, 2),
           "weight_copies_rotated": copies, "steps": steps}
    if bound == "hbm":
        out["frac_hbm_peak"] = round(nbytes / sec / 1e9 / HBM_PEAK_GBS, 4)
    else:
        tops = 2.0 * m * n * k / sec / 1e12
        out.update({"ops": 2 * m * n * k, "TOPS": round(tops, 2),
                    "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4)})
    return out


def cpu_baseline(n, k, budget_s):
    import oracle as o
    w = o.quantize("q4_k", o.seeded_normal(1, (n, k), 0.02))
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
    nbytes = w.nbytes + 4 * k + (k // 256) * 292 + 4 * n
    return {"value": round(nbytes / per / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
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

    head = run_case(b, HEADLINE, steps, warmup)
    sec = head["us"] / 1e6
    gbs = head["GBs"]
    if args.cases == "all":
        names = [c for c in CASES if c != HEADLINE]
    elif args.cases == "none":
        names = []
    else:
        names = [c for c in args.cases.split(",") if c]
    secondary = {name: run_case(b, name, steps, warmup) for name in names}
    if args.calibrate_copy:
        n = args.calibrate_copy << 20
        src = b.torch.empty(n, dtype=b.torch.uint8, device=b.dev)
        dst = b.torch.empty_like(src)
        b.torch.cuda.synchronize()
        dst.copy_(src)
        b.torch.cuda.synchronize()
    cpu = None if args.no_cpu else cpu_baseline(11008, 4096, args.cpu_seconds)

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
        "data": "synthetic (seeded N(0,0.02) weights quantized by the oracle's GGML reference "
                "quantizers, N(0,1) activations)",
        "config": {"workload": "production_mul_mat_q4_k_decode, config 3 W_up: N=11008 K=4096 "
                               "M=1, Q8_K activation quantize inside the timed call",
                   "N": 11008, "K": 4096, "M": 1,
                   "weight_copies_rotated": head["weight_copies_rotated"]},
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": profiled_traffic("q4k_decode_w_up"),
                     "algorithmic_bytes": head["algorithmic_bytes"],
                     "kernel": "q4k_gemv_m1_kernel<1,1024,2>"},
        "cpu_baseline": cpu,
        "configs": secondary,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
