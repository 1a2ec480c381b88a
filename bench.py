#!/usr/bin/env python3
"""Benchmark of the quantized GGML matmul hot path on one MI355X.

Headline (BASELINE.json metric): Q4_0 x Q8_1 GEMM TOPS at M=2048 (N = K = 4096),
with the decode GEMV's HBM GB/s at M=1 (N = K = 4096) reported beside it.

A "step" is one pass of the hot path over one batch: gemm_w4a32c8_q4_0_fp32_int8
on fp32 activations [2048, 4096] (quantize_q8_1 + the int8-MFMA GEMM), output
fp32 [2048, 4096].  Inputs are seeded synthetic tensors resident in HBM before
timing; the weights and activations rotate over several copies so successive
steps do not hit the 256 MB MALL on one buffer.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu-baseline]

Prints ONE JSON line.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [ROOT, os.path.join(ROOT, "k-search_amd")]

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, published
INT8_PEAK_TOPS = 5000.0      # MI355X dense int8 MFMA, published


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def time_events(fn, iters: int) -> float:
    """Average ms per call of fn() over iters calls, HIP events on torch's current stream."""
    import torch
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    s.record()
    for i in range(iters):
        fn(i)
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / iters


def cpu_baseline(M: int, N: int, K: int, rows: int, threads: int) -> dict:
    """The reference CPU path (quantize_row_q8_1_ref + gemm_w4a8_reference order) timed on
    `rows` activation rows of the workload with `threads` OpenMP threads."""
    import numpy as np
    from ksq import synth
    from oracle import oracle
    g = synth.rng(1)
    w = synth.weights(0, g, N, K)
    x = synth.activations(g, rows, K)
    t0 = time.perf_counter()
    a = oracle.quantize_q8_1(x)
    oracle.gemm(0, a, w, rows, N, K, nthreads=threads)
    dt = time.perf_counter() - t0
    return {"value": round(2.0 * rows * N * K / dt / 1e12, 6), "unit": "TOPS", "cores": threads,
            "kind": "port",
            "sample": f"{rows} of {M} activation rows (N=K={K}), quantize_row_q8_1_ref + gemm_w4a8_reference "
                      f"order, {dt:.1f} s with {threads} thread(s)"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build runs the quantized matmul path on a single "
              "MI355X (no collectives); run with --gpus 1", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    import ksq
    from ksq import ops, synth

    dev = torch.device("cuda:0")
    M, N, K = 2048, 4096, 4096
    copies = 8
    g = synth.rng(2024)
    log(f"bench: generating inputs M={M} N={N} K={K} x{copies} copies")
    w_np = synth.weights(ksq.W_Q4_0, g, N, K)
    x_np = synth.activations(g, M, K)
    W = [torch.from_numpy(w_np).to(dev) for _ in range(copies)]
    X = [torch.from_numpy(x_np).to(dev) for _ in range(copies)]
    out = torch.empty((M, N), dtype=torch.float32, device=dev)
    ws = torch.empty(ops.workspace_size(0, 0, M, N, K), dtype=torch.uint8, device=dev)
    AQ = [ops.quantize_q8_1(X[i]) for i in range(copies)]
    torch.cuda.synchronize()

    def step(i):
        ops.gemm(ksq.W_Q4_0, ksq.A_F32, W[i % copies], X[i % copies], M, N, K, out=out, workspace=ws)

    def gemm_only(i):
        ops.gemm(ksq.W_Q4_0, ksq.A_Q8_1, W[i % copies], AQ[i % copies], M, N, K, out=out)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    log(f"bench: timing {args.steps} steps")
    t0 = time.perf_counter()
    ms = time_events(step, args.steps)
    wall = (time.perf_counter() - t0) / args.steps * 1e3
    ops_per_step = 2.0 * M * N * K
    tops = ops_per_step / (ms * 1e-3) / 1e12

    gemm_ms = time_events(gemm_only, args.steps)
    gemm_tops = ops_per_step / (gemm_ms * 1e-3) / 1e12

    # ---- decode GEMV, config 0 shape, Q8_1 activations, 64 weight copies (600 MB > MALL)
    Mv, Nv, Kv = 1, 4096, 4096
    gcopies = 64
    wv_np = synth.weights(ksq.W_Q4_0, g, Nv, Kv)
    WV = [torch.from_numpy(wv_np).to(dev) for _ in range(gcopies)]
    xv = torch.from_numpy(synth.activations(g, Mv, Kv)).to(dev)
    aqv = ops.quantize_q8_1(xv)
    outv = torch.empty((Mv, Nv), dtype=torch.float32, device=dev)

    def gemv(i):
        ops.gemm(ksq.W_Q4_0, ksq.A_Q8_1, WV[i % gcopies], aqv, Mv, Nv, Kv, out=outv)

    for i in range(gcopies):
        gemv(i)
    gemv_ms = time_events(gemv, 4 * gcopies)
    gemv_bytes = Nv * (Kv // 32) * 18 + Mv * (Kv // 32) * 36 + Mv * Nv * 4
    gemv_gbs = gemv_bytes / (gemv_ms * 1e-3) / 1e9

    result = {
        "metric": "Q4_0×Q8_1 GEMM TOPS at M=2048; GEMV HBM GB/s at M=1 (N=K=4096)",
        "value": round(tops, 3),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded: Q4_0 nibbles U[0,15], d=|N(0,0.02)|; activations N(0,1))",
        "config": {"workload": "q4_0_q8_1_prefill_gemm", "M": M, "N": N, "K": K,
                   "entry": "gemm_w4a32c8_q4_0_fp32_int8 (quantize_q8_1 + int8 MFMA GEMM)",
                   "rotating_copies": copies, "wall_ms_per_step": round(wall, 4)},
        "roofline": {"bound": "mfma", "kernel": "mmq_kernel<0> (Q4_0 x Q8_1 int8 MFMA GEMM)",
                     "achieved": round(gemm_tops, 3), "peak": INT8_PEAK_TOPS, "unit": "TFLOP/s",
                     "frac": round(gemm_tops / INT8_PEAK_TOPS, 4), "traffic": None,
                     "avg_kernel_ms": round(gemm_ms, 5)},
        "gemv_m1": {"metric": "GEMV HBM GB/s at M=1 (N=K=4096)", "value": round(gemv_gbs, 1), "unit": "GB/s",
                    "avg_ms": round(gemv_ms, 5), "algorithmic_bytes": gemv_bytes,
                    "roofline": {"bound": "hbm", "achieved": round(gemv_gbs, 1), "peak": HBM_PEAK_GBS,
                                 "unit": "GB/s", "frac": round(gemv_gbs / HBM_PEAK_GBS, 4)},
                    "weight_copies": gcopies},
    }
    if not args.no_cpu_baseline:
        threads = min(16, os.cpu_count() or 1)
        log(f"bench: cpu baseline ({threads} threads)")
        result["cpu_baseline"] = cpu_baseline(M, N, K, rows=64, threads=threads)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
