#!/usr/bin/env python3
"""Benchmark of the quantized GGML matmul hot path on one MI355X.

Headline (BASELINE.json metric): Q4_0 x Q8_1 GEMM TOPS at M=2048 (N = K = 4096),
with the decode GEMV's HBM GB/s at M=1 (N = K = 4096) reported beside it.

A "step" is one pass of the hot path over one batch: gemm_w4a32c8_q4_0_fp32_int8
on fp32 activations [2048, 4096] -> fp32 [2048, 4096], i.e. quantize_q8_1 plus
the int8-MFMA GEMM.  Inputs are seeded synthetic tensors resident in HBM before
timing; weights and activations rotate over several copies so successive steps
do not re-read one buffer from the 256 MB MALL.  Launch sequences are captured
in HIP graphs and replayed, so host-side launch cost (ctypes) is not timed.  The W
untimed warm-up steps (default 256: two eager, the rest replays of the captured
step graph) bring the GPU clocks to their steady state before the K timed steps.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu-baseline]

Prints ONE JSON line on stdout (progress goes to stderr).
"""
from __future__ import annotations

import argparse
import json

import numpy as np
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [ROOT, os.path.join(ROOT, "k-search_amd")]

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, published
INT8_PEAK_TOPS = 5000.0      # MI355X dense int8 MFMA, published

# HBM bytes per launch from two rocprofv3 --pmc passes (FETCH_SIZE, WRITE_SIZE, KiB per
# dispatch, mean of 6) over `bench.py --only gemm|gemv`, scaled by the factors a plain
# 256 MiB copy gives the same counters (reads x2.0, writes x1.0); summaries in profiles/.
TRAFFIC_MMQ_Q4_0_M2048 = int((41715.8 * 2.0 + 32941.8 * 1.0) * 1024)
TRAFFIC_GEMV_Q4_0_M1 = int((4642.2 * 2.0 + 32.0 * 1.0) * 1024)


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def capture(fn, n: int):
    """A HIP graph holding fn(0) .. fn(n-1), launched on torch's capture stream."""
    import torch
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(n):
            fn(i)
    torch.cuda.synchronize()
    return g


def time_graph(g, replays: int) -> float:
    """Milliseconds for `replays` replays of graph g (HIP events, torch's current stream)."""
    import torch
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    s.record()
    for _ in range(replays):
        g.replay()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e)


def cpu_baseline(M: int, N: int, K: int, budget_s: float = 10.0) -> dict:
    """The reference CPU path (quantize_row_q8_1_ref + gemm_w4a8_reference's loop and
    accumulation order, restated in oracle/ksq_oracle.c) on the box's host cores, over
    a bounded sample of the workload's activation rows."""
    from ksq import synth
    from oracle import oracle
    threads = max(1, min(16, len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()))
    g = synth.rng(1)
    w = synth.weights(0, g, N, K)
    # calibrate on a few rows, then size the sample to ~budget_s
    probe = max(threads, 8)
    x = synth.activations(g, probe, K)
    t0 = time.perf_counter()
    oracle.gemm(0, oracle.quantize_q8_1(x), w, probe, N, K, nthreads=threads)
    per_row = (time.perf_counter() - t0) / probe
    rows = int(max(probe, min(M, budget_s / max(per_row, 1e-9))))
    x = synth.activations(g, rows, K)
    t0 = time.perf_counter()
    a = oracle.quantize_q8_1(x)
    oracle.gemm(0, a, w, rows, N, K, nthreads=threads)
    dt = time.perf_counter() - t0
    return {"value": round(2.0 * rows * N * K / dt / 1e12, 6), "unit": "TOPS", "cores": threads, "kind": "port",
            "sample": f"{rows} of {M} activation rows x N=K={K}: quantize_row_q8_1_ref + gemm_w4a8_reference "
                      f"loop order (oracle/ksq_oracle.c, gcc -O2, OpenMP over outputs), {dt:.2f} s"}


def graph_ms(fn, n: int, reps: int) -> float:
    """Average ms per fn(i) call over `reps` replays of a graph of n calls.  One eager call
    first, so the library's workspace pool is sized before capture (no hipMalloc inside)."""
    import torch
    fn(0)
    torch.cuda.synchronize()
    g = capture(fn, n)
    g.replay()
    return time_graph(g, reps) / (reps * n)


def hbm_entry(bytes_, ms, ops=None):
    gbs = bytes_ / (ms * 1e-3) / 1e9
    d = {"avg_ms": round(ms, 6), "algorithmic_bytes": int(bytes_), "GB/s": round(gbs, 1),
         "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                      "frac": round(gbs / HBM_PEAK_GBS, 4)}}
    if ops is not None:
        d["TOPS"] = round(ops / (ms * 1e-3) / 1e12, 3)
    return d


def other_configs(g, dev, reps: int) -> dict:
    """BASELINE configs 1, 3 and 4, each on rotating weight copies (> 256 MB MALL in total)."""
    import torch
    import ksq
    from ksq import ops, synth
    out = {}
    # config 1: Q8_0 x Q8_1, M in {1, 8, 32}, N = K = 4096
    N, K = 4096, 4096
    w = synth.weights(ksq.W_Q8_0, g, N, K)
    copies = 32
    Wc = [torch.from_numpy(w).to(dev) for _ in range(copies)]
    for M in (1, 8, 32):
        aq = ops.quantize_q8_1(torch.from_numpy(synth.activations(g, M, K)).to(dev))
        o = torch.empty((M, N), dtype=torch.float32, device=dev)
        ms = graph_ms(lambda i: ops.gemm(ksq.W_Q8_0, ksq.A_Q8_1, Wc[i % copies], aq, M, N, K, out=o), copies, reps)
        out[f"q8_0_M{M}"] = hbm_entry(N * (K // 32) * 34 + M * (K // 32) * 36 + M * N * 4, ms, 2.0 * M * N * K)
    del Wc
    # config 3: K-quants at M = 128, N = 14336, K = 4096
    M, N, K = 128, 14336, 4096
    aq = ops.quantize_q8_1(torch.from_numpy(synth.activations(g, M, K)).to(dev))
    o = torch.empty((M, N), dtype=torch.float32, device=dev)
    for wt, name, sb in ((ksq.W_Q4_K, "q4_K", 144), (ksq.W_Q6_K, "q6_K", 210)):
        w = synth.weights(wt, g, N, K)
        copies = 8
        Wc = [torch.from_numpy(w).to(dev) for _ in range(copies)]
        ms = graph_ms(lambda i: ops.gemm(wt, ksq.A_Q8_1, Wc[i % copies], aq, M, N, K, out=o), copies, reps)
        out[f"{name}_M128"] = hbm_entry(N * (K // 256) * sb + M * (K // 32) * 36 + M * N * 4, ms, 2.0 * M * N * K)
        del Wc
    # config 4: MoE, 512 tokens, 8 experts of 4096 -> 14336 Q4_0, top-2 (whole call: quantize,
    # route, group, zero-fill, grouped GEMM)
    T, E, N, K, k = 512, 8, 14336, 4096, 2
    w = np.stack([synth.weights(ksq.W_Q4_0, g, N, K) for _ in range(E)])
    copies = 2
    Wc = [torch.from_numpy(w).to(dev) for _ in range(copies)]
    x = torch.from_numpy(synth.activations(g, T, K)).to(dev)
    lg = torch.from_numpy(synth.router_logits(g, T, E)).to(dev)
    o = torch.empty((T, N), dtype=torch.float32, device=dev)
    ws = torch.empty(ops.moe_workspace_size(0, T, N, K, E, k), dtype=torch.uint8, device=dev)
    ms = graph_ms(lambda i: ops.moe_gemm(ksq.W_Q4_0, Wc[i % copies], x, lg, T, N, K, E, k, out=o, workspace=ws),
                  copies, reps)
    moe_bytes = E * N * (K // 32) * 18 + T * K * 4 + T * E * 4 + T * N * 4
    out["moe_q4_0_T512_E8_top2"] = hbm_entry(moe_bytes, ms, 2.0 * T * k * N * K)
    del Wc
    torch.cuda.empty_cache()
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=256,
                    help="untimed steps before the timed ones (the first two eager, the rest as replays of "
                         "the captured step graph): brings the GPU clocks to their steady state")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only", choices=["gemm", "gemv", "step", "copy"],
                    help="profiling mode: launch just that kernel sequence --steps times, eagerly, and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build runs the quantized matmul path on a single "
              "MI355X (no collectives); run with --gpus 1", file=sys.stderr)
        return 2

    import torch

    import ksq
    from ksq import ops, synth

    dev = torch.device("cuda:0")
    if args.only == "copy":
        # calibration for the FETCH_SIZE / WRITE_SIZE counters: a plain copy of 256 MiB
        src = torch.ones(64 << 20, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(args.warmup + args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"only": "copy", "bytes": src.numel() * 4, "launches": args.warmup + args.steps}))
        return 0
    M, N, K = 2048, 4096, 4096
    copies = 8
    g = synth.rng(2024)
    log(f"bench: inputs M={M} N={N} K={K}, {copies} rotating copies")
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

    if args.only in ("gemm", "step"):
        fn = gemm_only if args.only == "gemm" else step
        for i in range(args.warmup + args.steps):
            fn(i)
        torch.cuda.synchronize()
        print(json.dumps({"only": args.only, "launches": args.warmup + args.steps}), flush=True)
        return 0

    n_eager = min(args.warmup, 2)            # sizes the library's workspace pool before capture
    for i in range(n_eager):
        step(i)
    torch.cuda.synchronize()
    g_step = capture(step, args.steps)
    for _ in range(max(1, -(-(args.warmup - n_eager) // args.steps))):
        g_step.replay()
    torch.cuda.synchronize()
    log(f"bench: timing {args.steps} steps")
    t0 = time.perf_counter()
    ms = time_graph(g_step, 1) / args.steps
    wall = (time.perf_counter() - t0) / args.steps * 1e3
    ops_per_step = 2.0 * M * N * K
    tops = ops_per_step / (ms * 1e-3) / 1e12

    g_gemm = capture(gemm_only, args.steps)
    g_gemm.replay()
    gemm_ms = time_graph(g_gemm, 1) / args.steps
    gemm_tops = ops_per_step / (gemm_ms * 1e-3) / 1e12
    del g_step, g_gemm

    # ---- decode GEMV, config 0 shape: 64 weight copies (604 MB, > 2x the MALL)
    Mv, Nv, Kv = 1, 4096, 4096
    gcopies = 64
    wv_np = synth.weights(ksq.W_Q4_0, g, Nv, Kv)
    WV = [torch.from_numpy(wv_np).to(dev) for _ in range(gcopies)]
    xv = torch.from_numpy(synth.activations(g, Mv, Kv)).to(dev)
    aqv = ops.quantize_q8_1(xv)
    outv = torch.empty((Mv, Nv), dtype=torch.float32, device=dev)
    wsv = torch.empty(ops.workspace_size(0, 0, Mv, Nv, Kv), dtype=torch.uint8, device=dev)

    def gemv(i):
        ops.gemm(ksq.W_Q4_0, ksq.A_Q8_1, WV[i % gcopies], aqv, Mv, Nv, Kv, out=outv)

    def gemv_f32(i):
        ops.gemm(ksq.W_Q4_0, ksq.A_F32, WV[i % gcopies], xv, Mv, Nv, Kv, out=outv, workspace=wsv)

    if args.only == "gemv":
        for i in range(args.warmup + args.steps):
            gemv(i)
        torch.cuda.synchronize()
        print(json.dumps({"only": "gemv", "launches": args.warmup + args.steps}), flush=True)
        return 0

    reps = 8
    g_v = capture(gemv, gcopies)
    g_v.replay()
    gemv_ms = time_graph(g_v, reps) / (reps * gcopies)
    g_vf = capture(gemv_f32, gcopies)
    g_vf.replay()
    gemv_f32_ms = time_graph(g_vf, reps) / (reps * gcopies)
    gemv_bytes = Nv * (Kv // 32) * 18 + Mv * (Kv // 32) * 36 + Mv * Nv * 4
    gemv_gbs = gemv_bytes / (gemv_ms * 1e-3) / 1e9
    f32_bytes = Nv * (Kv // 32) * 18 + Mv * Kv * 4 + Mv * Nv * 4

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
        "data": "synthetic, seeded (Q4_0 nibbles U[0,15], d=|N(0,0.02)|; activations N(0,1))",
        "config": {"workload": "q4_0_q8_1_prefill_gemm (BASELINE config 2)", "M": M, "N": N, "K": K,
                   "entry": "gemm_w4a32c8_q4_0_fp32_int8: quantize_q8_1 + int8-MFMA GEMM",
                   "rotating_copies": copies, "host_wall_ms_per_step": round(wall, 5)},
        "roofline": {"bound": "mfma", "kernel": "mmq_kernel<0> (Q4_0 x Q8_1, v_mfma_i32_32x32x32_i8)",
                     "achieved": round(gemm_tops, 3), "peak": INT8_PEAK_TOPS, "unit": "TFLOP/s",
                     "frac": round(gemm_tops / INT8_PEAK_TOPS, 4), "traffic": TRAFFIC_MMQ_Q4_0_M2048,
                     "traffic_unit": "bytes per launch (algorithmic: %d)" % (
                         N * (K // 32) * 18 + M * (K // 32) * 36 + M * N * 4),
                     "avg_kernel_ms": round(gemm_ms, 5),
                     "note": "int8 ops = 2*M*N*K per launch over the HIP-event time of graph-replayed launches"},
        "gemv_m1": {"metric": "GEMV HBM GB/s at M=1 (N=K=4096)", "value": round(gemv_gbs, 1), "unit": "GB/s",
                    "entry": "ksq_gemm_q4_0_q8_1 (Q8_1 activations)", "avg_ms": round(gemv_ms, 6),
                    "algorithmic_bytes": gemv_bytes,
                    "roofline": {"bound": "hbm", "achieved": round(gemv_gbs, 1), "peak": HBM_PEAK_GBS,
                                 "unit": "GB/s", "frac": round(gemv_gbs / HBM_PEAK_GBS, 4),
                                 "traffic": TRAFFIC_GEMV_Q4_0_M1},
                    "fp32_entry_ms": round(gemv_f32_ms, 6),
                    "fp32_entry_gbs": round(f32_bytes / (gemv_f32_ms * 1e-3) / 1e9, 1),
                    "weight_copies": gcopies},
    }
    del WV, g_v, g_vf
    torch.cuda.empty_cache()
    log("bench: other BASELINE configs")
    result["configs"] = other_configs(g, dev, reps=4)
    if not args.no_cpu_baseline:
        log("bench: cpu baseline")
        result["cpu_baseline"] = cpu_baseline(M, N, K)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
