"""Writes the committed golden fixtures under tests/golden/ from the C oracle.

    python tests/golden/make_golden.py

Inputs come from a fixed seed (numpy PCG64); expected outputs are the oracle's
(quantize_row_q8_1_ref, the integer block dots, gemm_w4a8/w8a8_reference order,
the Q4_1/Q5_0/Q5_1 block formulas and the native W8A8C8 operator).
The fixtures pin the oracle against regressions and travel to the GPU box,
where the GPU path is compared against them without rebuilding anything.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.join(ROOT, "k-search_amd")]

from oracle import oracle  # noqa: E402
from ksq import synth  # noqa: E402


def main():
    g = np.random.default_rng(20240601)
    M, N, K = 4, 8, 64          # the 4x8x64 case
    x = synth.activations(g, M, K)
    x[1, 32:] = 0.0             # a zero block
    x[2, 0:8] = [127.0, 2.5, -2.5, 0.5, -0.5, 1.5, -126.5, 0.0]   # constructed ties (amax = 127 -> id = 1)
    x[2, 8:32] = 0.0
    a = oracle.quantize_q8_1(x)
    w4 = synth.weights(0, g, N, K)
    w8 = synth.weights(1, g, N, K)
    np.savez(os.path.join(HERE, "q4_0_q8_1_small.npz"), x=x, a_q8_1=a, w_q4_0=w4, w_q8_0=w8,
             sumi_q4_0=oracle.block_sumi(0, a, w4, M, N, K), c_q4_0=oracle.gemm(0, a, w4, M, N, K),
             sumi_q8_0=oracle.block_sumi(1, a, w8, M, N, K), c_q8_0=oracle.gemm(1, a, w8, M, N, K))

    M, N, K = 3, 5, 256         # the 3x5x256 case, all four weight formats
    x = synth.activations(g, M, K)
    a = oracle.quantize_q8_1(x)
    out = {"x": x, "a_q8_1": a}
    for wt, name in ((0, "q4_0"), (1, "q8_0"), (2, "q4_K"), (3, "q6_K")):
        w = synth.weights(wt, g, N, K)
        out["w_" + name] = w
        out["sumi_" + name] = oracle.block_sumi(wt, a, w, M, N, K)
        out["c_" + name] = oracle.gemm(wt, a, w, M, N, K)
        out["c64_" + name] = oracle.gemm_f64(wt, a, w, M, N, K)
    np.savez(os.path.join(HERE, "all_formats_3x5x256.npz"), **out)

    T, E, N, K, k = 16, 4, 64, 256, 2   # 16-token, 4-expert MoE
    logits = synth.router_logits(g, T, E)
    ids, wts = oracle.moe_route(logits, k)
    W = np.stack([synth.weights(0, g, N, K) for _ in range(E)])
    x = synth.activations(g, T, K)
    a = oracle.quantize_q8_1(x)
    np.savez(os.path.join(HERE, "moe_16x4.npz"), logits=logits, ids=ids, wts=wts, w=W, x=x, a_q8_1=a,
             out64=oracle.moe_q4_0_f64(W, a, ids, wts, T, N, K))

    g = np.random.default_rng(20240602)
    M, N, K = 3, 5, 256         # Q4_1 / Q5_0 / Q5_1 and the native W8A8C8 operator
    x = synth.activations(g, M, K)
    x[2, 0:6] = [127.0, 2.5, -2.5, 0.5, -126.5, 0.0]   # ties under both quantisers (d = 1 exactly)
    x[2, 6:32] = 0.0
    x[1, 32:64] *= 1e-5                                 # native rule: d < 1e-6 -> d = 1
    a = oracle.quantize_q8_1(x)
    out = {"x": x, "a_q8_1": a}
    for wt, name in ((4, "q4_1"), (5, "q5_0"), (6, "q5_1")):
        w = synth.weights(wt, g, N, K)
        out["w_" + name] = w
        out["sumi_" + name] = oracle.block_sumi(wt, a, w, M, N, K)
        out["c_" + name] = oracle.gemm(wt, a, w, M, N, K)
        out["c64_" + name] = oracle.gemm_f64(wt, a, w, M, N, K)
    w8 = synth.weights(1, g, N, K)
    a8s = oracle.quantize_q8s(x)
    out.update(w_q8_0=w8, a_q8s=a8s, sumi_q8s=oracle.block_sumi(1, a8s, w8, M, N, K),
               c_w8a8c8=oracle.gemm_w8a8c8(x, w8, M, N, K), c64_w8a8c8=oracle.gemm_q8s_f64(a8s, w8, M, N, K))
    wf = g.standard_normal((N, K), dtype=np.float32) * np.float32(0.05)
    out.update(wf=wf, w_q4_1_from_fp32=oracle.quantize_q4_1(wf))    # the harness' quantize_to_q4_1 path
    np.savez(os.path.join(HERE, "legacy_q8s_3x5x256.npz"), **out)
    print("fixtures written to", HERE)


if __name__ == "__main__":
    main()
