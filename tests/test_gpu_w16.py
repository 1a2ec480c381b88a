"""The dequantise-then-fp32 GEMM (W4A16 / W8A16) on the GPU against the CPU oracle.  GPU only.

Reference: gemm_w4a16_naive / gemm_w4a16_tiled / gemm_w8a16_naive (include/gemm_cuda_naive.cuh:
66-150, include/gemm_cuda_tiled.cuh:108-190), their CPU references (include/gemm_reference.h:
73-147) and the harness oracle of the fp32-activation definitions (llm_kernel_test/reference/
gemm_ref.py:51-97).  Bars: integer-valued inputs (d = 1, integer activations, all sums below
2^24) exact, np.array_equal, on both tiles, split and unsplit; random inputs within the fp32
accumulation bound of the fp64 dequantised product (|y - ref| <= 2^-24 * K * sum |a w|), and
within max relative error 1e-3 of the reference's own fp32 loop; identical results run to run.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL = 1e-3


@pytest.fixture(scope="module")
def dev():
    import torch
    assert torch.cuda.is_available(), "gpu tests need a GPU"
    from ksq import _lib
    _lib.lib()
    return torch.device("cuda:0")


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _rel_err(y, ref):
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    floor = 1e-3 * np.abs(ref).max(axis=-1, keepdims=True) + 1e-30
    return float((np.abs(y - ref) / np.maximum(np.abs(ref), floor)).max())


def _int_weights(wtype, g, N, K):
    nb = K // 32
    if wtype == 0:
        w = np.zeros((N, nb, 18), np.uint8)
        w[..., 0:2] = np.frombuffer(np.float16(1).tobytes(), np.uint8)
        w[..., 2:18] = g.integers(0, 256, size=(N, nb, 16), dtype=np.uint8)
        qs = w[..., 2:18].astype(np.int64)
        vals = np.concatenate([qs & 15, qs >> 4], axis=-1) - 8
    else:
        w = np.zeros((N, nb, 34), np.uint8)
        w[..., 0:2] = np.frombuffer(np.float16(1).tobytes(), np.uint8)
        w[..., 2:34] = g.integers(-128, 128, size=(N, nb, 32)).astype(np.int8).view(np.uint8)
        vals = w[..., 2:34].view(np.int8).astype(np.int64)
    return w, vals.reshape(N, K)


def _run(dev, wtype, x, w, M, N, K, workspace=False):
    import torch
    from ksq import ops
    ws = None
    if workspace:
        nbytes = ops.gemm_w16_workspace_size(M, N, K)
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev) if nbytes else None
    y = ops.gemm_w16(wtype, _t(x, dev), _t(w, dev), M, N, K, workspace=ws)
    eng = ops.last_engines()
    torch.cuda.synchronize()
    return y.cpu().numpy(), eng


@pytest.mark.parametrize("wtype", [0, 1])
@pytest.mark.parametrize("M,N,K", [(1, 256, 1024), (2, 300, 1024), (3, 520, 2048), (4, 130, 8320),
                                   (1, 4096, 14336), (7, 200, 320), (32, 384, 2048), (45, 130, 576),
                                   (300, 256, 1024), (129, 1024, 4096),
                                   # the decode form's 16 and 8 weight rows per workgroup (512+ workgroups)
                                   # with ragged last workgroups: 16 rows at N = 14336 and N = 8200
                                   # (8 rows past N), 8 rows at N = 4100 (4 past N)
                                   (1, 14336, 4096), (4, 8200, 1024), (2, 4100, 2048)])
def test_w16_integer_inputs_exact(dev, wtype, M, N, K):
    from ksq import ops
    g = np.random.default_rng(500 + 7 * M + wtype)
    w, vals = _int_weights(wtype, g, N, K)
    amax = 40 if wtype == 0 else 3            # sum |a w| < 2^24 at K = 4096
    x = g.integers(-amax, amax + 1, size=(M, K)).astype(np.float32)
    want = (x.astype(np.int64) @ vals.T)
    assert (np.abs(x.astype(np.int64)) @ np.abs(vals).T).max() < 2 ** 24
    y, eng = _run(dev, wtype, x, w, M, N, K)
    assert np.array_equal(y, want.astype(np.float32)), (wtype, M, N, K, float(np.abs(y - want).max()))
    assert "w16" in eng
    assert ("splitk" in eng) == (ops.gemm_w16_workspace_size(M, N, K) > 0)


@pytest.mark.parametrize("wtype", [0, 1])
@pytest.mark.parametrize("M,N,K", [(1, 4096, 4096), (3, 1000, 8192), (16, 512, 2048), (96, 640, 1536),
                                   (512, 512, 4096)])
def test_w16_random_vs_oracle(dev, oracle, wtype, M, N, K):
    from ksq import refcheck
    g = np.random.default_rng(600 + M + wtype)
    x = g.standard_normal((M, K), dtype=np.float32)
    if M > 1:
        x[0] *= np.float32(1e30)                 # wide range: the three-term split keeps products exact
        x[1] *= np.float32(1e-30)
    quant = oracle.quantize_q4_0 if wtype == 0 else oracle.quantize_q8_0
    w = quant(g.standard_normal((N, K), dtype=np.float32)).reshape(N, K // 32, -1)
    y, _ = _run(dev, wtype, x, w, M, N, K, workspace=True)
    wd = refcheck.dequantize(wtype, w)
    ref64 = x.astype(np.float64) @ wd.T
    bound = np.abs(x.astype(np.float64)) @ np.abs(wd).T
    assert np.all(np.abs(y - ref64) <= 2.0 ** -24 * K * bound)
    rows = np.unique(np.linspace(0, M - 1, min(M, 6)).astype(int))
    ref32 = oracle.gemm_w16(wtype, x[rows], w, len(rows), N, K)
    assert _rel_err(y[rows], ref32) < TOL
    y2, _ = _run(dev, wtype, x, w, M, N, K)
    assert np.array_equal(y, y2)


def test_w16_baseline_shapes(dev, oracle):
    """BASELINE config 0 and config 2 shapes (M = 1 and M = 2048, N = K = 4096) through the
    reference launchers' form (ksq_gemm_w4a16 / ksq_gemm_w8a16, library pool), sampled rows
    against the reference's fp32 loop."""
    import torch
    from ksq import _lib
    L = _lib.lib()
    N = K = 4096
    for wtype, entry in ((0, "ksq_gemm_w4a16"), (1, "ksq_gemm_w8a16")):
        for M in (1, 2048):
            g = np.random.default_rng(700 + M + wtype)
            x = g.standard_normal((M, K), dtype=np.float32)
            quant = oracle.quantize_q4_0 if wtype == 0 else oracle.quantize_q8_0
            w = quant(g.standard_normal((N, K), dtype=np.float32) * 0.02).reshape(N, K // 32, -1)
            xt, wt = _t(x, dev), _t(w, dev)
            y = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
            assert getattr(L, entry)(xt.data_ptr(), wt.data_ptr(), y.data_ptr(), M, N, K, None) == 0
            torch.cuda.synchronize()
            rows = np.unique(np.linspace(0, M - 1, min(M, 8)).astype(int))
            ref = oracle.gemm_w16(wtype, x[rows], w, len(rows), N, K)
            assert _rel_err(y.cpu().numpy()[rows], ref) < TOL, (entry, M)
