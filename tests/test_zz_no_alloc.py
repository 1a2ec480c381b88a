"""ksq_gemm_noalloc (the entry point that allocates nothing, its scratch a static device array)
against ksq_gemm, through the C ABI: two calls in a row, the second smaller, each bit-identical
to ksq_gemm on the same inputs (same kernels) and within the parity bar of the oracle; plus the
size limit.  GPU only."""
import ctypes

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


def _noalloc(wtype, atype, w, x, y, M, N, K):
    import torch
    from ksq import _lib
    return _lib.lib().ksq_gemm_noalloc(wtype, atype, w.data_ptr(), x.data_ptr(), y.data_ptr(), M, N, K,
                                       ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))


def _rel_err(y, ref):
    y = np.asarray(y, np.float64)
    floor = 1e-3 * np.abs(ref).max(axis=-1, keepdims=True) + 1e-30
    return float((np.abs(y - ref) / np.maximum(np.abs(ref), floor)).max())


def test_noalloc_two_calls_match_ksq_gemm(dev, oracle):
    """Call 1: config 2 (Q4_0, fp32, M = 2048, N = K = 4096; its 9.4 MB of quantised activations
    in the scratch).  Call 2, smaller: Q8_0, fp32, M = 32 (the quantised rows and 8 split-K
    partial results in the same scratch).  Call 3: unit-scale inputs, exact integer result."""
    import torch
    from ksq import ops, refcheck, synth
    g = np.random.default_rng(5100)
    for wtype, M, N, K in ((0, 2048, 4096, 4096), (1, 32, 4096, 4096)):
        w = synth.weights(wtype, g, N, K)
        x = synth.activations(g, M, K)
        wt, xt = _t(w, dev), _t(x, dev)
        y = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
        assert _noalloc(wtype, 0, wt, xt, y, M, N, K) == 0
        ref_dev = ops.gemm(wtype, 0, wt, xt, M, N, K)
        torch.cuda.synchronize()
        assert torch.equal(y, ref_dev), (wtype, M)
        rows = np.unique(np.concatenate([[0, M - 1], g.choice(M, 8)]))
        ref = oracle.gemm_f64(wtype, oracle.quantize_q8_1(x[rows]), w, len(rows), N, K)
        assert _rel_err(y.cpu().numpy()[rows], ref) <= TOL, (wtype, M)
    M, N, K = 16, 1024, 4096
    wu = refcheck.unit_weights(0, g, N, K)
    xu = refcheck.unit_activations(g, M, K, onehot=refcheck.onehot_pattern(M, K // 32))
    y = torch.empty((M, N), dtype=torch.float32, device=dev)
    assert _noalloc(0, 0, _t(wu, dev), _t(xu, dev), y, M, N, K) == 0
    torch.cuda.synchronize()
    exact, bound = refcheck.exact_gemm(0, oracle.quantize_q8_1(xu), wu)
    assert bound.max() < 2 ** 24
    assert np.array_equal(y.cpu().numpy(), exact.astype(np.float32))


def test_noalloc_rejects_calls_past_its_scratch(dev):
    """A call needing more than KSQ_NOALLOC_SCRATCH_BYTES returns KSQ_ERR_WORKSPACE and launches
    nothing (the output keeps its contents); ksq_gemm_workspace_size says why."""
    import torch
    from ksq import _lib
    L = _lib.lib()
    M, N, K = 8192, 256, 4096          # fp32 activations: 8192 * 128 * 36 = 37.7 MB of Q8_1 blocks
    assert L.ksq_gemm_workspace_size(0, 0, M, N, K) > _lib.NOALLOC_SCRATCH_BYTES
    w = torch.zeros((N, K // 32 * 18), dtype=torch.uint8, device=dev)
    x = torch.zeros((M, K), dtype=torch.float32, device=dev)
    y = torch.full((M, N), 7.0, dtype=torch.float32, device=dev)
    assert _noalloc(0, 0, w, x, y, M, N, K) == 5
    assert b"static scratch" in L.ksq_last_error_message()
    torch.cuda.synchronize()
    assert bool((y == 7.0).all())
    # pre-quantised input of the same shape needs no scratch and runs
    a = torch.zeros((M, K // 32 * 36), dtype=torch.uint8, device=dev)
    assert _noalloc(0, 1, w, a, y, M, N, K) == 0
    torch.cuda.synchronize()
    assert bool((y == 0.0).all())
