"""Calls on concurrent streams of one GPU without a caller workspace: each (device, stream) has
its own library pool, so two streams' calls in flight at once do not share scratch.  GPU only."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


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


@pytest.mark.parametrize("wtype,M,N,K", [(0, 256, 1024, 4096),    # fp32 rows quantised into the pool, MFMA GEMM
                                         (1, 64, 1024, 8192),     # split-K partial sums in the pool
                                         (0, 2048, 512, 2048)])   # planar quantised copy in the pool
def test_pool_per_stream_concurrent(dev, wtype, M, N, K):
    """Two streams each run the same call shape on their own inputs, back to back without
    synchronising, eight times; every output equals the same call made alone on the default
    stream."""
    import torch
    from ksq import ops, synth
    g = np.random.default_rng(6200 + wtype + M)
    ws = [_t(synth.weights(wtype, g, N, K), dev) for _ in range(2)]
    xs = [_t(synth.activations(g, M, K), dev) for _ in range(2)]
    want = [ops.gemm(wtype, 0, w, x, M, N, K) for w, x in zip(ws, xs)]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = [torch.empty((M, N), dtype=torch.float32, device=dev) for _ in range(2)]
    for rep in range(8):
        for o in outs:
            o.fill_(float("nan"))
        torch.cuda.synchronize()
        for i in range(2):
            with torch.cuda.stream(streams[i]):
                ops.gemm(wtype, 0, ws[i], xs[i], M, N, K, out=outs[i])
        torch.cuda.synchronize()
        for i in range(2):
            assert torch.equal(outs[i], want[i]), (rep, i)


def test_capture_borrows_warmed_pool(dev):
    """An eager call on one stream grows that stream's pool; capturing the same call (no caller
    workspace) on torch's capture stream then uses that pool, and every replay equals the eager
    output."""
    import torch
    from ksq import ops, synth
    g = np.random.default_rng(6300)
    M, N, K = 256, 1024, 4096
    w = _t(synth.weights(0, g, N, K), dev)
    x = _t(synth.activations(g, M, K), dev)
    out = torch.empty((M, N), dtype=torch.float32, device=dev)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        ops.gemm(0, 0, w, x, M, N, K, out=out)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    want = out.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ops.gemm(0, 0, w, x, M, N, K, out=out)
    for _ in range(3):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want)
    del graph


@pytest.mark.filterwarnings("ignore:The CUDA Graph is empty")   # the refused call captured nothing
def test_capture_refuses_to_grow_pool(dev):
    """With every pool released, a call that needs library scratch is refused during capture
    (KSQ_ERR_WORKSPACE, nothing launched), and runs once a workspace is passed."""
    import torch
    from ksq import _lib, ops, synth
    g = np.random.default_rng(6301)
    M, N, K = 256, 1024, 4096
    w = _t(synth.weights(0, g, N, K), dev)
    x = _t(synth.activations(g, M, K), dev)
    out = torch.empty((M, N), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    _lib.lib().ksq_release()
    graph = torch.cuda.CUDAGraph()
    with pytest.raises(_lib.KsqError) as err:
        with torch.cuda.graph(graph):
            ops.gemm(0, 0, w, x, M, N, K, out=out)
    assert _lib.STATUS[err.value.status] == "KSQ_ERR_WORKSPACE"
    del graph
    torch.cuda.synchronize()
    ws = torch.empty(ops.workspace_size(0, 0, M, N, K), dtype=torch.uint8, device=dev)
    want = ops.gemm(0, 0, w, x, M, N, K)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ops.gemm(0, 0, w, x, M, N, K, out=out, workspace=ws)
    out.fill_(float("nan"))
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, want)
    del graph
