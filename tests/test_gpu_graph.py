"""HIP-graph capture and replay of the library's calls, the way the bench and a serving loop run
them.  Each call is captured once (with a caller workspace, so nothing allocates during capture)
and the graph is replayed several times with eager work on the same buffers between the replays;
every replay's output must equal the eager call's, bit for bit.  GPU only."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

REPLAYS = 4


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


def _replays_match(fn, out, engines_must=None):
    """Eager call, capture, then REPLAYS replays each preceded by eager work that overwrites the
    output; every replay must reproduce the eager output exactly."""
    import torch
    from ksq import ops
    fn()
    torch.cuda.synchronize()
    if engines_must:
        assert engines_must <= ops.last_engines(), ops.last_engines()
    want = out.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    for r in range(REPLAYS):
        out.fill_(float("nan"))
        scratch = torch.randn(1 << 20, device=out.device).sum()   # unrelated eager work between replays
        torch.cuda.synchronize()
        assert torch.isfinite(scratch)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {r}"
    del g


# name, weight type, activation type (0 fp32, 1 Q8_1), M, N, K, forced MFMA tile configuration,
# engines the call must launch
GEMM_CASES = [
    ("planar_q4_0", 0, 0, 2048, 2048, 4096, 0, {"quantize", "mmq_planar"}),     # LDS-DMA GEMM
    ("planar_splitk_q4_1", 4, 0, 300, 520, 1280, 8, {"quantize", "mmq_planar", "splitk"}),
    ("tile128_q8_1_input", 0, 1, 512, 2048, 4096, 1, {"mmq1"}),
    ("decode_fused_fp32", 0, 0, 1, 4096, 4096, 0, {"gemv_direct_fq"}),
    ("q8_0_m32_splitk", 1, 0, 32, 4096, 8192, 0, {"quantize", "splitk"}),
    ("q8_0_m32_small_batch", 1, 0, 32, 4096, 4096, 0, {"quantize", "skinny"}),
    ("q4_k_m128", 2, 0, 128, 2048, 4096, 0, {"quantize"}),
]


@pytest.mark.parametrize("name,wtype,atype,M,N,K,cfg,engines", GEMM_CASES, ids=[c[0] for c in GEMM_CASES])
def test_gemm_graph_replays(dev, name, wtype, atype, M, N, K, cfg, engines):
    import torch
    from ksq import _lib, ops, synth
    g = np.random.default_rng(6000 + M + wtype)
    w = _t(synth.weights(wtype, g, N, K), dev)
    x = _t(synth.activations(g, M, K), dev)
    if atype == 1:
        x = ops.quantize_q8_1(x)
    L = _lib.lib()
    assert L.ksq_set_mmq_config(cfg) == 0
    try:
        ws = torch.empty(max(256, ops.workspace_size(wtype, atype, M, N, K)), dtype=torch.uint8, device=dev)
        out = torch.empty((M, N), dtype=torch.float32, device=dev)
        _replays_match(lambda: ops.gemm(wtype, atype, w, x, M, N, K, out=out, workspace=ws), out, engines)
    finally:
        L.ksq_set_mmq_config(0)


def test_moe_graph_replays(dev):
    """Config-4-like MoE call (route, group, quantise with the output zero-fill, grouped GEMM with
    atomics): replays start from the quantiser's zero-fill, so each equals the eager result."""
    import torch
    from ksq import ops, synth
    g = np.random.default_rng(6100)
    T, E, N, K, k = 256, 8, 2048, 2048, 2
    w = _t(np.stack([synth.weights(0, g, N, K) for _ in range(E)]), dev)
    x = _t(synth.activations(g, T, K), dev)
    lg = _t(synth.router_logits(g, T, E), dev)
    ws = torch.empty(ops.moe_workspace_size(0, T, N, K, E, k), dtype=torch.uint8, device=dev)
    out = torch.empty((T, N), dtype=torch.float32, device=dev)
    # top_k = 2: each output is the sum of exactly two products added onto zero, so the result
    # does not depend on the order of the atomics
    _replays_match(lambda: ops.moe_gemm(0, w, x, lg, T, N, K, E, k, out=out, workspace=ws), out,
                   {"moe_route", "moe_group"})


def test_planar_halves_graph_replays(dev):
    """The bench's timed launch alone: the LDS-DMA GEMM on pre-made planar activations."""
    import torch
    from ksq import ops, synth
    g = np.random.default_rng(6200)
    M, N, K = 1024, 1024, 2048
    w = _t(synth.weights(0, g, N, K), dev)
    planar = ops.quantize_planar(0, _t(synth.activations(g, M, K), dev))
    out = torch.empty((M, N), dtype=torch.float32, device=dev)
    _replays_match(lambda: ops.gemm_planar(0, w, planar, M, N, K, out=out), out, {"mmq_planar"})
