"""block_q8f (fp32 d_a and s_a) on the GPU against the CPU oracle.  GPU only.

The two reference quantisers that keep the Q8_1 scale and sum in fp32 — the deepseek_v2 W4A32C8
operator's (core/operators/quant_gemm/variants/deepseek_v2/w4a32c8_q4_0_fp32_int8/
reference.py:50-73) and the generated lm_head kernel's (best_kernels_GLM-5/quant_gemm/
w4a32c8_q4_0_fp32_int8_llama3_8b_lm_head_n128256_k4096/kernel.cu:85-107) — and the int8 MFMA
GEMM over their blocks.  Bars: the quantised bytes bit for bit; every integer block dot exact
(unit-scale inputs, np.array_equal, every MFMA tile configuration); fp32 outputs within max
relative error 1e-3 of the oracle's fp64 block formula (per element, floor 1e-3 of the row's max);
the deepseek_v2 drop-in symbol at its spec.json test configurations (M = 1, 2, 3, 4, 5, 8, 512,
N = K = 5120) against the oracle's restatement of the operator.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL = 1e-3
TWO24 = float(2 ** 24)
A_Q8F, A_F32_RNE, A_F32_LROUND = 5, 6, 7
RULE_OF = {A_F32_RNE: 0, A_F32_LROUND: 1}


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


def _edge_input(g, M, K):
    x = g.standard_normal((M, K), dtype=np.float32) * np.exp2(g.integers(-20, 12, (M, 1))).astype(np.float32)
    if M >= 6:
        x[0, :32] = 0.0                                                       # d = 1, s = 0
        x[1, :8] = [127.0, 2.5, -2.5, 3.5, 0.5, -0.5, -126.5, 1.25]           # d = 1: ties
        x[1, 8:32] = 0.0
        x[2, 32:64] = 0.0
        x[2, 32], x[2, 33] = 1e-12, -4e-13                                     # amax <= 1e-10
        x[3, 64:96] *= np.float32(1e-39)                                       # subnormal block
        x[4, 96:128] *= np.float32(1e30)                                       # large block
        x[5, :9] = [1e8, 1, 1, 1, 1, 1, 1, 1, -1e8]                            # sequential sum 0
        x[5, 9:32] = 0.0
    return x


@pytest.mark.parametrize("rule", [0, 1])
def test_quantize_q8f_bit_exact(dev, oracle, rule):
    import torch
    from ksq import ops
    g = np.random.default_rng(300 + rule)
    for M, K in ((1, 4096), (6, 1024), (257, 96), (1024, 4096)):
        x = _edge_input(g, M, K)
        q = ops.quantize_q8f(_t(x, dev), rule)
        torch.cuda.synchronize()
        assert np.array_equal(q.cpu().numpy(), oracle.quantize_q8f(x, rule)), (rule, M, K)


def _unit_case(g, wtype, M, N, K, atype):
    """Unit scales: d_w = 1; integer activations with one +-127 per block, so both rules give
    d_a = 1, q_a = x and s_a = the exact integer sum."""
    from ksq import refcheck
    from oracle import oracle
    w = refcheck.unit_weights(wtype, g, N, K)
    x = refcheck.unit_activations(g, M, K, qmax=min(127, refcheck.unit_qmax(wtype, K)),
                                  onehot=refcheck.onehot_pattern(M, K // 32))
    blocks = oracle.quantize_q8f(x, RULE_OF.get(atype, 0))
    ref, bound = refcheck.exact_gemm(wtype, blocks, w)
    assert bound.max() < TWO24, f"inputs too large for exact fp32 sums: {bound.max():.3e}"
    return w, (blocks if atype == A_Q8F else x), ref.astype(np.float32)


def _run(dev, wtype, atype, w, a, M, N, K, cfg=0):
    import torch
    from ksq import _lib, ops
    L = _lib.lib()
    assert L.ksq_set_mmq_config(cfg) == 0
    try:
        y = ops.gemm(wtype, atype, _t(w, dev), _t(a, dev), M, N, K)
        eng = ops.last_engines()
        torch.cuda.synchronize()
    finally:
        L.ksq_set_mmq_config(0)
    return y.cpu().numpy(), eng


@pytest.mark.parametrize("wtype", [0, 5, 1])
@pytest.mark.parametrize("atype", [A_Q8F, A_F32_RNE, A_F32_LROUND])
@pytest.mark.parametrize("M", [1, 2, 8, 33, 300])
def test_gemm_q8f_unit_scale_exact(dev, wtype, atype, M):
    g = np.random.default_rng(1000 * wtype + 10 * atype + M)
    N, K = 384, 1024
    w, a, ref = _unit_case(g, wtype, M, N, K, atype)
    y, eng = _run(dev, wtype, atype, w, a, M, N, K)
    assert np.array_equal(y, ref), (wtype, atype, M, float(np.abs(y - ref).max()))
    if atype != A_Q8F and M <= 2:
        # fp32 rows at decode sizes: quantised to block_q8f inside the decode kernel
        assert eng == {"gemv_direct_fq"}, eng
    else:
        assert any(e.startswith("mmq") for e in eng), eng
        assert ("quantize" in eng) == (atype != A_Q8F), eng


def _order_sensitive_blocks(g, M, K):
    """fp32 rows whose every block has a left-to-right fp32 sum different from the sum of its two
    16-element halves' partial sums (so the s field pins the summation order)."""
    out = np.empty((M * K // 32, 32), np.float32)
    n = 0
    while n < out.shape[0]:
        c = (g.standard_normal((4096, 32)) * 10.0 ** g.uniform(-3, 0, (4096, 1))).astype(np.float32)
        i = np.arange(4096)
        big = g.uniform(1e3, 3e4, 4096).astype(np.float32)
        c[i, g.integers(0, 16, 4096)] = big
        c[i, g.integers(16, 32, 4096)] = -big * np.float32(1.0 + 1e-4)
        seq = np.add.accumulate(c, axis=1, dtype=np.float32)[:, -1]
        halves = (np.add.accumulate(c[:, :16], axis=1, dtype=np.float32)[:, -1]
                  + np.add.accumulate(c[:, 16:], axis=1, dtype=np.float32)[:, -1]).astype(np.float32)
        keep = c[seq != halves]
        take = min(len(keep), out.shape[0] - n)
        out[n:n + take] = keep[:take]
        n += take
    return out.reshape(M, K)


@pytest.mark.parametrize("atype", [A_F32_RNE, A_F32_LROUND])
@pytest.mark.parametrize("M", [1, 2])
def test_q8f_decode_quantiser_readout(dev, oracle, atype, M):
    """The decode kernel's in-workgroup block_q8f quantiser, read back bit for bit:
    * Q4_0 weights whose quants are all 8 (value 0) with d_w = 1 in block r of row r only:
      output (m, r) = d_w * (d_a * 0 - 8 * s_a) = -8 * s_a of activation block r, exactly;
    * Q8_0 weights with one quant 1 at element k of block b in row 32 b + k (d_w = 1, others 0):
      output = d_a * q_a[k], the reference's own single rounding of that product.
    On blocks whose sequential and split sums differ, against the oracle's block_q8f bytes."""
    import torch
    from ksq import ops
    K = 4096
    nb = K // 32
    g = np.random.default_rng(5000 + 10 * atype + M)
    x = _order_sensitive_blocks(g, M, K)
    blocks = oracle.quantize_q8f(x, RULE_OF[atype]).reshape(M, nb, 40)
    s_ref = blocks[:, :, 4:8].copy().view(np.float32)[:, :, 0]
    # Q4_0 readout of s
    w4 = np.zeros((nb, nb, 18), np.uint8)
    w4[:, :, 2:] = 0x88
    w4[np.arange(nb), np.arange(nb), 0:2] = np.frombuffer(np.float16(1).tobytes(), np.uint8)
    y4 = ops.gemm(0, atype, _t(w4, dev), _t(x, dev), M, nb, K)
    eng = ops.last_engines()
    torch.cuda.synchronize()
    assert eng == {"gemv_direct_fq"}, eng
    assert np.array_equal(y4.cpu().numpy(), (np.float32(-8.0) * s_ref).astype(np.float32))
    # Q8_0 readout of d_a * q_a
    w8 = np.zeros((nb * 32, nb, 34), np.uint8)
    r = np.arange(nb * 32)
    w8[r, r // 32, 0:2] = np.frombuffer(np.float16(1).tobytes(), np.uint8)
    w8[r, r // 32, 2 + r % 32] = 1
    y8 = ops.gemm(1, atype, _t(w8, dev), _t(x, dev), M, nb * 32, K)
    eng = ops.last_engines()
    torch.cuda.synchronize()
    assert eng == {"gemv_direct_fq"}, eng
    ref8 = oracle.gemm_q8f(1, blocks.reshape(M, nb * 40), w8, M, nb * 32, K)
    assert np.array_equal(y8.cpu().numpy(), ref8)


@pytest.mark.parametrize("cfg", [1, 2, 3, 4, 5, 6, 7])
def test_gemm_q8f_every_tile_exact(dev, cfg):
    """Each MFMA tile configuration (forced) with block_q8f activations, Q4_0 and Q8_0."""
    for wtype in (0, 1):
        g = np.random.default_rng(2000 + 10 * cfg + wtype)
        M, N, K = 200, 320, 2048
        w, a, ref = _unit_case(g, wtype, M, N, K, A_F32_RNE)
        y, eng = _run(dev, wtype, A_F32_RNE, w, a, M, N, K, cfg=cfg)
        assert np.array_equal(y, ref), (cfg, wtype)
        assert f"mmq{cfg}" in eng, eng


@pytest.mark.parametrize("wtype", [0, 5, 1])
@pytest.mark.parametrize("atype", [A_F32_RNE, A_F32_LROUND])
def test_gemm_q8f_random_vs_oracle(dev, oracle, wtype, atype):
    g = np.random.default_rng(3000 + 10 * wtype + atype)
    M, N, K = 70, 256, 2048
    x = g.standard_normal((M, K), dtype=np.float32)
    wf = g.standard_normal((N, K), dtype=np.float32)
    quant = {0: oracle.quantize_q4_0, 5: oracle.quantize_q5_0, 1: oracle.quantize_q8_0}[wtype]
    w = quant(wf).reshape(N, K // 32, -1)
    y, _ = _run(dev, wtype, atype, w, x, M, N, K)
    blocks = oracle.quantize_q8f(x, RULE_OF[atype])
    ref = oracle.gemm_q8f(wtype, blocks, w, M, N, K, f64=True)
    assert _rel_err(y, ref) < TOL
    # the same blocks handed over pre-quantised give the same outputs
    y2, _ = _run(dev, wtype, A_Q8F, w, blocks, M, N, K)
    assert np.array_equal(y, y2)


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8, 512])
def test_deepseek_v2_dropin_spec_configs(dev, oracle, M):
    """gemm_w4a32c8_q4_0_fp32_int8_deepseek_v2 called as the harness calls a kernel (device
    pointers, null stream, no workspace) at the operator's spec.json test configurations,
    against the oracle's restatement of reference.py:run (fp32 block order) on sampled rows."""
    import torch
    from ksq import _lib
    L = _lib.lib()
    N = K = 5120
    g = np.random.default_rng(4000 + M)
    x = g.standard_normal((M, K), dtype=np.float32)
    w = oracle.quantize_q4_0(g.standard_normal((N, K), dtype=np.float32) * 0.05).reshape(N, K // 32, 18)
    wt, xt = _t(w, dev), _t(x, dev)
    y = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    L.gemm_w4a32c8_q4_0_fp32_int8_deepseek_v2(wt.data_ptr(), xt.data_ptr(), y.data_ptr(), M, N, K)
    torch.cuda.synchronize()
    assert L.ksq_last_error() == 0, L.ksq_last_error_message().decode()
    rows = np.unique(np.linspace(0, M - 1, min(M, 8)).astype(int))
    blocks = oracle.quantize_q8f(x[rows], 0)
    ref = oracle.gemm_q8f(0, blocks, w, len(rows), N, K)
    got = y.cpu().numpy()[rows]
    assert _rel_err(got, ref) < TOL


def test_runner_deepseek_v2_spec(dev, tmp_path):
    """The deepseek_v2 W4A32C8 operator run through the definition runner from its spec.json
    fields (name w4a32c8_q4_0_fp32_int8, entry "forward", model_architectures deepseek-v2,
    threshold 0.1, test_configs M = 1..5, 8, 512, N = K = 5120): it resolves to the block_q8f entry,
    and the runner's exact checks compare against the fp32-scale quantiser and block formula."""
    from ksq import _lib, runner
    spec = {"name": "w4a32c8_q4_0_fp32_int8", "variant": "W4A32C8", "family": "quant_gemm",
            "model_architectures": ["deepseek-v2"], "kernel": {"file": "kernel.cu", "entry_point": "forward"},
            "inputs": {"weight": {"dtype": "block_q4_0"}, "activation": {"dtype": "float32"}},
            "params": {"M": {"type": "int"}, "N": {"type": "int", "default": 5120},
                       "K": {"type": "int", "default": 5120}},
            "test_configs": [{"name": f"batch_{m}", "M": m} for m in (1, 2, 3, 4, 5, 8, 512)],
            "accuracy": {"metric": "nmse", "threshold": 0.1}}
    r = runner.DefinitionRunner(warmup=1, iterations=2, all_configs=True, log=lambda s: None).run(spec, str(tmp_path))
    assert r["compilation"]["entry_point"] == "gemm_w4a32c8_q4_0_fp32_int8_deepseek_v2"
    assert r["compilation"]["activation_type"] == _lib.A_F32_Q8F_RNE
    assert r["correctness"]["threshold"] == 0.1
    cases = r["correctness"]["test_cases"]
    assert [c["config"] for c in cases] == [f"batch_{m}" for m in (1, 2, 3, 4, 5, 8, 512)]
    for c in cases:
        ex = c["exact"]
        assert c["passed"] and ex["quantize_bit_exact"] and ex["block_dots_bit_exact"], c
        assert ex["max_rel_err_vs_fp64"] <= 1e-3, c
        assert ex["engines"], c
    assert (tmp_path / "test_results.json").exists()
