"""Parity of the HIP path (through the C ABI) with the CPU oracle.  GPU only.

Bars: bit-exact for the Q8_1 quantiser and every integer block dot (v_dot4
decode kernels and int8 MFMA tiles); fp32 outputs within max relative error
1e-3 of the fp64 oracle (TOL below; per element against |ref| with a floor of
1e-3 of the row's max |ref| so near-zero outputs do not dominate).  Full
BASELINE sizes are checked on sampled rows and through size-independent
properties.
"""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL = 1e-3
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


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


def _gpu_gemm(dev, wtype, w, x, M, N, K, atype=0, path=0):
    import torch
    from ksq import ops
    ops.set_path(path)
    try:
        out = ops.gemm(wtype, atype, _t(w, dev), _t(x, dev), M, N, K)
        torch.cuda.synchronize()
    finally:
        ops.set_path(0)
    return out.cpu().numpy()


# ------------------------------------------------------------------ quantiser
def test_quantize_q8_1_bit_exact(dev, oracle):
    import torch
    from ksq import ops
    g = np.random.default_rng(100)
    for M, K in ((1, 4096), (3, 1024), (257, 96), (2048, 4096)):
        x = g.standard_normal((M, K), dtype=np.float32)
        if M == 3:
            x[0, :32] = 0.0
            x[1, :8] = [127.0, 2.5, -2.5, 0.5, -0.5, 1.5, -126.5, 3.49999976]
            x[1, 8:32] = 0.0
            x[2, 32:64] *= 3e4
            x[2, 64:96] *= 1e-30
            # the general path: an infinite input, and a block so small that 1/d overflows
            x[0, 64] = np.inf
            x[0, 96:128] *= 1e-39
        q = ops.quantize_q8_1(_t(x, dev))
        torch.cuda.synchronize()
        assert np.array_equal(q.cpu().numpy(), oracle.quantize_q8_1(x)), (M, K)


def _planar_planes(buf, M, K):
    """(quants [M][K] int8, (d, nc) [K/32][Mp][2] float32, -s bits [K/128][Mp][4] uint16) of a
    planar block_q8_1 buffer (each plane 256-byte aligned, Mp = M rounded up to 128)."""
    a256 = lambda b: (b + 255) // 256 * 256  # noqa: E731
    mp, nb = (M + 127) // 128 * 128, K // 32
    q = buf[:M * K].view(np.int8).reshape(M, K)
    o = a256(M * K)
    dn = buf[o:o + nb * mp * 8].view(np.float32).reshape(nb, mp, 2)
    o += a256(nb * mp * 8)
    sa = buf[o:o + nb // 4 * mp * 8].view(np.uint16).reshape(nb // 4, mp, 4)
    return q, dn, sa


@pytest.mark.parametrize("wtype,M,K", [(0, 2048, 4096), (4, 300, 1024), (0, 1, 256)])
def test_quantize_planar_bit_exact(dev, oracle, wtype, M, K):
    """The LDS-DMA GEMM's planar activations hold exactly the oracle's block_q8_1 blocks: quants,
    d (divided by 8 for Q4_0) with -12582912 d beside it, and -s; rows past M are zeros."""
    import torch
    from ksq import ops
    g = np.random.default_rng(120 + M)
    x = g.standard_normal((M, K), dtype=np.float32)
    x[0, 64] = np.inf                      # the general path of the device quantiser
    x[M // 2, 96:128] *= 1e-39
    buf = ops.quantize_planar(wtype, _t(x, dev))
    torch.cuda.synchronize()
    q, dn, sa = _planar_planes(buf.cpu().numpy(), M, K)
    blk = oracle.quantize_q8_1(x)                               # [M][K/32][36]
    d16 = blk[:, :, 0:2].copy().view(np.float16)[:, :, 0]
    s16 = blk[:, :, 2:4].copy().view(np.uint16)[:, :, 0]
    assert np.array_equal(q, blk[:, :, 4:].reshape(M, K).view(np.int8))
    d = d16.astype(np.float32) * np.float32(0.125 if wtype == 0 else 1.0)
    assert np.array_equal(dn[:, :M, 0], d.T)
    assert np.array_equal(dn[:, :M, 1], (np.float32(-12582912.0) * d).T)
    want_sa = (s16 ^ 0x8000).T.reshape(K // 128, 4, M).transpose(0, 2, 1)
    assert np.array_equal(sa[:, :M, :], want_sa)
    assert not dn[:, M:, 0].any() and not dn[:, M:, 1].any()


@pytest.mark.parametrize("wtype,M,N,K", [(0, 2048, 4096, 4096), (4, 300, 520, 1280)])
def test_planar_halves_equal_fp32_call(dev, wtype, M, N, K):
    """ksq_debug_quantize_planar + ksq_debug_gemm_planar write what the fp32 ksq_gemm call writes,
    bit for bit (the bench times the GEMM half alone)."""
    import torch
    from ksq import _lib, ops, synth
    g = np.random.default_rng(130 + M)
    w = _t(synth.weights(wtype, g, N, K), dev)
    x = _t(synth.activations(g, M, K), dev)
    L = _lib.lib()
    assert L.ksq_set_mmq_config(8) == 0
    try:
        y = ops.gemm(wtype, 0, w, x, M, N, K)
        assert "mmq_planar" in ops.last_engines()
        y2 = ops.gemm_planar(wtype, w, ops.quantize_planar(wtype, x), M, N, K)
        assert ops.last_engines() & {"mmq_planar"}
        torch.cuda.synchronize()
    finally:
        L.ksq_set_mmq_config(0)
    assert torch.equal(y, y2)


@pytest.mark.parametrize("variant", [0, 1, 2, 3])
def test_quantize_q8_1_variants_bit_exact(dev, oracle, variant):
    """ksq_quantize_q8_1_variant: the reference's device quantiser (1), the NumPy harness
    quantiser (2) and the fused FP16 kernels' quantiser (3) against their oracle statements, bit
    for bit, over magnitudes 2^-20 .. 2^11, zero blocks, rounding ties, large sums; fp16 input
    with blocks whose d is subnormal in fp16 (variant 3); infinite inputs (1, 3)."""
    import torch
    from ksq import ops
    g = np.random.default_rng(150 + variant)
    for M, K in ((1, 4096), (5, 1024), (300, 96), (2048, 4096)):
        x = g.standard_normal((M, K), dtype=np.float32) * np.exp2(g.integers(-20, 12, (M, 1))).astype(np.float32)
        if M == 5:
            x[0, :32] = 0.0
            x[1, :8] = [127.0, 2.5, -2.5, 0.5, -0.5, 1.5, -126.5, 3.49999976]
            x[1, 8:32] = 0.0
            x[2, 32:64] *= 3e4 if variant != 3 else 1.0
            x[3, 64:96] = x[3, 64:96] * np.float32(2.0 ** -18)     # fp16: d below 2^-14
            if variant in (1, 3):
                x[4, 96] = np.inf
        if variant == 3:
            xh = x.astype(np.float16)
            q = ops.quantize_q8_1_variant(_t(xh, dev), 3)
            want = oracle.quantize_q8_1_variant(xh, 3)
        else:
            q = ops.quantize_q8_1_variant(_t(x, dev), variant)
            want = oracle.quantize_q8_1_variant(x, variant)
        torch.cuda.synchronize()
        assert np.array_equal(q.cpu().numpy(), want), (variant, M, K)


@pytest.mark.parametrize("wtype", [0, 1, 2, 4])
def test_fp16_activation_entries(dev, oracle, wtype):
    """fp16 activations (KSQ_A_F16): quantised by the fused FP16 kernels' rules, then every
    route (decode, small-batch, MFMA); and, for Q4_0, the reference's gemm_q4_0_fp16_fused
    orientation (M weight rows, output [M][N]).  Bar: TOL against the oracle on the same
    quantised blocks."""
    import torch
    from ksq import ops, synth
    from ksq._lib import A_F16
    g = np.random.default_rng(170 + wtype)
    for M, N, K in ((1, 300, 512), (3, 1024, 2048), (8, 4096, 1024), (64, 520, 768), (300, 256, 4096)):
        w = synth.weights(wtype, g, N, K)
        xh = synth.activations(g, M, K).astype(np.float16)
        ref = oracle.gemm_f64(wtype, oracle.quantize_q8_1_variant(xh, 3), w, M, N, K)
        wt = _t(w, dev)
        y = ops.gemm(wtype, A_F16, wt, _t(xh, dev), M, N, K)
        eng = ops.last_engines() - {"quantize"}
        torch.cuda.synchronize()
        assert _rel_err(y.cpu().numpy(), ref) <= TOL, (M, N, K)
        if wtype == 0:
            yt = ops.gemm_q4_0_fp16_fused(wt, _t(xh, dev), N, M, K)
            eng_t = ops.last_engines() - {"quantize", "transpose"}
            torch.cuda.synchronize()
            assert _rel_err(yt.cpu().numpy().T, ref) <= TOL, (M, N, K)
            # the same kernels give the same bits (up to 8 rows the fused entry takes the decode
            # kernels where ksq_gemm may take the small-batch MFMA kernel)
            if eng_t == eng:
                assert np.array_equal(yt.cpu().numpy(), y.cpu().numpy().T), (M, N, K)


def test_golden_fixture_on_gpu(dev):
    """The committed fixtures reproduce on the GPU with no CPU oracle in the loop."""
    import torch
    from ksq import ops
    z = np.load(os.path.join(GOLDEN, "q4_0_q8_1_small.npz"), allow_pickle=False)
    M, K = z["x"].shape
    N = z["w_q4_0"].shape[0]
    a = ops.quantize_q8_1(_t(z["x"], dev))
    torch.cuda.synchronize()
    assert np.array_equal(a.cpu().numpy(), z["a_q8_1"])
    s = ops.block_sumi(0, _t(z["w_q4_0"], dev), a, M, N, K).cpu().numpy()
    assert np.array_equal(s, z["sumi_q4_0"])
    z2 = np.load(os.path.join(GOLDEN, "all_formats_3x5x256.npz"), allow_pickle=False)
    M, K = z2["x"].shape
    for wt, name in ((0, "q4_0"), (1, "q8_0"), (2, "q4_K"), (3, "q6_K")):
        w = z2["w_" + name]
        N = w.shape[0]
        s = ops.block_sumi(wt, _t(w, dev), _t(z2["a_q8_1"], dev), M, N, K).cpu().numpy()
        assert np.array_equal(s, z2["sumi_" + name]), name
        y = _gpu_gemm(dev, wt, w, z2["x"], M, N, K)
        assert _rel_err(y, z2["c64_" + name]) <= TOL, name


# ------------------------------------------------------------------ integer block dots
ALL_WTYPES = [0, 1, 2, 3, 4, 5, 6]      # Q4_0 Q8_0 Q4_K Q6_K Q4_1 Q5_0 Q5_1


@pytest.mark.parametrize("wtype", ALL_WTYPES)
def test_block_sumi_dot4_bit_exact(dev, oracle, wtype):
    from ksq import ops, synth
    g = np.random.default_rng(200 + wtype)
    M, N, K = 5, 37, 512
    w = synth.weights(wtype, g, N, K)
    a = oracle.quantize_q8_1(synth.activations(g, M, K) * 2)
    got = ops.block_sumi(wtype, _t(w, dev), _t(a, dev), M, N, K).cpu().numpy()
    assert np.array_equal(got, oracle.block_sumi(wtype, a, w, M, N, K))


@pytest.mark.parametrize("wtype", ALL_WTYPES)
def test_block_sumi_mfma_bit_exact(dev, oracle, wtype):
    from ksq import ops, synth
    g = np.random.default_rng(300 + wtype)
    M, N, K = 160, 96, 512          # ragged against the 128 x 128 tile
    w = synth.weights(wtype, g, N, K)
    a = oracle.quantize_q8_1(synth.activations(g, M, K))
    # extreme blocks: all -128 activations against all-15 nibbles / all 127 weights
    a[0, 0, 4:] = np.uint8(0x80)
    got = ops.block_sumi(wtype, _t(w, dev), _t(a, dev), M, N, K, mfma=True).cpu().numpy()
    assert np.array_equal(got, oracle.block_sumi(wtype, a, w, M, N, K))


# ------------------------------------------------------------------ fp32 outputs
@pytest.mark.parametrize("M", [1, 2, 3, 5, 8])
def test_q4_0_gemv_config0(dev, oracle, M):
    """Config 0 shape (N = K = 4096) at the decode batch sizes of the definitions."""
    from ksq import synth
    g = np.random.default_rng(400 + M)
    N, K = 4096, 4096
    w = synth.weights(0, g, N, K)
    x = synth.activations(g, M, K)
    y = _gpu_gemm(dev, 0, w, x, M, N, K)
    ref = oracle.gemm_f64(0, oracle.quantize_q8_1(x), w, M, N, K)
    assert _rel_err(y, ref) <= TOL


@pytest.mark.parametrize("M", [1, 8, 32])
def test_q8_0_config1(dev, oracle, M):
    from ksq import synth
    g = np.random.default_rng(500 + M)
    N, K = 4096, 4096
    w = synth.weights(1, g, N, K)
    x = synth.activations(g, M, K)
    y = _gpu_gemm(dev, 1, w, x, M, N, K)
    ref = oracle.gemm_f64(1, oracle.quantize_q8_1(x), w, M, N, K)
    assert _rel_err(y, ref) <= TOL


@pytest.mark.parametrize("wtype,path", [(w, p) for w in ALL_WTYPES for p in (1, 2)])
def test_paths_agree_small(dev, oracle, wtype, path):
    """Both the v_dot4 and the MFMA path on ragged shapes."""
    from ksq import synth
    g = np.random.default_rng(600 + 10 * wtype + path)
    for M, N, K in ((1, 1, 256), (7, 33, 512), (130, 200, 768), (64, 128, 256), (200, 96, 1024)):
        w = synth.weights(wtype, g, N, K)
        x = synth.activations(g, M, K)
        y = _gpu_gemm(dev, wtype, w, x, M, N, K, path=path)
        ref = oracle.gemm_f64(wtype, oracle.quantize_q8_1(x), w, M, N, K)
        assert _rel_err(y, ref) <= TOL, (M, N, K)


def test_q4_0_prefill_config2_sampled(dev, oracle):
    """Config 2 (M = 2048, N = K = 4096) on the MFMA path; 48 sampled rows against the oracle."""
    from ksq import synth
    g = np.random.default_rng(700)
    M, N, K = 2048, 4096, 4096
    w = synth.weights(0, g, N, K)
    x = synth.activations(g, M, K)
    y = _gpu_gemm(dev, 0, w, x, M, N, K)
    rows = np.sort(g.choice(M, 48, replace=False))
    rows[0], rows[-1] = 0, M - 1
    ref = oracle.gemm_f64(0, oracle.quantize_q8_1(x[rows]), w, len(rows), N, K)
    assert _rel_err(y[rows], ref) <= TOL
    assert np.isfinite(y).all()


@pytest.mark.parametrize("wtype", [2, 3])
def test_kquant_config3_sampled(dev, oracle, wtype):
    """Config 3 shape (M = 128, N = 14336, K = 4096); 16 sampled rows against the oracle."""
    from ksq import synth
    g = np.random.default_rng(800 + wtype)
    M, N, K = 128, 14336, 4096
    w = synth.weights(wtype, g, N, K)
    x = synth.activations(g, M, K)
    y = _gpu_gemm(dev, wtype, w, x, M, N, K)
    rows = np.sort(g.choice(M, 16, replace=False))
    ref = oracle.gemm_f64(wtype, oracle.quantize_q8_1(x[rows]), w, len(rows), N, K)
    assert _rel_err(y[rows], ref) <= TOL


@pytest.mark.parametrize("wtype", ALL_WTYPES)
def test_prequantized_entry_matches_fp32_entry(dev, oracle, wtype):
    """ksq_gemm_*_q8_1 on oracle-quantised activations == the fp32 entry (same bits in)."""
    from ksq import synth
    g = np.random.default_rng(900 + wtype)
    M, N, K = 4, 96, 1024
    w = synth.weights(wtype, g, N, K)
    x = synth.activations(g, M, K)
    y32 = _gpu_gemm(dev, wtype, w, x, M, N, K, atype=0)
    yq = _gpu_gemm(dev, wtype, w, oracle.quantize_q8_1(x), M, N, K, atype=1)
    assert np.array_equal(y32, yq)


def _order_sensitive_rows(g, M, K):
    """fp32 activation rows whose every block has its left-to-right fp32 sum and the sum of its two
    16-element halves' partial sums rounding to different fp16 values (so the s field of
    block_q8_1 pins the reference's summation order), with |d| and |s| inside fp16's range."""
    f16 = np.float16
    out = np.empty((M * K // 32, 32), np.float32)
    n = 0
    while n < out.shape[0]:
        c = (g.standard_normal((4096, 32)) * 10.0 ** g.uniform(-3, 0, (4096, 1))).astype(np.float32)
        i = np.arange(4096)
        big = g.uniform(1e3, 3e4, 4096).astype(np.float32)
        c[i, g.integers(0, 16, 4096)] = big
        c[i, g.integers(16, 32, 4096)] = -big * np.float32(1.0 + 1e-4) * g.choice([1, -1], 4096).astype(np.float32)
        seq = np.add.accumulate(c, axis=1, dtype=np.float32)[:, -1]
        halves = (np.add.accumulate(c[:, :16], axis=1, dtype=np.float32)[:, -1]
                  + np.add.accumulate(c[:, 16:], axis=1, dtype=np.float32)[:, -1]).astype(np.float32)
        keep = c[(seq.astype(f16) != halves.astype(f16)) & np.isfinite(seq.astype(f16))]
        take = min(len(keep), out.shape[0] - n)
        out[n:n + take] = keep[:take]
        n += take
    return out.reshape(M, K)


# (weight type, activation type (0 fp32, 4 fp16), M, N, K, the engines that must quantise in-kernel)
IN_KERNEL_QUANT_CASES = [
    (0, 0, 1, 512, 4096, {"gemv_direct_fq"}),      # lane-pair quantiser, one round
    (0, 0, 2, 512, 4096, {"gemv_direct_fq"}),      # lane pairs, two rounds
    (0, 0, 1, 256, 14336, {"gemv_direct_fq"}),     # lane pairs, 3.5 rounds
    (1, 0, 1, 384, 2048, {"gemv_direct_fq"}),
    (5, 0, 1, 384, 2048, {"gemv_direct_fq"}),
    (0, 0, 4, 512, 2048, {"gemv_mr_fq"}),          # 3-8 rows: a block per lane
    (0, 4, 1, 512, 4096, {"gemv_direct_fq"}),      # fp16 by the fused FP16 kernels' rules
    (0, 4, 2, 512, 2048, {"gemv_direct_fq"}),
]


@pytest.mark.parametrize("wtype,atype,M,N,K,engines", IN_KERNEL_QUANT_CASES)
def test_in_kernel_quantisers_bit_exact(dev, oracle, wtype, atype, M, N, K, engines):
    """The fused fp32 / fp16 entries quantise inside the GEMV workgroups; on blocks whose s field
    depends on the summation order (see _order_sensitive_rows) their output equals, bit for bit,
    the pre-quantised entry's output on the oracle's blocks (quantize_row_q8_1_ref, or the fused
    FP16 quantiser for fp16): the same block bytes went in, and the per-row arithmetic after the
    quantisation is the same code (types without a min term, so no fma contraction differs)."""
    from ksq import ops, synth
    g = np.random.default_rng(2300 + 17 * wtype + M + K + atype)
    w = synth.weights(wtype, g, N, K)
    x = _order_sensitive_rows(g, M, K)
    if atype == 4:
        x = x.astype(np.float16)
        blocks = oracle.quantize_q8_1_variant(x, 3)
    else:
        blocks = oracle.quantize_q8_1(x)
    y = _gpu_gemm(dev, wtype, w, x, M, N, K, atype=atype)
    eng = ops.last_engines()
    yq = _gpu_gemm(dev, wtype, w, blocks, M, N, K, atype=1)
    assert eng == engines, eng
    assert np.isfinite(y).all()
    assert np.array_equal(y, yq)


def test_unaligned_weight_uses_generic_path(dev, oracle):
    """A weight tensor starting 2 bytes into its buffer (blocks are only 2-byte aligned)."""
    import torch
    from ksq import ops, synth
    g = np.random.default_rng(1000)
    M, N, K = 3, 50, 512
    w = synth.weights(0, g, N, K).reshape(-1)
    buf = torch.zeros(w.size + 16, dtype=torch.uint8, device=dev)
    buf[2:2 + w.size] = _t(w, dev)
    x = synth.activations(g, M, K)
    y = ops.gemm(0, 0, buf[2:2 + w.size], _t(x, dev), M, N, K)
    torch.cuda.synchronize()
    ref = oracle.gemm_f64(0, oracle.quantize_q8_1(x), w, M, N, K)
    assert _rel_err(y.cpu().numpy(), ref) <= TOL


def test_k_zero_writes_zeros(dev):
    import torch
    from ksq import ops
    out = torch.full((3, 5), 7.0, device=dev)
    ops.gemm(0, 0, torch.zeros(1, dtype=torch.uint8, device=dev), torch.zeros(4, device=dev), 3, 5, 0, out=out)
    torch.cuda.synchronize()
    assert torch.count_nonzero(out).item() == 0


def test_forward_harness_convention(dev, oracle):
    """forward(weight, activation, M, N, K) as the reference harness calls it, plus its NMSE gate."""
    import torch
    from ksq import forward, synth
    g = np.random.default_rng(1100)
    M, N, K = 8, 4096, 4096
    w = synth.weights(0, g, N, K)
    x = synth.activations(g, M, K)
    y = forward(_t(w, dev), _t(x, dev), M, N, K, entry="gemm_w4a32c8_q4_0_fp32_int8")
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    assert y.shape == (M, N) and y.dtype == np.float32
    ref_deq = x.astype(np.float64) @ oracle.dequantize(0, w.reshape(N, -1), N, K).astype(np.float64).T
    nmse = np.mean((y - ref_deq) ** 2) / np.mean(ref_deq ** 2)
    assert nmse < 0.05           # unified_test_runner.py:411,433-438


# ------------------------------------------------------------------ expert-grouped MoE
def _moe_case(dev, oracle, T, E, N, K, top_k, renorm, seed, wtype=0):
    import torch
    from ksq import ops, synth
    g = np.random.default_rng(seed)
    W = np.stack([synth.weights(wtype, g, N, K) for _ in range(E)])
    x = synth.activations(g, T, K)
    logits = synth.router_logits(g, T, E)
    out, ids, wts = ops.moe_gemm(wtype, _t(W, dev), _t(x, dev), _t(logits, dev), T, N, K, E, top_k, renorm=renorm,
                                 return_routing=True)
    torch.cuda.synchronize()
    ids_ref, wts_ref = oracle.moe_route(logits, top_k, renorm=renorm)
    assert np.array_equal(ids.cpu().numpy(), ids_ref)
    assert np.allclose(wts.cpu().numpy(), wts_ref, rtol=1e-6, atol=0)
    return W, x, logits, out.cpu().numpy(), ids_ref, wts.cpu().numpy()


def test_moe_golden_fixture(dev, oracle):
    import torch
    from ksq import ops
    z = np.load(os.path.join(GOLDEN, "moe_16x4.npz"), allow_pickle=False)
    T, E = z["logits"].shape
    N, K = z["w"].shape[1], z["w"].shape[2] * 32
    top_k = z["ids"].shape[1]
    out, ids, wts = ops.moe_gemm(0, _t(z["w"], dev), _t(z["x"], dev), _t(z["logits"], dev), T, N, K, E, top_k,
                                 return_routing=True)
    torch.cuda.synchronize()
    assert np.array_equal(ids.cpu().numpy(), z["ids"])
    assert _rel_err(out.cpu().numpy(), z["out64"]) <= TOL


@pytest.mark.parametrize("T,E,N,K,top_k,renorm", [(40, 4, 96, 256, 2, False), (37, 8, 160, 512, 3, True),
                                                  (300, 6, 128, 256, 1, False), (400, 2, 300, 512, 2, False),
                                                  (500, 3, 136, 256, 3, True)])
def test_moe_small(dev, oracle, T, E, N, K, top_k, renorm):
    """Small routed MoE cases against the oracle; the last two average 384+ rows per expert, so the
    grouped GEMM runs on 128-row tiles (top_k = 2 by atomics, top_k = 3 through the per-entry
    scratch)."""
    W, x, logits, y, ids, wts = _moe_case(dev, oracle, T, E, N, K, top_k, renorm, 1200 + T)
    ref = oracle.moe_q4_0_f64(W, oracle.quantize_q8_1(x), ids, wts, T, N, K)
    assert _rel_err(y, ref) <= TOL


@pytest.mark.parametrize("T,E,N,K,top_k,renorm", [(1100, 8, 128, 256, 2, False), (200, 64, 96, 256, 2, True),
                                                  (300, 40, 64, 256, 3, False)])
def test_moe_routing_own_launch(dev, oracle, T, E, N, K, top_k, renorm):
    """From T * E = 8192 on, routing runs as its own launch over the chip before the grouping
    workgroup: the same routing as the oracle (ids exact, weights to 1e-6) and the same output as
    the caller-routed entry given those ids (bit for bit at top_k = 2, whose two additions onto zero
    are order-free), within the tolerance of the oracle."""
    import torch
    from ksq import ops
    assert T * E >= 8192   # past the library's threshold (KSQ_MOE_ROUTE_SPLIT_TE)
    W, x, logits, y, ids, wts = _moe_case(dev, oracle, T, E, N, K, top_k, renorm, 1400 + T)
    ref = oracle.moe_q4_0_f64(W, oracle.quantize_q8_1(x), ids, wts, T, N, K)
    assert _rel_err(y, ref) <= TOL
    if top_k == 2:
        y2 = ops.moe_gemm_routed(0, _t(W, dev), _t(x, dev), _t(ids, dev), _t(wts, dev), T, N, K, E)
        torch.cuda.synchronize()
        assert np.array_equal(y, y2.cpu().numpy())


def test_moe_routed_matches_routing_entry(dev, oracle):
    """Caller-supplied routing reproduces the routed entry bit for bit (top_k = 2 sums are order-free)."""
    import torch
    from ksq import ops
    T, E, N, K = 64, 4, 128, 512
    W, x, logits, y, ids, wts = _moe_case(dev, oracle, T, E, N, K, 2, False, 1300)
    y2 = ops.moe_gemm_routed(0, _t(W, dev), _t(x, dev), _t(ids, dev), _t(wts, dev), T, N, K, E)
    torch.cuda.synchronize()
    assert np.array_equal(y, y2.cpu().numpy())


def test_moe_config4_sampled(dev, oracle):
    """Config 4: 512 tokens, 8 experts of 4096 -> 14336 Q4_0, top-2; 12 sampled tokens checked in full."""
    T, E, N, K = 512, 8, 14336, 4096
    W, x, logits, y, ids, wts = _moe_case(dev, oracle, T, E, N, K, 2, False, 1400)
    counts = np.bincount(ids.ravel(), minlength=E)
    assert counts.sum() == T * 2 and (counts > 0).all()
    g = np.random.default_rng(1401)
    toks = np.sort(g.choice(T, 12, replace=False))
    ref = oracle.moe_q4_0_f64(W, oracle.quantize_q8_1(x[toks]), ids[toks], wts[toks], len(toks), N, K)
    assert _rel_err(y[toks], ref) <= TOL
    assert np.isfinite(y).all()


@pytest.mark.parametrize("cfg", [1, 2, 3, 4, 5, 6, 7, 8])
@pytest.mark.parametrize("wtype", ALL_WTYPES)
def test_mfma_tile_configs(dev, oracle, cfg, wtype):
    """Every MFMA tile configuration (K step 4 is not used for K-quants: they take the automatic tile;
    configuration 8 is the LDS-DMA GEMM for Q4_0 / Q4_1, the 128 x 128 tile for the rest)."""
    from ksq import _lib, synth
    g = np.random.default_rng(1500 + 10 * cfg + wtype)
    M, N, K = 150, 136, 512
    w = synth.weights(wtype, g, N, K)
    x = synth.activations(g, M, K)
    _lib.lib().ksq_set_mmq_config(cfg)
    try:
        y = _gpu_gemm(dev, wtype, w, x, M, N, K, path=2)
    finally:
        _lib.lib().ksq_set_mmq_config(0)
    ref = oracle.gemm_f64(wtype, oracle.quantize_q8_1(x), w, M, N, K)
    assert _rel_err(y, ref) <= TOL


SKINNY_WTYPES = [0, 1, 4, 5, 6]          # the 32-element block types of the 4x4x4-MFMA kernel


@pytest.mark.parametrize("wtype", SKINNY_WTYPES)
def test_skinny_small_batch(dev, oracle, wtype):
    """The 4x4x4-MFMA small-batch kernel (path 3) for M = 1..32 on ragged shapes: N not a multiple
    of the 16-row workgroup, K steps with a partial last step (K/32 not a multiple of 4), one K
    step in all, and enough steps for every wave count (4, 8, 16 waves per workgroup)."""
    from ksq import synth
    g = np.random.default_rng(2400 + wtype)
    for M, N, K in ((1, 37, 96), (2, 100, 544), (3, 16, 32), (4, 4096, 4096), (5, 75, 1056), (7, 260, 2048),
                    (8, 1536, 5120), (6, 4100, 4096), (12, 300, 2048), (20, 1040, 4096), (32, 4096, 1024)):
        w = synth.weights(wtype, g, N, K)
        x = synth.activations(g, M, K)
        y = _gpu_gemm(dev, wtype, w, x, M, N, K, path=3)
        ref = oracle.gemm_f64(wtype, oracle.quantize_q8_1(x), w, M, N, K)
        assert _rel_err(y, ref) <= TOL, (M, N, K)


@pytest.mark.parametrize("M", [1, 3, 8, 20])
def test_skinny_q8s_native(dev, oracle, M):
    """Q8_0 weights with block_q8s activations (the native W8A8C8 operator's blocks) on path 3
    (M = 20: the 16x16x32-MFMA form)."""
    from ksq import synth
    g = np.random.default_rng(2500 + M)
    N, K = 530, 2048
    w = synth.weights(1, g, N, K)
    x = synth.activations(g, M, K)
    y = _gpu_gemm(dev, 1, w, x, M, N, K, atype=2, path=3)
    ref = oracle.gemm_q8s_f64(oracle.quantize_q8s(x), w, M, N, K)
    assert _rel_err(y, ref) <= TOL


ENGINE_FAMILIES = {"decode": {"gemv_row", "gemv_row_fq", "gemv_direct", "gemv_direct_fq", "gemv_mr", "gemv_mr_fq",
                               "gemv_kq"},
                   "skinny": {"skinny"}, "mmq": {f"mmq{c}" for c in range(1, 8)} | {"mmq_planar"}}


def _family(engines):
    fams = {f for f, names in ENGINE_FAMILIES.items() if engines & names}
    assert len(fams) == 1, engines
    return fams.pop()


@pytest.mark.parametrize("wtype,M,N,K,expect", [
    (0, 6, 11008, 4096, "skinny"), (4, 5, 18944, 3584, "skinny"), (1, 7, 14336, 4096, "skinny"),
    (0, 8, 4096, 4096, "skinny"), (4, 3, 2560, 2560, "decode"), (0, 3, 4096, 4096, "decode"),
    (0, 2, 7168, 512, "decode"), (1, 4, 9728, 2560, "skinny"), (4, 8, 18944, 3584, "skinny"),
    (0, 5, 3584, 18944, "skinny"), (1, 8, 7168, 7168, "skinny"), (5, 4, 12288, 5120, "skinny"),
    (0, 8, 18432, 7168, "mmq"), (1, 8, 18432, 7168, "skinny"), (0, 6, 5120, 12288, "decode"),
    (1, 8, 512, 7168, "decode"),
    # 9-32 rows: the small-batch kernel where measured faster, else the MFMA GEMM
    (0, 16, 4096, 4096, "skinny"), (1, 12, 4096, 14336, "skinny"), (0, 16, 7168, 7168, "mmq"),
    (1, 24, 4096, 4096, "skinny"), (0, 32, 4096, 4096, "skinny"), (5, 16, 4096, 4096, "skinny"),
    (6, 32, 4096, 4096, "skinny"), (1, 32, 14336, 4096, "mmq"), (1, 32, 7168, 7168, "mmq"), (2, 20, 4096, 4096, "mmq"),
    (2, 8, 4096, 4096, "mmq"), (3, 7, 12288, 5120, "mmq"), (2, 5, 7168, 7168, "decode"),
    (1, 2, 4096, 4096, "decode"), (0, 2, 14336, 4096, "decode"), (2, 5, 12288, 5120, "mmq"),
    (2, 6, 7168, 512, "mmq"), (2, 8, 4096, 1024, "decode")])
def test_small_m_default_routing(dev, oracle, wtype, M, N, K, expect):
    """M = 2..32 by default: large matrices take the MFMA GEMM (the measured crossovers), short
    rows on wide matrices the 4x4x4-MFMA small-batch kernel, the rest the decode kernel (the
    engine family each shape takes is asserted); each way the fp32 entry matches the oracle,
    with the library pool and with a caller workspace of exactly ksq_gemm_workspace_size bytes."""
    import torch
    from ksq import ops, synth
    g = np.random.default_rng(2300 + M)
    w = synth.weights(wtype, g, N, K)
    x = synth.activations(g, M, K)
    wt, xt = _t(w, dev), _t(x, dev)
    y1 = ops.gemm(wtype, 0, wt, xt, M, N, K)
    assert _family(ops.last_engines()) == expect
    ws = torch.empty(max(ops.workspace_size(wtype, 0, M, N, K), 1), dtype=torch.uint8, device=dev)
    y2 = ops.gemm(wtype, 0, wt, xt, M, N, K, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    ref = oracle.gemm_f64(wtype, oracle.quantize_q8_1(x), w, M, N, K)
    assert _rel_err(y1.cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("wtype,M,N,K", [(4, 1, 3584, 18944), (0, 2, 520, 8192), (2, 1, 264, 8192),
                                         (3, 2, 136, 16384), (1, 1, 300, 8704), (5, 2, 200, 8192),
                                         (6, 1, 96, 12288), (1, 1, 100, 18432)])
def test_long_row_decode(dev, oracle, wtype, M, N, K):
    """M = 1, 2 on long rows: from 576 blocks (M = 1) or 256 blocks (M = 2) the decode kernel
    stages the activation rows in LDS once per workgroup instead of reading them per wave, below
    that per wave from L2; fp32 and pre-quantised entries against the oracle."""
    from ksq import ops, synth
    g = np.random.default_rng(2400 + K + M)
    w = synth.weights(wtype, g, N, K)
    x = synth.activations(g, M, K)
    wt, xt = _t(w, dev), _t(x, dev)
    q = oracle.quantize_q8_1(x)
    ref = oracle.gemm_f64(wtype, q, w, M, N, K)
    y = ops.gemm(wtype, 0, wt, xt, M, N, K).cpu().numpy()
    assert _rel_err(y, ref) <= TOL
    yq = ops.gemm(wtype, 1, wt, _t(q, dev), M, N, K).cpu().numpy()
    assert _rel_err(yq, ref) <= TOL


@pytest.mark.parametrize("wtype", [0, 1, 4, 5, 6])
@pytest.mark.parametrize("M", [1, 2])
def test_direct_decode_kernel(dev, oracle, wtype, M):
    """The register-direct decode kernels (1-2 activation rows, block pairs loaded straight into
    VGPRs; pre-quantised activations, or fp32 ones quantised per workgroup): 1, 2, 4 and 8 rows
    per workgroup (8 = two rows per wave), a ragged last workgroup, and the cases they must leave to the LDS kernel (odd
    block count; weights only 2-byte aligned); weights 4 bytes into their buffer still take
    them.  Bars: TOL against the oracle for both entries."""
    import torch
    from ksq import ops, synth
    g = np.random.default_rng(2600 + 10 * wtype + M)
    for N, K, off in ((50, 256, 0), (600, 512, 0), (1101, 2048, 0), (257, 4096, 4), (300, 224, 0),
                      (130, 1024, 2), (2051, 1024, 0), (1000, 14336, 0), (2049, 12288, 0)):
        w = synth.weights(wtype, g, N, K).reshape(-1)
        x = synth.activations(g, M, K)
        q = oracle.quantize_q8_1(x)
        buf = torch.zeros(w.size + 16, dtype=torch.uint8, device=dev)
        buf[off:off + w.size] = _t(w, dev)
        y = ops.gemm(wtype, 1, buf[off:off + w.size], _t(q, dev), M, N, K)
        y32 = ops.gemm(wtype, 0, buf[off:off + w.size], _t(x, dev), M, N, K)
        torch.cuda.synchronize()
        ref = oracle.gemm_f64(wtype, q, w, M, N, K)
        assert _rel_err(y.cpu().numpy(), ref) <= TOL, (N, K, off)
        assert _rel_err(y32.cpu().numpy(), ref) <= TOL, (N, K, off)


@pytest.mark.parametrize("wtype", [0, 1, 4, 5, 6])
@pytest.mark.parametrize("M", [3, 5, 8, 11])
def test_direct_decode_multirow(dev, oracle, wtype, M):
    """The register-direct decode kernel for 3-8 activation rows (LDS-DMA-staged activations,
    decode kernel forced): one and two rows per wave, 1-4 waves per row, K tiles (8 rows of
    224 blocks), a ragged last workgroup, 11 rows as chunks of 8 + 3, and the cases left to
    gemv_row_kernel (odd block count; 256-511 four-row workgroups).  Bar: TOL against the
    oracle."""
    from ksq import synth
    g = np.random.default_rng(2800 + 10 * wtype + M)
    for N, K in ((300, 512), (2051, 1024), (2049, 12288), (1030, 7168), (4100, 224), (1536, 1024), (512, 7168)):
        w = synth.weights(wtype, g, N, K)
        x = synth.activations(g, M, K)
        q = oracle.quantize_q8_1(x)
        y = _gpu_gemm(dev, wtype, w, q, M, N, K, atype=1, path=1)
        ref = oracle.gemm_f64(wtype, q, w, M, N, K)
        assert _rel_err(y, ref) <= TOL, (N, K)
        if M <= 8:
            # the fp32 entry: small grids quantise inside the same kernel (one K tile)
            y32 = _gpu_gemm(dev, wtype, w, x, M, N, K, atype=0, path=0)
            assert _rel_err(y32, ref) <= TOL, (N, K, "fp32")


@pytest.mark.parametrize("M", [3, 5, 8])
def test_direct_decode_multirow_q4_k(dev, oracle, M):
    """The 3-8-row register-direct decode kernel on Q4_K (lane task = the unit pair sharing one
    32-byte quant span, activation pairs staged by LDS DMA): 1-2 rows per wave, 1-4 waves per
    row, K tiles, a ragged last workgroup, and a grid of 256-511 four-row workgroups (left to
    gemv_row_kernel).  Bar: TOL against the oracle."""
    from ksq import synth
    g = np.random.default_rng(2900 + M)
    for N, K in ((300, 512), (2051, 1024), (2049, 12288), (1030, 7168), (1536, 1024), (4100, 7168)):
        w = synth.weights(2, g, N, K)
        x = synth.activations(g, M, K)
        q = oracle.quantize_q8_1(x)
        y = _gpu_gemm(dev, 2, w, q, M, N, K, atype=1, path=1)
        ref = oracle.gemm_f64(2, q, w, M, N, K)
        assert _rel_err(y, ref) <= TOL, (N, K)


@pytest.mark.parametrize("wtype", [2, 3])
@pytest.mark.parametrize("M", [1, 2])
def test_direct_decode_kquant(dev, oracle, wtype, M):
    """The register-direct decode kernel on Q4_K / Q6_K (lane tasks = unit pairs sharing their
    quant bytes; Q6_K super-blocks are 210 bytes, so odd ones are 2-byte aligned and re-aligned
    in registers): 1, 2 and 4 rows per workgroup, odd super-block counts per row, weights 4 bytes
    into their buffer, pre-quantised and fp32 entries.  Bars: TOL against the oracle."""
    import torch
    from ksq import ops, synth
    g = np.random.default_rng(2700 + 10 * wtype + M)
    for N, K, off in ((50, 256, 0), (601, 768, 0), (1101, 2048, 0), (257, 4096, 4), (131, 1280, 4),
                      (1000, 14336, 0)):
        w = synth.weights(wtype, g, N, K).reshape(-1)
        x = synth.activations(g, M, K)
        q = oracle.quantize_q8_1(x)
        buf = torch.zeros(w.size + 16, dtype=torch.uint8, device=dev)
        buf[off:off + w.size] = _t(w, dev)
        y = ops.gemm(wtype, 1, buf[off:off + w.size], _t(q, dev), M, N, K)
        y32 = ops.gemm(wtype, 0, buf[off:off + w.size], _t(x, dev), M, N, K)
        torch.cuda.synchronize()
        ref = oracle.gemm_f64(wtype, q, w, M, N, K)
        assert _rel_err(y.cpu().numpy(), ref) <= TOL, (N, K, off)
        assert _rel_err(y32.cpu().numpy(), ref) <= TOL, (N, K, off)


@pytest.mark.parametrize("wtype,M,N,K", [(0, 1, 7168, 512), (1, 2, 9728, 2560), (4, 3, 4096, 4096),
                                         (6, 4, 2560, 2560), (0, 8, 18944, 3584)])
def test_prequantized_small_m_routing(dev, oracle, wtype, M, N, K):
    """block_q8_1 input at M = 1..8 through the default routing (the small-batch kernel from
    M = 1 on short rows) against the oracle."""
    from ksq import ops, synth
    g = np.random.default_rng(2600 + M)
    w = synth.weights(wtype, g, N, K)
    x = synth.activations(g, M, K)
    q = oracle.quantize_q8_1(x)
    y = ops.gemm(wtype, 1, _t(w, dev), _t(q, dev), M, N, K).cpu().numpy()
    ref = oracle.gemm_f64(wtype, q, w, M, N, K)
    assert _rel_err(y, ref) <= TOL


# ------------------------------------------------------------------ Q4_1 / Q5_0 / Q5_1
def test_golden_fixture_legacy_on_gpu(dev):
    import torch
    from ksq import ops
    z = np.load(os.path.join(GOLDEN, "legacy_q8s_3x5x256.npz"), allow_pickle=False)
    M, K = z["x"].shape
    for wt, name in ((4, "q4_1"), (5, "q5_0"), (6, "q5_1")):
        w = z["w_" + name]
        N = w.shape[0]
        for mfma in (False, True):
            s = ops.block_sumi(wt, _t(w, dev), _t(z["a_q8_1"], dev), M, N, K, mfma=mfma).cpu().numpy()
            assert np.array_equal(s, z["sumi_" + name]), (name, mfma)
        for path in (1, 2):
            y = _gpu_gemm(dev, wt, w, z["x"], M, N, K, path=path)
            assert _rel_err(y, z["c64_" + name]) <= TOL, (name, path)
    q = ops.quantize_q8s(_t(z["x"], dev))
    torch.cuda.synchronize()
    assert np.array_equal(q.cpu().numpy(), z["a_q8s"])


ENTRY_OF = {4: "gemm_w4a32c8_q4_1_fp32_int8", 5: "gemm_w5a32c8_q5_0_fp32_int8", 6: "gemm_w5a32c8_q5_1_fp32_int8"}


@pytest.mark.parametrize("wtype", [4, 5, 6])
@pytest.mark.parametrize("M", [1, 2, 5, 8, 64, 512])
def test_legacy_definition_shapes(dev, oracle, wtype, M):
    """The Q4_1 definitions' shape family (qwen3_4b att_out N = K = 2560; batch_1 .. batch_512) through
    the definition entry point, sampled rows against the fp64 oracle."""
    import torch
    from ksq import forward, synth
    g = np.random.default_rng(1600 + 10 * wtype + M)
    N, K = 2560, 2560
    w = synth.weights(wtype, g, N, K)
    x = synth.activations(g, M, K)
    y = forward(_t(w, dev), _t(x, dev), M, N, K, entry=ENTRY_OF[wtype])
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    rows = np.arange(M) if M <= 8 else np.sort(g.choice(M, 8, replace=False))
    ref = oracle.gemm_f64(wtype, oracle.quantize_q8_1(x[rows]), w, len(rows), N, K)
    assert _rel_err(y[rows], ref) <= TOL


def test_q4_1_harness_flow_nmse(dev, oracle):
    """The harness flow for a w4a32c8_q4_1 definition: fp32 weights -> quantize_to_q4_1, then the
    NMSE gate against dequantise-then-fp32-matmul (reference_q4_1_fp32_gemm, gemm_ref.py:156-199)."""
    import torch
    from ksq import forward
    g = np.random.default_rng(1700)
    M, N, K = 4, 4096, 4096
    wf = g.standard_normal((N, K), dtype=np.float32)
    x = g.standard_normal((M, K), dtype=np.float32)
    w = oracle.quantize_q4_1(wf)
    y = forward(_t(w, dev), _t(x, dev), M, N, K, entry="gemm_w4a32c8_q4_1_fp32_int8")
    torch.cuda.synchronize()
    ref = x.astype(np.float64) @ oracle.dequantize(4, w.reshape(N, -1), N, K).astype(np.float64).T
    nmse = np.mean((y.cpu().numpy() - ref) ** 2) / np.mean(ref ** 2)
    assert nmse < 0.05


@pytest.mark.parametrize("wtype", [4, 5, 6])
def test_moe_legacy_types(dev, oracle, wtype):
    """The grouped MoE GEMM with Q4_1 / Q5_0 / Q5_1 experts: composition of the dense oracle."""
    T, E, N, K, top_k = 48, 4, 96, 512, 2
    W, x, logits, y, ids, wts = _moe_case(dev, oracle, T, E, N, K, top_k, False, 1800 + wtype, wtype=wtype)
    a = oracle.quantize_q8_1(x)
    dense = np.stack([oracle.gemm_f64(wtype, a, W[e], T, N, K) for e in range(E)])
    ref = sum(wts[:, s, None] * dense[ids[:, s], np.arange(T)] for s in range(top_k))
    assert _rel_err(y, ref) <= TOL


# ------------------------------------------------------------------ native W8A8C8 operator
def test_quantize_q8s_bit_exact(dev, oracle):
    import torch
    from ksq import ops
    g = np.random.default_rng(1900)
    for M, K in ((1, 7168), (5, 1024), (513, 96)):
        x = g.standard_normal((M, K), dtype=np.float32)
        if M == 5:
            x[0, :32] = 0.0
            x[1, :6] = [127.0, 2.5, -2.5, 0.5, -126.5, 3.49999976]
            x[1, 6:32] = 0.0
            x[2, 32:64] *= 1e-5
            x[3, 64:96] *= 1e4
        q = ops.quantize_q8s(_t(x, dev))
        torch.cuda.synchronize()
        assert np.array_equal(q.cpu().numpy(), oracle.quantize_q8s(x)), (M, K)


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8, 512])
def test_w8a8c8_native_spec_configs(dev, oracle, M):
    """spec.json test_configs of the native operator (M = 1..8, 512; N = K = 7168 defaults) through its
    own symbol; sampled rows against the fp64 oracle and the operator-order fp32 oracle."""
    import torch
    from ksq import forward, synth
    g = np.random.default_rng(2000 + M)
    N, K = 7168, 7168
    w = synth.weights(1, g, N, K)
    x = synth.activations(g, M, K)
    y = forward(_t(w, dev), _t(x, dev), M, N, K, entry="gemm_w8a8c8_q8_0_q8_1")
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    rows = np.arange(M) if M <= 8 else np.sort(g.choice(M, 6, replace=False))
    a = oracle.quantize_q8s(x[rows])
    ref = oracle.gemm_q8s_f64(a, w, len(rows), N, K)
    assert _rel_err(y[rows], ref) <= TOL
    ref32 = oracle.gemm_w8a8c8(x[rows], w, len(rows), N, K, nthreads=oracle.max_threads())
    assert _rel_err(y[rows], ref32) <= TOL


@pytest.mark.parametrize("path", [1, 2])
def test_w8a8c8_block_dots_and_paths(dev, oracle, path):
    """Integer block dots of the q8s activations are bit-exact on both engines; outputs of both paths."""
    import torch
    from ksq import _lib, ops, synth
    g = np.random.default_rng(2100 + path)
    M, N, K = 70, 96, 512
    w = synth.weights(1, g, N, K)
    x = synth.activations(g, M, K)
    x[3, :64] *= 1e-6
    a = oracle.quantize_q8s(x)
    s = ops.block_sumi(1, _t(w, dev), _t(a, dev), M, N, K, mfma=(path == 2)).cpu().numpy()
    assert np.array_equal(s, oracle.block_sumi(1, a, w, M, N, K))
    y = _gpu_gemm(dev, 1, w, x, M, N, K, atype=_lib.A_F32_Q8S, path=path)
    assert _rel_err(y, oracle.gemm_q8s_f64(a, w, M, N, K)) <= TOL
    yq = _gpu_gemm(dev, 1, w, a, M, N, K, atype=_lib.A_Q8S, path=path)
    assert np.array_equal(y, yq)


# ------------------------------------------------------------------ definition runner
@pytest.mark.parametrize("name", ["w4a32c8_q4_0_fp32_int8_qwen3_4b_att_out_n2560_k2560",
                                  "w4a32c8_q4_1_fp32_int8_qwen3_4b_att_out_n2560_k2560",
                                  "w8a32c8_q8_0_fp32_int8_qwen3_4b_att_out_n2560_k2560"])
def test_runner_definition_end_to_end(dev, tmp_path, name):
    """One definition through ksq.runner: compilation (entry resolved), NMSE gate, exact checks,
    timing, GGML comparison and test_results.json in the reference schema."""
    import json
    from ksq import runner
    d = next(t for t in runner.definitions_table() if t["name"] == name)
    r = runner.DefinitionRunner(warmup=1, iterations=3, log=lambda s: None).run(runner.spec_from_table(d),
                                                                                  str(tmp_path))
    assert r["compilation"]["success"]
    assert r["correctness"]["passed"], r["correctness"]
    for c in r["correctness"]["test_cases"]:
        assert c["exact"]["quantize_bit_exact"] and c["exact"]["block_dots_bit_exact"]
        assert c["exact"]["max_rel_err_vs_fp64"] <= TOL and c["nmse"] < 0.05
    assert [b["config"] for b in r["performance"]["benchmarks"]] == ["single_token", "small_batch", "large_batch"]
    assert all(b["tflops"] > 0 and "ggml" in b for b in r["performance"]["benchmarks"])
    saved = json.load(open(tmp_path / "test_results.json"))
    assert set(saved) >= {"attempt_id", "variant", "op_type", "tested_at", "spec", "compilation", "correctness",
                          "performance"}


def test_runner_native_spec(dev, tmp_path):
    """The native W8A8C8 operator's spec.json form (kernel.entry_point, params defaults N = K = 7168)."""
    from ksq import runner
    spec = {"name": "w8a8c8_q8_0_q8_1", "kernel": {"file": "kernel.cu", "entry_point": "forward"},
            "inputs": {"weight": {"dtype": "block_q8_0"}, "activation": {"dtype": "float32"}},
            "params": {"M": {"type": "int"}, "N": {"default": 7168}, "K": {"default": 7168}},
            "accuracy": {"metric": "nmse", "threshold": 0.05}}
    r = runner.DefinitionRunner(warmup=1, iterations=2, log=lambda s: None).run(spec, str(tmp_path))
    assert r["compilation"]["entry_point"] == "gemm_w8a8c8_q8_0_q8_1"
    assert r["correctness"]["passed"], r["correctness"]


# ------------------------------------------------------------------ split-K MFMA path
@pytest.mark.parametrize("wtype,M,N,K", [(1, 32, 4096, 4096), (0, 16, 512, 7168), (4, 24, 1536, 5120),
                                         (3, 40, 640, 2048), (5, 9, 300, 4096)])
def test_mfma_split_k(dev, oracle, wtype, M, N, K):
    """Small-M grids split along K (partials in the workspace, reduced in split order): the result
    matches the oracle, repeats bit for bit, and is the same with a caller workspace of
    ksq_gemm_workspace_size bytes as with the library pool."""
    import torch
    from ksq import ops, synth
    g = np.random.default_rng(2200 + M)
    w = synth.weights(wtype, g, N, K)
    x = synth.activations(g, M, K)
    wt, xt = _t(w, dev), _t(x, dev)
    ops.set_path(2)
    try:
        y1 = ops.gemm(wtype, 0, wt, xt, M, N, K)
        y2 = ops.gemm(wtype, 0, wt, xt, M, N, K)
        nbytes = ops.workspace_size(wtype, 0, M, N, K)
        assert nbytes >= M * (K // 32) * 36
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        y3 = ops.gemm(wtype, 0, wt, xt, M, N, K, workspace=ws)
        torch.cuda.synchronize()
    finally:
        ops.set_path(0)
    assert torch.equal(y1, y2) and torch.equal(y1, y3)
    rows = np.arange(M) if M <= 16 else np.sort(g.choice(M, 12, replace=False))
    ref = oracle.gemm_f64(wtype, oracle.quantize_q8_1(x[rows]), w, len(rows), N, K)
    assert _rel_err(y1.cpu().numpy()[rows], ref) <= TOL


def test_stream_read_calibration(dev):
    """ksq_debug_stream_read reads every byte: its per-workgroup XOR words match numpy's over the
    same 32 KiB chunks (ragged last chunk included)."""
    import torch
    from ksq import ops
    g = np.random.default_rng(2900)
    for nbytes in (16, 32768, 9437184, 100000 - 100000 % 16):
        a = g.integers(0, 256, nbytes, dtype=np.uint8)
        got = ops.stream_read(_t(a, dev))
        torch.cuda.synchronize()
        words = np.pad(a, (0, (-nbytes) % 32768)).view(np.uint32).reshape(-1, 8192)
        want = np.bitwise_xor.reduce(words, axis=1)
        assert np.array_equal(got.cpu().numpy().view(np.uint32), want), nbytes
    # the per-workgroup size of the read-size curve: 4 KiB (one load per thread) to 256 KiB (rounds of
    # 8 loads per thread), ragged last workgroup included
    for nbytes, wg in ((9437184, 4096), (9437184, 36864), (100000 - 100000 % 16, 65536), (1 << 22, 262144)):
        a = g.integers(0, 256, nbytes, dtype=np.uint8)
        got = ops.stream_read(_t(a, dev), wg_bytes=wg)
        torch.cuda.synchronize()
        words = np.pad(a, (0, (-nbytes) % wg)).view(np.uint32).reshape(-1, wg // 4)
        want = np.bitwise_xor.reduce(words, axis=1)
        assert np.array_equal(got.cpu().numpy().view(np.uint32), want), (nbytes, wg)
