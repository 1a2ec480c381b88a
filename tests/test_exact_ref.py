"""CPU pins of the unit-scale exact reference (k-search_amd/ksq/refcheck.py: exact_gemm,
weight_terms, the K-quant field decoders and the unit-scale input generators) against the C
oracle, which the GPU exactness tests (tests/test_gpu_exact.py) and the definition runner rely on.
"""
import numpy as np
import pytest

ALL = [0, 1, 2, 3, 4, 5, 6]


@pytest.mark.parametrize("wtype", ALL)
def test_exact_gemm_matches_oracle_general(oracle, wtype):
    """Arbitrary (non-unit) scales: the regrouped product equals the oracle's fp64 block formula."""
    from ksq import refcheck, synth
    g = np.random.default_rng(9100 + wtype)
    M, N, K = 5, 7, 512
    w = synth.weights(wtype, g, N, K)
    a = oracle.quantize_q8_1(synth.activations(g, M, K))
    y, bound = refcheck.exact_gemm(wtype, a, w)
    ref = oracle.gemm_f64(wtype, a, w, M, N, K)
    assert np.abs(y - ref).max() <= 1e-12 * np.abs(ref).max()
    assert (bound >= np.abs(y) - 1e-9).all()


@pytest.mark.parametrize("wtype", ALL)
@pytest.mark.parametrize("onehot", [False, True])
def test_unit_scale_inputs_are_exact(oracle, wtype, onehot):
    """fp32 unit activations quantise (by the oracle's quantize_row_q8_1_ref) to d = 1, q = x and
    s = sum(x) on non-zero blocks and to all-zero blocks elsewhere; the exact result then equals
    the oracle's fp64 formula and its reference-order fp32 loop bit for bit."""
    from ksq import refcheck
    g = np.random.default_rng(9200 + wtype + 10 * onehot)
    M, N, K = 9, 24, 1024
    nb = K // 32
    oh = refcheck.onehot_pattern(M, nb, every=2, seed=1) if onehot else None
    w = refcheck.unit_weights(wtype, g, N, K)
    x = refcheck.unit_activations(g, M, K, qmax=12 if wtype in (2, 3) else 127, onehot=oh)
    a = oracle.quantize_q8_1(x)
    d = a[..., 0:2].copy().view(np.float16)[..., 0].astype(np.float64)
    s = a[..., 2:4].copy().view(np.float16)[..., 0].astype(np.float64)
    q = a[..., 4:].view(np.int8).astype(np.float64)
    xb = x.reshape(M, nb, 32).astype(np.float64)
    nz = np.abs(xb).max(axis=-1) > 0
    assert (d[nz] == 1).all() and (d[~nz] == 0).all()
    assert np.array_equal(q, xb) and np.array_equal(s, xb.sum(axis=-1))
    if onehot:
        assert nz[1::2].sum() == (M // 2) and nz[0::2].all()
    y, bound = refcheck.exact_gemm(wtype, a, w)
    assert bound.max() < 2 ** 24
    assert np.array_equal(y, np.round(y))
    assert np.array_equal(y, oracle.gemm_f64(wtype, a, w, M, N, K))
    assert np.array_equal(y.astype(np.float32), oracle.gemm(wtype, a, w, M, N, K))


@pytest.mark.parametrize("wtype", ALL)
def test_unit_q8_1_blocks_are_exact(oracle, wtype):
    """Pre-quantised unit blocks (d = 1, independent s, quants down to -128)."""
    from ksq import refcheck
    g = np.random.default_rng(9300 + wtype)
    M, N, K = 6, 20, 512
    w = refcheck.unit_weights(wtype, g, N, K)
    a = refcheck.unit_q8_1(g, M, K, qmax=15 if wtype in (2, 3) else 128, onehot=refcheck.onehot_pattern(M, K // 32))
    assert (a[..., 4:].view(np.int8) == -128).any() or wtype in (2, 3)
    y, bound = refcheck.exact_gemm(wtype, a, w)
    assert bound.max() < 2 ** 24
    assert np.array_equal(y, oracle.gemm_f64(wtype, a, w, M, N, K))


def test_unit_q8s_blocks_are_exact(oracle):
    """The native W8A8C8 activations: fp32 unit input quantises (its own rules) to d = 1, q = x;
    zero blocks to d = 1 (its d < 1e-6 rule) with zero quants."""
    from ksq import refcheck
    g = np.random.default_rng(9400)
    M, N, K = 5, 16, 512
    w = refcheck.unit_weights(1, g, N, K)
    x = refcheck.unit_activations(g, M, K, qmax=63, onehot=refcheck.onehot_pattern(M, K // 32))
    a = oracle.quantize_q8s(x)
    assert (a[..., 0:4].copy().view(np.float32) == 1).all()
    assert np.array_equal(a[..., 4:].view(np.int8).reshape(M, K).astype(np.float32), x)
    y, _ = refcheck.exact_gemm(1, a, w, q8s=True)
    assert np.array_equal(y, oracle.gemm_q8s_f64(a, w, M, N, K))
    a2 = refcheck.unit_q8s(g, M, K)
    y2, _ = refcheck.exact_gemm(1, a2, w, q8s=True)
    assert np.array_equal(y2, oracle.gemm_q8s_f64(a2, w, M, N, K))


@pytest.mark.parametrize("wtype", [2, 3])
def test_kquant_field_decoders_match_oracle(oracle, wtype):
    """refcheck's K-quant decoders (written from the public layout) give the oracle's dequantised
    values: Weff + the per-sub-block min term (Q4_K) / Weff (Q6_K)."""
    from ksq import refcheck, synth
    g = np.random.default_rng(9500 + wtype)
    N, K = 6, 768
    w = synth.weights(wtype, g, N, K)
    weff, coef = refcheck.weight_terms(wtype, w)
    vals = weff + np.repeat(coef, 32, axis=1)
    ref = oracle.dequantize(wtype, w, N, K).astype(np.float64)
    assert np.allclose(vals, ref, rtol=1e-6, atol=1e-12)


def test_unit_weights_cover_the_fields():
    """Unit weights keep every quant field random: Q4_K 6-bit scales / mins with the high bits
    set, Q6_K negative scales, Q5 high bits, Q4_1 / Q5_1 negative and positive offsets."""
    from ksq import refcheck
    g = np.random.default_rng(9600)
    w = refcheck.unit_weights(2, g, 64, 512)
    s = w[..., 4:16]
    assert (s[..., 0:8] >> 6).any() and (s[..., 8:12] & 0x0F).max() == 15
    w6 = refcheck.unit_weights(3, g, 64, 512)
    assert (w6[..., 192:208].view(np.int8) < 0).any()
    for wt in (4, 6):
        _, m, _ = refcheck.unpack(wt, refcheck.unit_weights(wt, g, 64, 512))
        assert m.min() < 0 < m.max() and np.array_equal(m, np.round(m))


@pytest.mark.parametrize("wtype", [0, 2, 3])
def test_exact_check_sees_a_single_wrong_block(oracle, wtype):
    """A plausible engine mistake confined to one block (its two nibble halves swapped, or for the
    K-quants a sub-block's scale replaced by its neighbour's) changes the exact output of the
    one-hot rows on that block and of the dense rows, so array equality detects it."""
    from ksq import refcheck
    g = np.random.default_rng(9700 + wtype)
    M, N, K = 8, 12, 512
    nb = K // 32
    oh = refcheck.onehot_pattern(M, nb, every=2, seed=0)
    w = refcheck.unit_weights(wtype, g, N, K)
    x = refcheck.unit_activations(g, M, K, qmax=12 if wtype in (2, 3) else 127, onehot=oh)
    a = oracle.quantize_q8_1(x)
    y, _ = refcheck.exact_gemm(wtype, a, w)
    bad = w.copy()
    b = int(oh[1])
    if wtype == 0:
        qs = bad[:, b, 2:18]
        bad[:, b, 2:18] = (qs >> 4) | ((qs & 0x0F) << 4)
    elif wtype == 2:
        sb, j = divmod(b, 8)
        sc = bad[:, sb, 4 + (j % 4)].copy()
        bad[:, sb, 4 + (j % 4)] = bad[:, sb, 4 + ((j + 1) % 4)]
        bad[:, sb, 4 + ((j + 1) % 4)] = sc
    else:
        sb, j = divmod(b, 8)
        bad[:, sb, 192 + 2 * j] = bad[:, sb, 192 + 2 * j] ^ np.uint8(0x01)
    y_bad, _ = refcheck.exact_gemm(wtype, a, bad)
    assert not np.array_equal(y_bad[1], y[1])
    assert not np.array_equal(y_bad[0], y[0])
