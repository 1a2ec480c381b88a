"""Pins for the CPU oracle (oracle/ksq_oracle.c).  CPU only.

The reference ships no golden vectors for this path (its tests grade by NMSE
only), so the oracle is pinned by exhaustive/closed-form checks, independent
numpy formulations (tests/npref.py), hand-computed known answers and the
committed fixtures under tests/golden/.
"""
import os

import numpy as np
import pytest

import npref

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# ---------------------------------------------------------------- fp16
def test_f16_to_f32_exhaustive(oracle):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_bits_to_f32(int(v)) for v in h], dtype=np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_rne(oracle):
    g = np.random.default_rng(1)
    # every binary16 exponent range incl. subnormals, overflow and exact ties
    x = (g.standard_normal(200000) * np.exp2(g.integers(-30, 20, 200000))).astype(np.float32)
    ties = (np.arange(1, 4000, dtype=np.float32) + np.float32(0.5)) * np.float32(2.0 ** -14)
    special = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e6, -1e6, 2.0 ** -24, 2.0 ** -25,
                        2.0 ** -25 * 1.0000001, 2.0 ** -26, 5.960464477539063e-08, np.inf, -np.inf],
                       dtype=np.float32)
    x = np.concatenate([x, ties, -ties, special])
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    got = np.array([oracle.f32_to_f16_bits(float(v)) for v in x], dtype=np.uint16)
    assert np.array_equal(got, want)


# ---------------------------------------------------------------- Q8_1 quantiser
def test_quantize_q8_1_matches_numpy_restatement(oracle):
    g = np.random.default_rng(2)
    x = g.standard_normal((16, 1024), dtype=np.float32)
    x[3, :32] = 0.0                                   # zero block
    x[5, 32:64] *= 1e-30                              # tiny but normal amax
    x[7, 64:96] *= 3e4                                # |sum| beyond 65504: s rounds to +-inf
    with np.errstate(over="ignore"):
        assert np.array_equal(oracle.quantize_q8_1(x), npref.quantize_q8_1(x))


def test_quantize_q8_1_known_answers(oracle):
    # amax = 127 -> d = 1, id = 1 exactly: q = roundf(x) and the ties show the rounding mode
    blk = np.zeros(32, dtype=np.float32)
    blk[:8] = [127.0, 2.5, -2.5, 0.5, -0.5, 1.5, -126.5, 3.49999976]
    q = oracle.quantize_q8_1(blk[None, :])[0, 0]
    d = np.frombuffer(q[0:2].tobytes(), np.float16)[0]
    s = np.frombuffer(q[2:4].tobytes(), np.float16)[0]
    qs = q[4:].view(np.int8)
    assert d == np.float16(1.0)
    assert s == np.float16(np.float32(127 + 2.5 - 2.5 + 0.5 - 0.5 + 1.5 - 126.5 + 3.49999976))
    # half away from zero (roundf), not half-even (rint / __float2int_rn / np.round)
    assert list(qs[:8]) == [127, 3, -3, 1, -1, 2, -127, 3]
    assert np.all(qs[8:] == 0)
    # zero block: d = 0, s = 0, q = 0 (the C++ rule; the numpy harness quantiser uses d = 1)
    z = oracle.quantize_q8_1(np.zeros((1, 32), np.float32))[0, 0]
    assert np.all(z == 0)


def test_q8_1_variant_device_kernel(oracle):
    """quantize_q8_1_kernel (quantize.h:301-336): against a numpy restatement with np.rint and
    a cumsum sequential sum, plus the ties that separate it from quantize_row_q8_1_ref."""
    g = np.random.default_rng(40)
    x = g.standard_normal((16, 1024), dtype=np.float32) * np.exp2(g.integers(-20, 12, (16, 1))).astype(np.float32)
    x[3, :32] = 0.0
    x[7, 64:96] *= 3e4
    assert np.array_equal(oracle.quantize_q8_1_variant(x, 1), npref.quantize_q8_1_device_rint(x))
    blk = np.zeros((1, 32), dtype=np.float32)
    blk[0, :8] = [127.0, 2.5, -2.5, 0.5, -0.5, 1.5, -126.5, 3.49999976]
    qs = oracle.quantize_q8_1_variant(blk, 1)[0, 0, 4:].view(np.int8)
    assert list(qs[:8]) == [127, 2, -2, 0, 0, 2, -126, 3]          # half to even
    assert list(oracle.quantize_q8_1_variant(blk, 0)[0, 0, 4:12].view(np.int8)) == [127, 3, -3, 1, -1, 2, -127, 3]
    assert np.all(oracle.quantize_q8_1_variant(np.zeros((1, 32), np.float32), 1) == 0)
    # an infinite input: amax = d = inf, id = 0, inf * 0 = NaN converts to 0 on the device
    inf = np.zeros((1, 32), dtype=np.float32)
    inf[0, 0], inf[0, 1] = np.inf, 3.0
    q = oracle.quantize_q8_1_variant(inf, 1)[0, 0]
    assert np.all(q[4:] == 0) and q[0:2].view(np.float16)[0] == np.inf


def test_q8_1_variant_numpy_harness(oracle):
    """quantize_to_q8_1 (llm_kernel_test/reference/quantize.py:165-214): bit for bit against
    NumPy running the harness' own expressions (NumPy fixes the pairwise sum order, the
    float32 true division and the half-even round), over magnitudes from 2^-20 to 2^11."""
    g = np.random.default_rng(41)
    x = g.standard_normal((64, 1024), dtype=np.float32) * np.exp2(g.integers(-20, 12, (64, 1))).astype(np.float32)
    x[3, :32] = 0.0                                    # d = 1 for the all-zero block
    x[9, 32:64] *= 3e4
    assert np.array_equal(oracle.quantize_q8_1_variant(x, 2), npref.quantize_q8_1_numpy_harness(x))
    z = oracle.quantize_q8_1_variant(np.zeros((1, 32), np.float32), 2)[0, 0]
    assert z[0:2].view(np.float16)[0] == np.float16(1.0) and np.all(z[2:] == 0)
    blk = np.zeros((1, 32), dtype=np.float32)
    blk[0, :6] = [127.0, 2.5, -2.5, 0.5, -0.5, 1.5]
    assert list(oracle.quantize_q8_1_variant(blk, 2)[0, 0, 4:10].view(np.int8)) == [127, 2, -2, 0, 0, 2]
    # blocks whose fp16 s differs between NumPy's pairwise order and a left-to-right sum:
    # the oracle follows NumPy on each
    g2 = np.random.default_rng(7)
    hits = []
    while len(hits) < 3:
        b = (g2.standard_normal(32) * np.exp2(g2.integers(-6, 10, 32))).astype(np.float32)
        if np.sum(b).astype(np.float16) != np.cumsum(b, dtype=np.float32)[-1].astype(np.float16):
            hits.append(b)
    for b in hits:
        got = oracle.quantize_q8_1_variant(b[None, :], 2)[0, 0, 2:4].view(np.float16)[0]
        assert got == np.sum(b).astype(np.float16)


def test_q8_1_variant_fused_f16(oracle):
    """quantize_fp16_to_q8_1_smem (gemm_fused.cuh:76-145): fp16 input, q from 1/half(d),
    roundf, clamp +-127.  Checked on blocks whose sums are exact in any order against a numpy
    statement, on ties, and on a value where 1/half(d) and 1/d round differently.  The tree
    order of the sum: test_q8_1_variant_fused_f16_tree_sum."""
    g = np.random.default_rng(42)
    # multiples of 2^-8 below 2^7: every partial sum of 32 is exact in fp32
    xi = g.integers(-2 ** 15, 2 ** 15, (32, 256)).astype(np.float32) * np.float32(2.0 ** -8)
    x = xi.astype(np.float16)
    got = oracle.quantize_q8_1_variant(x, 3)
    a = x.astype(np.float32).reshape(32, 8, 32)
    d = (np.abs(a).max(axis=2) / np.float32(127.0)).astype(np.float32)
    dh = d.astype(np.float16)
    idv = (np.float32(1.0) / dh.astype(np.float32)).astype(np.float32)
    y = (a * idv[:, :, None]).astype(np.float64)
    q = (np.sign(y) * np.floor(np.abs(y) + 0.5)).clip(-127, 127).astype(np.int8)
    assert np.array_equal(got[:, :, 0:2].view(np.float16)[:, :, 0], dh)
    assert np.array_equal(got[:, :, 2:4].view(np.float16)[:, :, 0], a.sum(axis=2, dtype=np.float64).astype(np.float16))
    assert np.array_equal(got[:, :, 4:].view(np.int8), q)
    blk = np.zeros((1, 32), dtype=np.float16)
    blk[0, :6] = [127.0, 2.5, -2.5, 0.5, -0.5, -127.0]
    assert list(oracle.quantize_q8_1_variant(blk, 3)[0, 0, 4:10].view(np.int8)) == [127, 3, -3, 1, -1, -127]
    # 1/half(d) against 1/d: amax = 100 -> d = 0.787401..., half(d) = 0.78759766
    d32 = np.float32(100.0) / np.float32(127.0)
    i_h = np.float32(1.0) / np.float32(np.float16(d32))
    i_d = np.float32(1.0) / d32
    cand = np.arange(-100.0, 100.0, 2.0 ** -4).astype(np.float16).astype(np.float32)
    rh = np.floor(np.abs(cand * i_h) + 0.5)
    rd = np.floor(np.abs(cand * i_d) + 0.5)
    v = cand[np.flatnonzero(rh != rd)[0]]
    blk = np.zeros((1, 32), dtype=np.float16)
    blk[0, 0], blk[0, 1] = 100.0, v
    q1 = int(oracle.quantize_q8_1_variant(blk, 3)[0, 0, 5].view(np.int8))
    assert abs(q1) == int(np.floor(np.abs(v * i_h) + 0.5)) != int(np.floor(np.abs(v * i_d) + 0.5))


def test_quantize_q8_1_amax_maps_to_127(oracle):
    g = np.random.default_rng(3)
    x = g.standard_normal((64, 256), dtype=np.float32)
    q = oracle.quantize_q8_1(x).reshape(64 * 8, 36)
    qs = q[:, 4:].view(np.int8).astype(int)
    xb = x.reshape(64 * 8, 32)
    i = np.abs(xb).argmax(axis=1)
    assert np.all(np.abs(qs[np.arange(len(i)), i]) == 127)
    assert np.all(np.sign(qs[np.arange(len(i)), i]) == np.sign(xb[np.arange(len(i)), i]))


# ---------------------------------------------------------------- integer block dots
def _q4_0_block(d, qs):
    b = np.zeros(18, np.uint8)
    b[0:2] = np.array([d], np.float16).view(np.uint8)
    b[2:] = qs
    return b


def _q8_1_block(d, s, qa):
    b = np.zeros(36, np.uint8)
    b[0:2] = np.array([d], np.float16).view(np.uint8)
    b[2:4] = np.array([s], np.float16).view(np.uint8)
    b[4:] = np.asarray(qa, np.int8).view(np.uint8)
    return b


def test_sumi_q4_0_known_answers(oracle):
    L = oracle.lib()
    p = lambda a: a.ctypes.data  # noqa: E731
    w15 = _q4_0_block(1.0, np.full(16, 0xFF, np.uint8))
    assert L.ksq_ref_sumi_q4_0_q8_1(p(w15), p(_q8_1_block(1, 0, [127] * 32))) == 15 * 127 * 32
    assert L.ksq_ref_sumi_q4_0_q8_1(p(w15), p(_q8_1_block(1, 0, [-128] * 32))) == -61440
    # qs[i] = i | (15 - i) << 4: element k<16 is k, element k>=16 is 31-k
    wi = _q4_0_block(1.0, np.array([i | ((15 - i) << 4) for i in range(16)], np.uint8))
    assert L.ksq_ref_sumi_q4_0_q8_1(p(wi), p(_q8_1_block(1, 0, [1] * 32))) == 240
    # qa[k] = k: sum_k<16 k*k + sum_k<16 (k+16)*(15-k) = 1240 + 2480 = 3720
    assert L.ksq_ref_sumi_q4_0_q8_1(p(wi), p(_q8_1_block(1, 0, list(range(32))))) == 3720
    # qa[k] = k for k < 16 only: 1240 for the low/high split order; the consecutive-pair
    # nibble order (the bug in gemm_cuda_dp4a.cuh:119-143) would give 932
    qa = [k if k < 16 else 0 for k in range(32)]
    assert L.ksq_ref_sumi_q4_0_q8_1(p(wi), p(_q8_1_block(1, 0, qa))) == 1240
    assert sum(k * ((k // 2) if k % 2 == 0 else 15 - k // 2) for k in range(16)) == 932


def test_sumi_matches_bruteforce(oracle):
    from ksq import synth
    g = np.random.default_rng(4)
    for wtype in (0, 1):
        M, N, K = 3, 5, 256
        w = synth.weights(wtype, g, N, K)
        a = oracle.quantize_q8_1(synth.activations(g, M, K) * 3)
        assert np.array_equal(oracle.block_sumi(wtype, a, w, M, N, K), npref.sumi(wtype, a, w))


# ---------------------------------------------------------------- GEMM
@pytest.mark.parametrize("wtype", [0, 1])
def test_gemm_matches_fp64_block_formula(oracle, wtype):
    from ksq import synth
    g = np.random.default_rng(5 + wtype)
    M, N, K = 4, 8, 512
    w = synth.weights(wtype, g, N, K)
    a = oracle.quantize_q8_1(synth.activations(g, M, K))
    ref = npref.gemm_f64(wtype, a, w)
    c32 = oracle.gemm(wtype, a, w, M, N, K)
    c64 = oracle.gemm_f64(wtype, a, w, M, N, K)
    assert np.allclose(c64, ref, rtol=1e-12, atol=1e-12 * np.abs(ref).max())
    assert np.abs(c32 - ref).max() <= 1e-5 * np.abs(ref).max()
    # a transposed product or a dropped s-term would not agree
    assert not np.allclose(c32.T[:4, :4], ref[:4, :4], rtol=1e-3)


def test_gemm_q4_0_near_dequant_matmul(oracle):
    """The harness' fp32 oracle (dequantise W, fp32 matmul; gemm_ref.py:51-97) agrees to quantisation noise."""
    from ksq import synth
    g = np.random.default_rng(7)
    M, N, K = 4, 64, 1024
    w = synth.weights(0, g, N, K)
    x = synth.activations(g, M, K)
    c = oracle.gemm(0, oracle.quantize_q8_1(x), w, M, N, K)
    ref = x.astype(np.float64) @ oracle.dequantize(0, w.reshape(N, -1), N, K).astype(np.float64).T
    nmse = np.mean((c - ref) ** 2) / np.mean(ref ** 2)
    assert nmse < 1e-3        # the harness threshold is 0.05 (unified_test_runner.py:411)


def test_golden_fixtures(oracle):
    """Committed vectors (tests/golden/make_golden.py) still reproduce."""
    path = os.path.join(GOLDEN, "q4_0_q8_1_small.npz")
    z = np.load(path, allow_pickle=False)
    a = oracle.quantize_q8_1(z["x"])
    assert np.array_equal(a, z["a_q8_1"])
    M, K = z["x"].shape
    N = z["w_q4_0"].shape[0]
    assert np.array_equal(oracle.block_sumi(0, a, z["w_q4_0"], M, N, K), z["sumi_q4_0"])
    assert np.array_equal(oracle.gemm(0, a, z["w_q4_0"], M, N, K), z["c_q4_0"])
    assert np.array_equal(oracle.block_sumi(1, a, z["w_q8_0"], M, N, K), z["sumi_q8_0"])
    assert np.array_equal(oracle.gemm(1, a, z["w_q8_0"], M, N, K), z["c_q8_0"])


def test_golden_fixtures_legacy_q8s(oracle):
    z = np.load(os.path.join(GOLDEN, "legacy_q8s_3x5x256.npz"), allow_pickle=False)
    x = z["x"]
    M, K = x.shape
    a = oracle.quantize_q8_1(x)
    assert np.array_equal(a, z["a_q8_1"])
    for wt, name in ((4, "q4_1"), (5, "q5_0"), (6, "q5_1")):
        w = z["w_" + name]
        N = w.shape[0]
        assert np.array_equal(oracle.block_sumi(wt, a, w, M, N, K), z["sumi_" + name])
        assert np.array_equal(oracle.gemm(wt, a, w, M, N, K), z["c_" + name])
        assert np.allclose(oracle.gemm_f64(wt, a, w, M, N, K), npref.gemm_legacy_f64(wt, a, w), rtol=1e-12)
    w8 = z["w_q8_0"]
    N = w8.shape[0]
    assert np.array_equal(oracle.quantize_q8s(x), z["a_q8s"])
    assert np.array_equal(npref.quantize_q8s(x), z["a_q8s"])
    assert np.array_equal(oracle.gemm_w8a8c8(x, w8, M, N, K), z["c_w8a8c8"])
    assert np.array_equal(oracle.quantize_q4_1(z["wf"]), z["w_q4_1_from_fp32"])
    assert np.array_equal(npref.quantize_q4_1(z["wf"]), z["w_q4_1_from_fp32"])


# ---------------------------------------------------------------- K-quants
def test_q4_K_encoder_decoder_round_trip(oracle):
    g = np.random.default_rng(8)
    for _ in range(20):
        sc = g.integers(0, 64, 8)
        mn = g.integers(0, 64, 8)
        q = g.integers(0, 16, 256)
        d, dmin = np.float16(abs(g.standard_normal()) * 0.02), np.float16(abs(g.standard_normal()) * 0.02)
        blk = npref.encode_q4_K(d, dmin, sc, mn, q)
        for j in range(8):
            assert oracle.q4_K_scale_min(j, blk[4:16]) == (sc[j], mn[j])
        y = oracle.dequantize(2, blk[None, :], 1, 256)[0]
        d32, m32 = np.float32(d), np.float32(dmin)
        want = np.array([(d32 * np.float32(sc[e // 32])) * np.float32(q[e]) - m32 * np.float32(mn[e // 32])
                         for e in range(256)], np.float32)
        assert np.array_equal(y, want)


def test_q6_K_encoder_decoder_round_trip(oracle):
    g = np.random.default_rng(9)
    for _ in range(20):
        sc = g.integers(-128, 128, 16)
        q = g.integers(0, 64, 256)
        d = np.float16(abs(g.standard_normal()) * 0.002)
        blk = npref.encode_q6_K(d, sc, q)
        y = oracle.dequantize(3, blk[None, :], 1, 256)[0]
        want = np.array([np.float32(d) * np.float32(sc[e // 16]) * np.float32(q[e] - 32) for e in range(256)],
                        np.float32)
        assert np.array_equal(y, want)


def test_q4_K_zero_scales_and_single_subblock(oracle):
    g = np.random.default_rng(10)
    x = g.standard_normal((1, 256), dtype=np.float32)
    a = oracle.quantize_q8_1(x)
    q = g.integers(0, 16, 256)
    blk = npref.encode_q4_K(0.5, 0.25, np.zeros(8, int), np.zeros(8, int), q)
    assert oracle.gemm(2, a, blk[None, :], 1, 1, 256)[0, 0] == 0.0
    sc = np.zeros(8, int); sc[3] = 5
    mn = np.zeros(8, int); mn[3] = 7
    blk = npref.encode_q4_K(0.5, 0.25, sc, mn, q)
    da, sa, qa = npref.unpack_q8_1(a[0])
    want = 0.5 * da[3] * 5 * int(np.dot(q[96:128], qa[3])) - 0.25 * sa[3] * 7
    assert abs(oracle.gemm(2, a, blk[None, :], 1, 1, 256)[0, 0] - want) <= 1e-6 * abs(want)


@pytest.mark.parametrize("wtype", [2, 3])
def test_kquant_gemm_vs_encoded_fields(oracle, wtype):
    """Integer-sum oracle path vs fp64 dot of fields drawn before encoding."""
    g = np.random.default_rng(11 + wtype)
    M, N, K = 3, 4, 512
    nsb = K // 256
    x = g.standard_normal((M, K), dtype=np.float32)
    a = oracle.quantize_q8_1(x)
    da, sa, qa = npref.unpack_q8_1(a)                 # [M, nb], [M, nb], [M, nb, 32]
    aval = (da[..., None] * qa).reshape(M, K)
    w = np.zeros((N, nsb, 144 if wtype == 2 else 210), np.uint8)
    want = np.zeros((M, N))
    for n in range(N):
        for s in range(nsb):
            if wtype == 2:
                sc, mn, q = g.integers(0, 64, 8), g.integers(0, 64, 8), g.integers(0, 16, 256)
                d, dmin = np.float16(0.01 + 0.01 * g.random()), np.float16(0.01 + 0.01 * g.random())
                w[n, s] = npref.encode_q4_K(d, dmin, sc, mn, q)
                wsc = float(d) * np.repeat(sc, 32) * q                   # scale part per element
                want[:, n] += aval[:, 256 * s:256 * (s + 1)] @ wsc
                want[:, n] -= float(dmin) * (sa[:, 8 * s:8 * (s + 1)] @ mn)
            else:
                sc, q = g.integers(-128, 128, 16), g.integers(0, 64, 256)
                d = np.float16(0.001 + 0.001 * g.random())
                w[n, s] = npref.encode_q6_K(d, sc, q)
                want[:, n] += aval[:, 256 * s:256 * (s + 1)] @ (float(d) * np.repeat(sc, 16) * (q - 32))
    c64 = oracle.gemm_f64(wtype, a, w, M, N, K)
    c32 = oracle.gemm(wtype, a, w, M, N, K)
    assert np.allclose(c64, want, rtol=1e-10, atol=1e-10 * np.abs(want).max())
    assert np.abs(c32 - want).max() <= 1e-5 * np.abs(want).max()


# ---------------------------------------------------------------- MoE
def test_moe_route_and_composition(oracle):
    from ksq import synth
    g = np.random.default_rng(12)
    T, E, N, K, k = 16, 4, 32, 256, 2
    logits = synth.router_logits(g, T, E)
    logits[0, 1] = logits[0, 2] = 5.0                          # tie -> lower index first
    ids, wts = oracle.moe_route(logits, k)
    assert list(ids[0]) == [1, 2]
    order = np.argsort(-logits, axis=1, kind="stable")[:, :k]
    assert np.array_equal(ids, order)
    p = np.exp(logits - logits.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    assert np.allclose(wts, np.take_along_axis(p, order, 1), rtol=1e-6)
    _, wren = oracle.moe_route(logits, k, renorm=True)
    assert np.allclose(wren.sum(1), 1.0, rtol=1e-6)
    # composition with the dense oracle
    W = np.stack([synth.weights(0, g, N, K) for _ in range(E)])
    a = oracle.quantize_q8_1(synth.activations(g, T, K))
    out = oracle.moe_q4_0_f64(W, a, ids, wts, T, N, K)
    dense = np.stack([oracle.gemm_f64(0, a, W[e], T, N, K) for e in range(E)])   # [E, T, N]
    want = sum(wts[:, s, None] * dense[ids[:, s], np.arange(T)] for s in range(k))
    assert np.allclose(out, want, rtol=1e-12, atol=1e-12 * np.abs(want).max())
    counts = np.bincount(ids.ravel(), minlength=E)
    assert counts.sum() == T * k


# ---------------------------------------------------------------- Q4_1 / Q5_0 / Q5_1
LEGACY = (4, 5, 6)


@pytest.mark.parametrize("wtype", LEGACY)
def test_legacy_known_answer_blocks(oracle, wtype):
    """Blocks encoded from chosen fields (npref.encode_legacy) decode to d*q + m / (q-16)*d, and
    the integer dot against a ramp is the hand-computable sum."""
    q = np.array([(7 * e + 3) % (16 if wtype == 4 else 32) for e in range(32)])
    d, m = 0.125, -1.5
    blk = npref.encode_legacy(wtype, d, m, q)
    y = oracle.dequantize(wtype, blk[None, :], 1, 32)[0]
    want = (q - 16) * d if wtype == 5 else q * d + m
    assert np.array_equal(y, want.astype(np.float32))
    qa = np.arange(32) - 16
    a = _q8_1_block(1.0, 0.0, qa)
    assert oracle.sumi_legacy(wtype, blk, a) == int(np.dot(q, qa))
    # element order: a ramp over the first 16 activations only sees the low nibbles / qh bits 0..15
    a16 = _q8_1_block(1.0, 0.0, [k if k < 16 else 0 for k in range(32)])
    assert oracle.sumi_legacy(wtype, blk, a16) == int(np.dot(q[:16], np.arange(16)))


@pytest.mark.parametrize("wtype", (5, 6))
def test_legacy_qh_bit_order(oracle, wtype):
    """Only element e has bit 4 set: the dot with a one-hot activation at e sees 16, elsewhere 0."""
    for e in (0, 7, 8, 15, 16, 23, 31):
        q = np.zeros(32, int)
        q[e] = 16
        blk = npref.encode_legacy(wtype, 1.0, 0.0, q)
        for k in (e, (e + 1) % 32, (e + 16) % 32):
            qa = np.zeros(32, int)
            qa[k] = 1
            assert oracle.sumi_legacy(wtype, blk, _q8_1_block(1.0, 0.0, qa)) == (16 if k == e else 0)


@pytest.mark.parametrize("wtype", LEGACY)
def test_legacy_sumi_and_gemm_vs_numpy(oracle, wtype):
    from ksq import synth
    g = np.random.default_rng(20 + wtype)
    M, N, K = 4, 6, 512
    w = synth.weights(wtype, g, N, K)
    a = oracle.quantize_q8_1(synth.activations(g, M, K) * 2)
    _, _, qw = npref.unpack_legacy(wtype, w)
    _, _, qa = npref.unpack_q8_1(a)
    assert np.array_equal(oracle.block_sumi(wtype, a, w, M, N, K), np.einsum("mbk,nbk->mnb", qa, qw))
    ref = npref.gemm_legacy_f64(wtype, a, w)
    c64 = oracle.gemm_f64(wtype, a, w, M, N, K)
    c32 = oracle.gemm(wtype, a, w, M, N, K)
    assert np.allclose(c64, ref, rtol=1e-12, atol=1e-12 * np.abs(ref).max())
    assert np.abs(c32 - ref).max() <= 1e-5 * np.abs(ref).max()
    if wtype != 5:
        # the reference's "m * s8 / 4" (gemm_quant_formats.cuh:148, :266) is not what the harness computes
        dw, mw, _ = npref.unpack_legacy(wtype, w)
        _, sa, _ = npref.unpack_q8_1(a)
        quarter = ref - 0.75 * np.einsum("nb,mb->mn", mw, sa)
        assert np.abs(c32 - quarter).max() > 1e-2 * np.abs(ref).max()


@pytest.mark.parametrize("wtype", LEGACY)
def test_legacy_formula_vs_dequantised_matmul(oracle, wtype):
    """sum_b (d q + m) . x over the original fp32 x: the s term carries the exact block sums, so the
    integer formula equals the dequantised product up to the activation quantisation noise."""
    from ksq import synth
    g = np.random.default_rng(30 + wtype)
    M, N, K = 3, 16, 1024
    w = synth.weights(wtype, g, N, K)
    x = synth.activations(g, M, K)
    c = oracle.gemm(wtype, oracle.quantize_q8_1(x), w, M, N, K)
    ref = x.astype(np.float64) @ oracle.dequantize(wtype, w.reshape(N, -1), N, K).astype(np.float64).T
    assert np.mean((c - ref) ** 2) / np.mean(ref ** 2) < 1e-3


def test_quantize_q4_1_matches_harness_restatement(oracle):
    g = np.random.default_rng(40)
    x = g.standard_normal((8, 512), dtype=np.float32)
    x[1, :32] = 0.25                                   # constant block: scale 1, all q = 0
    x[2, 32:64] = np.linspace(-1, 1, 32, dtype=np.float32)
    assert np.array_equal(oracle.quantize_q4_1(x), npref.quantize_q4_1(x))
    y = oracle.dequantize(4, oracle.quantize_q4_1(x).reshape(8, -1), 8, 512)
    xb, yb = x.reshape(-1, 32), y.reshape(-1, 32)
    span = xb.max(1) - xb.min(1)
    assert np.all(np.abs(xb - yb).max(1) <= span / 15 * 0.5 + 2e-3 * (np.abs(xb).max(1) + span))


@pytest.mark.parametrize("wtype", (5, 6))
def test_quantize_q5_round_trip(oracle, wtype):
    g = np.random.default_rng(41 + wtype)
    x = g.standard_normal((8, 256), dtype=np.float32)
    q = oracle.quantize_q5_0(x) if wtype == 5 else oracle.quantize_q5_1(x)
    y = oracle.dequantize(wtype, q.reshape(8, -1), 8, 256).reshape(-1, 32)
    xb = x.reshape(-1, 32)
    # Q5_0 covers [-16, 15] steps with the largest magnitude at -16: a value of the opposite
    # sign and equal magnitude clamps to 15, one full step off; elsewhere half a step
    step = np.abs(xb).max(1) / 16 if wtype == 5 else (xb.max(1) - xb.min(1)) / 31
    bound = step * (1.0 if wtype == 5 else 0.5)
    assert np.all(np.abs(xb - y).max(1) <= bound + 2e-3 * np.abs(xb).max(1) + 1e-6)
    if wtype == 5:
        inner = np.abs(xb) < 0.9 * np.abs(xb).max(1, keepdims=True)
        assert np.all(np.where(inner, np.abs(xb - y), 0).max(1) <= step * 0.5 + 2e-3 * np.abs(xb).max(1) + 1e-6)


# ---------------------------------------------------------------- native W8A8C8 operator
def test_quantize_q8s_matches_numpy_restatement(oracle):
    g = np.random.default_rng(50)
    x = g.standard_normal((16, 512), dtype=np.float32)
    x[3, :32] = 0.0                                    # zero block -> d = 1, q = 0
    x[4, 32:64] *= 1e-5                                # amax/127 < 1e-6 -> d = 1, q = round(x) = 0
    x[5, 64:96] *= 1e4
    assert np.array_equal(oracle.quantize_q8s(x), npref.quantize_q8s(x))


def test_quantize_q8s_known_answers(oracle):
    blk = np.zeros(32, np.float32)
    blk[:6] = [127.0, 2.5, -2.5, 0.5, -126.5, 3.49999976]      # d = 1 exactly: ties round away from zero
    q = oracle.quantize_q8s(blk[None, :])[0, 0]
    assert q[0:4].view(np.float32)[0] == np.float32(1.0)
    assert list(q[4:10].view(np.int8)) == [127, 3, -3, 1, -127, 3]
    tiny = np.full((1, 32), 1e-5, np.float32)
    t = oracle.quantize_q8s(tiny)[0, 0]
    assert t[0:4].view(np.float32)[0] == np.float32(1.0) and np.all(t[4:] == 0)
    # true division: find x where x / d and x * (1/d) round to different integers
    g = np.random.default_rng(51)
    found = 0
    for _ in range(20000):
        amax = np.float32(g.uniform(0.5, 2.0))
        d = np.float32(amax / np.float32(127))
        k = int(g.integers(1, 127))
        x = np.float32((k + 0.5) * d)
        for cand in (x, np.nextafter(x, np.float32(0)), np.nextafter(x, np.float32(9))):
            by_div = np.float64(np.float32(cand / d))
            by_mul = np.float64(np.float32(cand * np.float32(np.float32(1) / d)))
            if np.floor(by_div + 0.5) != np.floor(by_mul + 0.5):
                b = np.zeros((1, 32), np.float32)
                b[0, 0], b[0, 1] = amax, cand
                got = int(oracle.quantize_q8s(b)[0, 0, 5].view(np.int8))
                assert got == int(np.floor(by_div + 0.5))
                found += 1
    assert found > 0


def test_gemm_w8a8c8_composition(oracle):
    """The whole operator (per-output re-quantisation) equals quantise-once then the block formula."""
    from ksq import synth
    g = np.random.default_rng(52)
    M, N, K = 5, 7, 512
    w = synth.weights(1, g, N, K)
    x = synth.activations(g, M, K)
    x[1, :64] *= 1e-6
    c = oracle.gemm_w8a8c8(x, w, M, N, K)
    a = oracle.quantize_q8s(x)
    c64 = oracle.gemm_q8s_f64(a, w, M, N, K)
    d_a = a[..., 0:4].copy().view(np.float32)[..., 0].astype(np.float64)
    dw, qw = npref.unpack_q8_0(w)
    qa = a[..., 4:].view(np.int8).astype(np.int64)
    want = np.einsum("nb,mb,mnb->mn", dw, d_a, np.einsum("mbk,nbk->mnb", qa, qw).astype(np.float64))
    assert np.allclose(c64, want, rtol=1e-12, atol=1e-12 * np.abs(want).max())
    assert np.abs(c - want).max() <= 1e-5 * np.abs(want).max()
    # a Q8_1 (fp16 scale) activation path is a different operator: it differs at the fp16 level
    q81 = oracle.gemm(1, oracle.quantize_q8_1(x), w, M, N, K)
    assert np.abs(q81 - want).max() > 1e-7 * np.abs(want).max()


# ---- byte-literal K-quant super-blocks (written from the public GGML field description) ----
# Q4_K: {fp16 d, fp16 dmin, u8 scales[12], u8 qs[128]}; value of element 64g + 32h + l
# = d * sc_j * q - dmin * m_j, j = 2g + h, q = low (h = 0) or high (h = 1) nibble of qs[32g + l];
# 6-bit (sc_j, m_j): j < 4 in the low 6 bits of scales[j] / scales[j + 4]; j >= 4 low 4 bits in
# scales[j + 4] (sc low nibble, m high nibble), top 2 bits in the top 2 bits of scales[j - 4] (sc)
# and scales[j] (m).  Chosen fields: d = 1, dmin = 0.5,
#   sc = 1, 2, 3, 4, 37, 46, 55, 63      m = 5, 6, 7, 8, 17, 29, 42, 60
# packed by hand:
#   scales[0..3]  = 1|2<<6, 2|2<<6, 3|3<<6, 4|3<<6         = 0x81 0x82 0xC3 0xC4
#   scales[4..7]  = 5|1<<6, 6|1<<6, 7|2<<6, 8|3<<6         = 0x45 0x46 0x87 0xC8
#   scales[8..11] = 5|1<<4, 14|13<<4, 7|10<<4, 15|12<<4     = 0x15 0xDE 0xA7 0xCF
# qs: group g bytes 0x15, 0x26, 0x37, 0x48 (low nibble 5 + g, high 1 + g) except byte l = 31 of
# every group, 0x9A (low 10, high 9).
Q4_K_LITERAL = bytes([0x00, 0x3C, 0x00, 0x38,
                      0x81, 0x82, 0xC3, 0xC4, 0x45, 0x46, 0x87, 0xC8, 0x15, 0xDE, 0xA7, 0xCF]
                     + [0x15] * 31 + [0x9A] + [0x26] * 31 + [0x9A] + [0x37] * 31 + [0x9A] + [0x48] * 31 + [0x9A])
# hand-computed values per sub-block j for l < 31 and l = 31:
#   j0 1*5-2.5=2.5  1*10-2.5=7.5 | j1 2*1-3=-1    2*9-3=15     | j2 3*6-3.5=14.5  3*10-3.5=26.5
#   j3 4*2-4=4      4*9-4=32     | j4 37*7-8.5=250.5 37*10-8.5=361.5 | j5 46*3-14.5=123.5 46*9-14.5=399.5
#   j6 55*8-21=419  55*10-21=529 | j7 63*4-30=222 63*9-30=537
Q4_K_VALUES = [(2.5, 7.5), (-1.0, 15.0), (14.5, 26.5), (4.0, 32.0), (250.5, 361.5), (123.5, 399.5),
               (419.0, 529.0), (222.0, 537.0)]
# Q6_K: {u8 ql[128], u8 qh[64], i8 scales[16], fp16 d}; element 128n + 32Q + l of half n, quarter Q:
# q = 4 bits of ql (Q0: low of ql[64n+l], Q1: low of ql[64n+32+l], Q2: high of ql[64n+l], Q3:
# high of ql[64n+32+l]) | bits 2Q, 2Q+1 of qh[32n+l] as bits 4-5; value d * sc[8n + 2Q + l/16] * (q - 32).
# Chosen: d = 0.25; ql half 0 = 0x21 x32, 0x43 x32; half 1 = 0x65 x32, 0x87 x32 except ql[5] = 0x2F;
# qh half 0 = 0xE4 (Q0..Q3 high bits 0, 1, 2, 3), half 1 = 0x1B (3, 2, 1, 0);
# scales = -128 127 -3 5 -7 11 -13 17 19 -23 29 -31 37 -41 43 -47.
# So q - 32: half 0 Q0..Q3 = 1-32, 19-32, 34-32, 52-32 = -31 -13 2 20; half 1 = 53-32, 39-32, 22-32,
# 8-32 = 21 7 -10 -24; element 5 (ql 0x2F): 15-32 = -17.
Q6_K_LITERAL = bytes([0x2F if i == 5 else 0x21 for i in range(32)] + [0x43] * 32 + [0x65] * 32 + [0x87] * 32
                     + [0xE4] * 32 + [0x1B] * 32
                     + [0x80, 0x7F, 0xFD, 0x05, 0xF9, 0x0B, 0xF3, 0x11, 0x13, 0xE9, 0x1D, 0xE1, 0x25, 0xD7, 0x2B, 0xD1]
                     + [0x00, 0x34])
# hand-computed values for the 16 sixteen-element sub-blocks (0.25 * sc * (q - 32)); element 5: 0.25*-128*-17
Q6_K_VALUES = [992.0, -984.25, 9.75, -16.25, -3.5, 5.5, -65.0, 85.0,
               99.75, -120.75, 50.75, -54.25, -92.5, 102.5, -258.0, 282.0]


def test_q4_K_byte_literal(oracle):
    """The oracle's Q4_K decoder on a hand-packed super-block: distinct scales and mins in all 16
    six-bit slots (high bits of j >= 4 included) and distinct quants per group and half, so a
    swapped scale/min high-bit source, a swapped nibble/sub-block pairing or a wrong group order
    each changes some value."""
    assert len(Q4_K_LITERAL) == 144
    blk = np.frombuffer(Q4_K_LITERAL, dtype=np.uint8)
    sc = [1, 2, 3, 4, 37, 46, 55, 63]
    mn = [5, 6, 7, 8, 17, 29, 42, 60]
    for j in range(8):
        assert oracle.q4_K_scale_min(j, blk[4:16]) == (sc[j], mn[j])
    got = oracle.dequantize(2, blk[None, None, :], 1, 256)[0]
    want = np.empty(256)
    for j, (v, v31) in enumerate(Q4_K_VALUES):
        want[32 * j:32 * j + 32] = v
        want[32 * j + 31] = v31
    assert np.array_equal(got.astype(np.float64), want)
    # integer block dot of sub-block 4 against an all-ones Q8_1 block (d = 1, s = 32): 31*7 + 10
    a = np.zeros((1, 8, 36), np.uint8)
    a[..., 0:2] = np.array([1.0], np.float16).view(np.uint8)
    a[..., 2:4] = np.array([32.0], np.float16).view(np.uint8)
    a[..., 4:] = 1
    assert oracle.block_sumi(2, a, blk[None, None, :], 1, 1, 256)[0, 0].tolist() == \
        [31 * 5 + 10, 31 * 1 + 9, 31 * 6 + 10, 31 * 2 + 9, 31 * 7 + 10, 31 * 3 + 9, 31 * 8 + 10, 31 * 4 + 9]


def test_q6_K_byte_literal(oracle):
    """The oracle's Q6_K decoder on a hand-packed super-block: distinct ql nibbles and qh bit pairs
    per quarter and half, sixteen distinct int8 scales (-128 and 127 included), so a swapped quarter
    order, qh bit pair, scale index or half changes some value."""
    assert len(Q6_K_LITERAL) == 210
    blk = np.frombuffer(Q6_K_LITERAL, dtype=np.uint8)
    got = oracle.dequantize(3, blk[None, None, :], 1, 256)[0].astype(np.float64)
    want = np.repeat(np.array(Q6_K_VALUES), 16)
    want[5] = 0.25 * -128 * -17
    assert np.array_equal(got, want)
    a = np.zeros((1, 8, 36), np.uint8)
    a[..., 0:2] = np.array([1.0], np.float16).view(np.uint8)
    a[..., 4:] = 1
    s = oracle.block_sumi(3, a, blk[None, None, :], 1, 1, 256)[0, 0]
    # sixteen-element sums of (q - 32): half 0 -31, -13, 2, 20 per quarter; element 5 is -17
    assert s.tolist()[:8] == [15 * -31 + -17, 16 * -31, 16 * -13, 16 * -13, 16 * 2, 16 * 2, 16 * 20, 16 * 20]
    assert s.tolist()[8:] == [16 * 21, 16 * 21, 16 * 7, 16 * 7, 16 * -10, 16 * -10, 16 * -24, 16 * -24]


def test_q8_1_variant_fused_f16_tree_sum(oracle):
    """The fused FP16 quantiser's s is the shared-memory tree of gemm_fused.cuh:93-121 (x[i] + x[i+16],
    then + 8, + 4, + 2 apart, then s0 + s1, all fp32): on blocks whose fp16 s differs between that
    tree and a left-to-right fp32 sum, the oracle follows the tree (restated here by halving)."""
    g = np.random.default_rng(43)

    def tree(b):
        v = b.astype(np.float32)
        while v.size > 1:
            h = v.size // 2
            v = (v[:h] + v[h:]).astype(np.float32)
        return v[0]

    hits = 0
    for _ in range(20000):
        # one 2048 and a +-1 or 3 (an fp16 rounding tie of s near 2049) among fp16-subnormal-scale
        # values that a left-to-right fp32 sum absorbs one by one but the tree adds up first
        bf = np.zeros(32, np.float32)
        bf[g.integers(0, 32)] = 2048.0
        bf[g.integers(0, 32)] += np.float32(g.choice([1.0, 3.0, -1.0]))
        small = g.integers(1, 4, size=32) * np.float32(2.0 ** -14) * g.choice([-1, 1], size=32)
        bf = np.where((bf == 0) & (g.random(32) < 0.8), small, bf).astype(np.float32)
        b = bf.astype(np.float16)
        bf = b.astype(np.float32)
        t, seq = np.float32(tree(bf)).astype(np.float16), np.cumsum(bf, dtype=np.float32)[-1].astype(np.float16)
        if t == seq:
            continue
        got = oracle.quantize_q8_1_variant(b[None, :], 3)[0, 0, 2:4].view(np.float16)[0]
        assert got == t, (got, t, seq)
        hits += 1
        if hits == 5:
            break
    assert hits == 5


# ---- block_q8f: fp32 d_a and s_a (deepseek_v2 operator reference.py:50-73; lm_head kernel.cu:85-107)

def _q8f_fields(blk):
    blk = np.ascontiguousarray(blk)
    return blk[0:4].view(np.float32)[0], blk[4:8].view(np.float32)[0], blk[8:40].view(np.int8)


def test_quantize_q8f_known_answers(oracle):
    """Hand-computed blocks: with amax = 127 both rules have d = 1 and differ only in how ties
    round (reference.py's round(): half to even; lroundf: half away from zero)."""
    blk = np.zeros((1, 32), np.float32)
    blk[0, :8] = [127.0, 2.5, -2.5, 3.5, 0.5, -0.5, -126.5, 1.25]
    d, s, q = _q8f_fields(oracle.quantize_q8f(blk, 0)[0, 0])
    assert d == 1.0 and s == 5.25
    assert list(q[:8]) == [127, 2, -2, 4, 0, 0, -126, 1] and not q[8:].any()
    d, s, q = _q8f_fields(oracle.quantize_q8f(blk, 1)[0, 0])
    assert d == 1.0 and s == 5.25
    assert list(q[:8]) == [127, 3, -3, 4, 1, -1, -127, 1] and not q[8:].any()
    # all-zero block: d = 1 (reference.py: `if a_max > 0 else 1.0`; kernel.cu: a_max > 1e-10)
    for rule in (0, 1):
        d, s, q = _q8f_fields(oracle.quantize_q8f(np.zeros((1, 32), np.float32), rule)[0, 0])
        assert d == 1.0 and s == 0.0 and not q.any()


def test_quantize_q8f_tiny_block(oracle):
    """0 < amax <= 1e-10: the deepseek_v2 rule keeps d = amax/127; the lm_head rule sets d = 1
    while its scale is 127/1e-10, so the quants stay non-zero (kernel.cu:88-89)."""
    blk = np.zeros((1, 32), np.float32)
    blk[0, 0], blk[0, 1] = 1e-12, -4e-13
    d, _, q = _q8f_fields(oracle.quantize_q8f(blk, 0)[0, 0])
    assert d == np.float32(1e-12) / np.float32(127.0) and q[0] == 127 and q[1] == -51   # -50.8
    d, _, q = _q8f_fields(oracle.quantize_q8f(blk, 1)[0, 0])
    assert d == 1.0 and q[0] == 1 and q[1] == -1                                         # 1.27, -0.508


def test_quantize_q8f_fp32_fields_and_sequential_sum(oracle):
    """d and s are stored as fp32 (no fp16 rounding) and s is the left-to-right fp32 sum: with
    1e8, seven 1s and -1e8 every 1 is absorbed (the ulp of 1e8 is 8), giving 0 where NumPy's
    pairwise sum and the exact sum give 7."""
    blk = np.zeros((1, 32), np.float32)
    blk[0, :9] = [1e8, 1, 1, 1, 1, 1, 1, 1, -1e8]
    for rule in (0, 1):
        _, s, _ = _q8f_fields(oracle.quantize_q8f(blk, rule)[0, 0])
        assert s == 0.0 and float(np.sum(blk)) == 7.0
    blk = np.zeros((1, 32), np.float32)
    blk[0, :2] = [1.0, 0.0001]
    for rule in (0, 1):
        d, s, _ = _q8f_fields(oracle.quantize_q8f(blk, rule)[0, 0])
        assert d != np.float32(np.float16(d)) and s != np.float32(np.float16(s))
        assert s == np.float32(1.0001) or s == np.float32(1.0) + np.float32(0.0001)


def test_quantize_q8f_division_vs_scale(oracle):
    """The deepseek_v2 rule divides by d (a_val / d_a); the lm_head rule multiplies by 127/amax.
    Blocks where the two give different integers pin which one each rule uses."""
    g = np.random.default_rng(61)
    seen = {0: 0, 1: 0}
    for _ in range(20000):
        amax = np.float32(g.uniform(0.5, 2.0))
        d = np.float32(amax / np.float32(127))
        scale = np.float32(np.float32(127) / amax)
        k = int(g.integers(1, 127))
        x = np.float32((k + 0.5) * d)
        lo, hi = np.nextafter(x, np.float32(0)), np.nextafter(x, np.float32(9))
        for cand in (x, lo, hi, np.nextafter(lo, np.float32(0)), np.nextafter(hi, np.float32(9))):
            by_div = float(np.float32(cand / d))
            by_mul = float(np.float32(cand * scale))
            rne_div, away_mul = round(by_div), int(np.floor(by_mul + 0.5))
            if rne_div != int(np.floor(by_div + 0.5)) or away_mul != round(by_mul):
                continue   # a tie: covered by the known-answer test
            b = np.zeros((1, 32), np.float32)
            b[0, 0], b[0, 1] = amax, cand
            if round(by_div) != round(by_mul):
                assert int(_q8f_fields(oracle.quantize_q8f(b, 0)[0, 0])[2][1]) == rne_div
                assert int(_q8f_fields(oracle.quantize_q8f(b, 1)[0, 0])[2][1]) == away_mul
                seen[0] += 1
    assert seen[0] > 0


def _int_weights(wtype, g, N, K):
    """Q4_0 / Q5_0 / Q8_0 weights with d = 1 and their integer values [N, K] decoded by hand
    from the byte layout (element j < 16 in the low nibble of qs[j], j >= 16 in the high one)."""
    nb = K // 32
    if wtype == 0:
        w = np.zeros((N, nb, 18), np.uint8)
        w[..., 0:2] = np.frombuffer(np.float16(1).tobytes(), np.uint8)
        w[..., 2:18] = g.integers(0, 256, size=(N, nb, 16), dtype=np.uint8)
        qs = w[..., 2:18].astype(np.int64)
        vals = np.concatenate([qs & 15, qs >> 4], axis=-1) - 8
    elif wtype == 5:
        w = np.zeros((N, nb, 22), np.uint8)
        w[..., 0:2] = np.frombuffer(np.float16(1).tobytes(), np.uint8)
        w[..., 2:22] = g.integers(0, 256, size=(N, nb, 20), dtype=np.uint8)
        qh = w[..., 2:6].astype(np.int64)
        hbit = np.stack([(qh[..., j // 8] >> (j % 8)) & 1 for j in range(32)], axis=-1)
        qs = w[..., 6:22].astype(np.int64)
        vals = np.concatenate([qs & 15, qs >> 4], axis=-1) + 16 * hbit - 16
    else:
        w = np.zeros((N, nb, 34), np.uint8)
        w[..., 0:2] = np.frombuffer(np.float16(1).tobytes(), np.uint8)
        w[..., 2:34] = g.integers(-128, 128, size=(N, nb, 32)).astype(np.int8).view(np.uint8)
        vals = w[..., 2:34].view(np.int8).astype(np.int64)
    return w, vals.reshape(N, K)


@pytest.mark.parametrize("wtype", [0, 5, 1])
@pytest.mark.parametrize("rule", [0, 1])
def test_gemm_q8f_unit_scale_is_integer_matmul(oracle, wtype, rule):
    """Unit scales (d_w = 1; integer activations with one +-127 per block, so d_a = 1, q_a = x
    and s_a = sum x exactly): every block term d_w*(d_a*sumi - c*s_a) is the integer
    sum_k x_k * (q_k - c), so the fp32 oracle must equal x @ values^T exactly."""
    g = np.random.default_rng(70 + wtype + 10 * rule)
    M, N, K = 5, 7, 256
    w, vals = _int_weights(wtype, g, N, K)
    x = g.integers(-20, 21, size=(M, K // 32, 32)).astype(np.float32)
    x[:, :, 3] = 127.0
    x = x.reshape(M, K)
    a = oracle.quantize_q8f(x, rule)
    assert np.all(a[..., 0:4].copy().view(np.float32) == 1.0)
    y = oracle.gemm_q8f(wtype, a, w, M, N, K)
    want = x.astype(np.int64) @ vals.T
    assert np.array_equal(y, want.astype(np.float32))
    assert np.array_equal(oracle.gemm_q8f(wtype, a, w, M, N, K, f64=True), want.astype(np.float64))


def test_gemm_q8f_fp32_order_vs_fp64(oracle):
    """Random scales: the fp32 block-order accumulation stays within fp32 rounding of the fp64 one,
    and the fp64 one is the dequantised product d_a*q_a . d_w*(q_w - 8) plus the -8*d_w*s_a term
    computed from the fields in numpy."""
    from ksq import refcheck
    g = np.random.default_rng(80)
    M, N, K = 6, 9, 512
    x = g.standard_normal((M, K)).astype(np.float32)
    w = oracle.quantize_q4_0(g.standard_normal((N, K)).astype(np.float32)).reshape(N, K // 32, 18)
    for rule in (0, 1):
        a = oracle.quantize_q8f(x, rule)
        y32 = oracle.gemm_q8f(0, a, w, M, N, K)
        y64 = oracle.gemm_q8f(0, a, w, M, N, K, f64=True)
        A, s = refcheck.act_terms(a)
        d, _, q = refcheck.unpack(0, w)
        want = A @ (d[..., None] * q).reshape(N, K).T - 8.0 * s @ d.T
        assert np.allclose(y64, want, rtol=1e-12, atol=1e-9)
        assert np.max(np.abs(y32 - y64)) <= 1e-5 * np.max(np.abs(y64))


# ---- W4A16 / W8A16 dequantise-then-fp32 (gemm_reference.h:73-147)

@pytest.mark.parametrize("wtype", [0, 1])
def test_gemm_w16_integer_inputs_exact(oracle, wtype):
    """Integer activations and d = 1: every product and partial sum is an exact integer, so the
    oracle must equal the integer matmul with the weights decoded by hand (pins which nibble is
    which element: element k < 16 = low nibble of qs[k], k >= 16 = high nibble of qs[k - 16])."""
    g = np.random.default_rng(90 + wtype)
    M, N, K = 4, 6, 320
    w, vals = _int_weights(wtype, g, N, K)
    x = g.integers(-50, 51, size=(M, K)).astype(np.float32)
    assert np.array_equal(oracle.gemm_w16(wtype, x, w, M, N, K), (x.astype(np.int64) @ vals.T).astype(np.float32))


def test_gemm_w4a16_interleaved_order(oracle):
    """gemm_w4a16_reference adds element k then element k + 16 (k = 0..15), not k ascending:
    with A[0] = 1e8, A[16] = 1, A[1] = -1e8 and every dequantised weight 1, its fp32 sum is
    1e8 + 1 -> 1e8 (absorbed), then - 1e8 -> 0, where ascending order gives 1."""
    w = np.zeros((1, 1, 18), np.uint8)
    w[0, 0, 0:2] = np.frombuffer(np.float16(1).tobytes(), np.uint8)
    w[0, 0, 2:18] = 0x99                      # every quant 9: value 9 - 8 = 1
    x = np.zeros((1, 32), np.float32)
    x[0, 0], x[0, 16], x[0, 1] = 1e8, 1.0, -1e8
    assert oracle.gemm_w16(0, x, w, 1, 1, 32)[0, 0] == 0.0
    assert float(np.float32(np.float32(1e8) - np.float32(1e8)) + np.float32(1.0)) == 1.0


@pytest.mark.parametrize("wtype", [0, 1])
def test_gemm_w16_vs_dequantised_matmul(oracle, wtype):
    """Random fp32 activations: the oracle's fp32 loop within fp32 accumulation error of the fp64
    product of the activations with the weights dequantised in numpy (gemm_ref.py:51-97's form)."""
    from ksq import refcheck
    g = np.random.default_rng(95 + wtype)
    M, N, K = 5, 7, 1024
    x = g.standard_normal((M, K)).astype(np.float32)
    quant = oracle.quantize_q4_0 if wtype == 0 else oracle.quantize_q8_0
    w = quant(g.standard_normal((N, K)).astype(np.float32)).reshape(N, K // 32, -1)
    ref = x.astype(np.float64) @ refcheck.dequantize(wtype, w).T
    y = oracle.gemm_w16(wtype, x, w, M, N, K)
    bound = np.abs(x.astype(np.float64)) @ np.abs(refcheck.dequantize(wtype, w)).T
    assert np.all(np.abs(y - ref) <= 2.0 ** -24 * K * bound)
