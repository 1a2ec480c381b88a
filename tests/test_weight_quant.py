"""The device weight quantisers (ksq_quantize_weights): fp32 -> block_q4_0 / block_q8_0 by the
reference's device kernels quantize_q4_0_kernel / quantize_q8_0_kernel (include/quantize.h:221-297,
rule WQ_DEVICE) or its CPU references quantize_row_q4_0_ref / quantize_row_q8_0_ref
(include/quantize.h:34-68, 110-131, rule WQ_REF).  The oracle's statements are pinned on hand-worked
blocks (rounding ties, NaN, zero blocks), the library is checked against them bit for bit."""
import numpy as np
import pytest


def _q4_nibbles(blk):
    """block_q4_0 bytes -> the 32 quants q (0..15) in element order."""
    qs = np.asarray(blk[2:18], dtype=np.uint8)
    return np.concatenate([qs & 0x0F, qs >> 4]).astype(int)


def _tie_block(scale):
    """amax = 7 * scale / 7 ... : a block whose d is exactly `scale` (d = amax / 7 for Q4_0 with
    amax = 7 * scale), so x * id lands on the listed multiples exactly."""
    x = np.zeros(32, dtype=np.float32)
    x[:6] = np.array([7.0, 2.5, -2.5, 0.5, 1.5, -7.0], dtype=np.float32) * scale
    x[16] = -0.5 * scale
    return x


def test_q4_0_rounding_rules_known_answers(oracle):
    """d = 1: 2.5 -> 2 (half to even) or 3 (roundf); -2.5 -> -2 or -3; 0.5 -> 0 or 1; -0.5 -> 0 or
    -1 (as (int)roundf(-0.5) = -1); 1.5 -> 2 either way; q = value + 8 clamped to [0, 15]."""
    x = _tie_block(1.0)[None, :]
    dev = oracle.quantize_weights(0, x, 0)[0, 0]
    ref = oracle.quantize_weights(0, x, 1)[0, 0]
    assert bytes(dev[:2]) == bytes(ref[:2]) == b"\x00\x3c"          # half(1.0)
    want_dev = [15, 10, 6, 8, 10, 1] + [8] * 10 + [8] + [8] * 15
    want_ref = [15, 11, 5, 9, 10, 1] + [8] * 10 + [7] + [8] * 15
    assert _q4_nibbles(dev).tolist() == want_dev
    assert _q4_nibbles(ref).tolist() == want_ref


def test_q8_0_rounding_rules_known_answers(oracle):
    """d = 1 (amax = 127): 2.5 -> 2 / 3, -0.5 -> 0 / -1, 126.5 -> 126 / 127, -127 -> -127."""
    x = np.zeros((1, 32), dtype=np.float32)
    x[0, :5] = [127.0, 2.5, -0.5, 126.5, -127.0]
    dev = oracle.quantize_weights(1, x, 0)[0, 0]
    ref = oracle.quantize_weights(1, x, 1)[0, 0]
    assert bytes(dev[:2]) == bytes(ref[:2]) == b"\x00\x3c"
    assert dev[2:7].astype(np.int8).tolist() == [127, 2, 0, 126, -127]
    assert ref[2:7].astype(np.int8).tolist() == [127, 3, -1, 127, -127]


def test_weight_quant_nan_and_zero_blocks(oracle):
    """A NaN element: fmaxf / std::max skip it for amax; its product converts to 0 on the device
    (Q4_0 q = 8, Q8_0 q = 0) and to INT32_MIN through the x86 (int) cast (Q4_0 clamps to 0, Q8_0
    to -128).  An all-zero block: d = 0, id = 0, every q = 0 (+ 8 for Q4_0), half(0) = 0."""
    x = np.zeros((2, 32), dtype=np.float32)
    x[0, :3] = [7.0, np.nan, 1.0]
    for rule, q4_nan, q8_nan in ((0, 8, 0), (1, 0, -128)):
        b4 = oracle.quantize_weights(0, x, rule)
        assert _q4_nibbles(b4[0, 0])[:3].tolist() == [15, q4_nan, 9]
        assert bytes(b4[1, 0][:2]) == b"\x00\x00" and _q4_nibbles(b4[1, 0]).tolist() == [8] * 32
        b8 = oracle.quantize_weights(1, x * np.float32(127.0 / 7.0), rule)
        assert b8[0, 0][3].astype(np.int8) == q8_nan
        assert bytes(b8[1, 0][:2]) == b"\x00\x00" and not b8[1, 0][2:].any()


def test_weight_quant_rules_agree_off_ties(oracle):
    """Away from exact .5 products and NaN the two rules round alike, so on random data they agree
    byte for byte (a dropped +8, a swapped nibble order or a wrong divisor in one of them fails)."""
    g = np.random.default_rng(77)
    x = (g.standard_normal((64, 512)) * np.exp2(g.integers(-10, 10, (64, 1)))).astype(np.float32)
    for wt in (0, 1):
        assert np.array_equal(oracle.quantize_weights(wt, x, 0), oracle.quantize_weights(wt, x, 1))
    # Q8_0 dequantises to within half a step of x, plus the step's fp16 rounding (q = x / d with
    # the fp32 d, stored as half(d): |q| <= 127 steps off by at most 2^-11 each)
    xs = (g.standard_normal((64, 512)) * np.exp2(g.integers(0, 6, (64, 1)))).astype(np.float32)
    b = oracle.quantize_weights(1, xs, 0)
    d = np.repeat(b[:, :, :2].copy().view(np.float16)[:, :, 0].astype(np.float32), 32, axis=1)
    deq = b[:, :, 2:].astype(np.int8).astype(np.float32).reshape(64, 512) * d
    assert np.all(np.abs(deq - xs) <= (0.5 + 127.0 * 2.0 ** -11) * d)


def test_weight_quant_abi_rejects_bad_arguments():
    from ksq import _lib
    L = _lib.lib()
    assert L.ksq_quantize_weights(2, 0, None, None, 64, None) == 4      # KSQ_ERR_TYPE: Q4_K
    assert L.ksq_quantize_weights(0, 2, None, None, 64, None) == 4      # unknown rule
    assert L.ksq_quantize_weights(0, 0, None, None, 48, None) == 2      # KSQ_ERR_SHAPE: k % 32
    assert L.ksq_quantize_weights(0, 0, None, None, 64, None) == 1      # KSQ_ERR_NULL
    assert L.ksq_quantize_weights(1, 1, None, None, 0, None) == 0       # empty: no-op


@pytest.fixture(scope="module")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


@pytest.mark.gpu
@pytest.mark.parametrize("wtype", [0, 1])
@pytest.mark.parametrize("rule", [0, 1])
def test_gpu_weight_quant_bit_exact(dev, oracle, wtype, rule):
    """ksq_quantize_weights against the oracle's statement of the same rule, bit for bit: random
    rows over magnitudes 2^-20 .. 2^11, the tie / NaN / zero blocks above, an infinite element
    (d = inf, id = 0, inf * 0 = NaN), and a block whose d is a tiny subnormal."""
    import torch
    from ksq import ops
    g = np.random.default_rng(900 + 2 * wtype + rule)
    x = (g.standard_normal((48, 1024)) * np.exp2(g.integers(-20, 12, (48, 1)))).astype(np.float32)
    x[0, :32] = _tie_block(1.0)
    x[1, :32] = _tie_block(2.0 ** -6)
    x[2, :3] = [7.0, np.nan, 1.0]
    x[2, 3:32] = 0.0
    x[3, :32] = 0.0
    x[4, 5] = np.inf
    x[5, :32] = 0.0
    x[5, 7] = np.float32(1e-44)
    q = ops.quantize_weights(wtype, torch.from_numpy(x).to(dev), rule)
    torch.cuda.synchronize()
    want = oracle.quantize_weights(wtype, x, rule)
    assert np.array_equal(q.cpu().numpy(), want)


@pytest.mark.gpu
def test_gpu_weight_quant_feeds_the_gemm(dev, oracle):
    """Weights quantised on the device run through the GEMM exactly as the oracle's blocks do."""
    import torch
    import ksq
    from ksq import ops
    g = np.random.default_rng(901)
    M, N, K = 16, 256, 512
    w = g.standard_normal((N, K)).astype(np.float32)
    x = g.standard_normal((M, K)).astype(np.float32)
    for wt in (0, 1):
        qw = ops.quantize_weights(wt, torch.from_numpy(w).to(dev), 0)
        y = ops.gemm(wt, ksq.A_F32, qw, torch.from_numpy(x).to(dev), M, N, K)
        y2 = ops.gemm(wt, ksq.A_F32, torch.from_numpy(oracle.quantize_weights(wt, w, 0)).to(dev),
                      torch.from_numpy(x).to(dev), M, N, K)
        torch.cuda.synchronize()
        assert torch.equal(y, y2)
