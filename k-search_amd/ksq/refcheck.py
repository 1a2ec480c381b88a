"""Numpy checks used by the definition runner (ksq.runner) to verify libksq outputs.

These are the exact checks of the quantized-matmul path, restated in numpy so the
runner can verify a result on the machine it runs on:

  quantize_q8_1       quantize_row_q8_1_ref (kernelevalplus-main/include/quantize.h:165-193):
                      d = amax/127 (fp32), id = 1/d, q = clamp(roundf(x*id)), sequential
                      fp32 sum, d and sum stored as fp16
  block_sumi          the per-block integer dots of gemm_reference.h:200-212 / :253-256 and
                      kernels/gemm/gemm_quant_formats.cuh:126-137, :170-200, :230-257
  gemm_f64            the block formulas accumulated in fp64 (llm_kernel_test/reference/
                      gemm_ref.py:100-153 and :274-330)
  dequantize          block -> fp32 values (gemm_ref.py:51-97, :156-199)

Nothing here computes an output for a caller: results come from libksq only, and these
functions are the checker the runner compares them with.
"""
from __future__ import annotations

import numpy as np

# weight type -> (block bytes, offset of d, offset of m or None, offset of qh or None,
#                 offset of qs, quant kind)  for the 32-element block types
LAYOUT = {
    0: (18, 0, None, None, 2, "nib"),    # Q4_0: value (q - 8) d
    1: (34, 0, None, None, 2, "i8"),     # Q8_0: value q d
    4: (20, 0, 2, None, 4, "nib"),       # Q4_1: value q d + m
    5: (22, 0, None, 2, 6, "nib5"),      # Q5_0: value (q - 16) d
    6: (24, 0, 2, 4, 8, "nib5"),         # Q5_1: value q d + m
}


def _f16(b: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(b).view(np.float16)[..., 0].astype(np.float64)


def quantize_q8_1(x: np.ndarray) -> np.ndarray:
    """fp32 [M, K] -> block_q8_1 bytes [M, K/32, 36]."""
    x = np.asarray(x, dtype=np.float32)
    M, K = x.shape
    xb = x.reshape(M, K // 32, 32)
    amax = np.abs(xb).max(axis=-1)
    ssum = np.cumsum(xb, axis=-1, dtype=np.float32)[..., -1]      # left-to-right fp32 sum
    d = (amax / np.float32(127.0)).astype(np.float32)
    safe = np.where(d > 0, d, np.float32(1.0))
    idv = np.where(d > 0, np.float32(1.0) / safe, np.float32(0.0)).astype(np.float32)
    v = (xb * idv[..., None]).astype(np.float32).astype(np.float64)
    q = np.clip(np.sign(v) * np.floor(np.abs(v) + 0.5), -128, 127).astype(np.int8)   # half away from zero
    out = np.empty((M, K // 32, 36), dtype=np.uint8)
    with np.errstate(over="ignore"):
        out[..., 0:2] = d.astype(np.float16)[..., None].view(np.uint8)
        out[..., 2:4] = ssum.astype(np.float16)[..., None].view(np.uint8)
    out[..., 4:] = q.view(np.uint8)
    return out


def unpack(wtype: int, w: np.ndarray):
    """[N, nb, bytes] -> (d, m or None, q) with q the stored quants (int64, unsigned for the
    nibble types, signed for Q8_0)."""
    nbytes, do, mo, ho, qo, kind = LAYOUT[wtype]
    d = _f16(w[..., do:do + 2])
    m = _f16(w[..., mo:mo + 2]) if mo is not None else None
    if kind == "i8":
        q = w[..., qo:qo + 32].view(np.int8).astype(np.int64)
    else:
        qs = w[..., qo:qo + 16].astype(np.int64)
        q = np.concatenate([qs & 0x0F, qs >> 4], axis=-1)
        if kind == "nib5":
            q = q + 16 * np.unpackbits(np.ascontiguousarray(w[..., ho:ho + 4]), axis=-1,
                                       bitorder="little").astype(np.int64)
    return d, m, q


def dequantize(wtype: int, w: np.ndarray) -> np.ndarray:
    """[N, nb, bytes] -> fp64 values [N, nb*32]."""
    d, m, q = unpack(wtype, w)
    if wtype == 0:
        v = d[..., None] * (q - 8)
    elif wtype == 5:
        v = d[..., None] * (q - 16)
    elif wtype == 1:
        v = d[..., None] * q
    else:
        v = d[..., None] * q + m[..., None]
    return v.reshape(w.shape[0], -1)


def block_sumi(wtype: int, a: np.ndarray, w: np.ndarray) -> np.ndarray:
    """Integer block dots [M, N, nb] of block_q8_1 activations [M, nb, 36] with weights [N, nb, bytes]."""
    _, _, qw = unpack(wtype, w)
    qa = a[..., 4:36].view(np.int8).astype(np.int64)
    return np.einsum("mbk,nbk->mnb", qa, qw)


def gemm_f64(wtype: int, a: np.ndarray, w: np.ndarray) -> np.ndarray:
    """Block formula in fp64: Q4_0 d_w(d_a S - 8 s_a), Q8_0 d_w d_a S, Q5_0 d_w(d_a S - 16 s_a),
    Q4_1 / Q5_1 d_w d_a S + m_w s_a."""
    dw, mw, _ = unpack(wtype, w)
    da, sa = _f16(a[..., 0:2]), _f16(a[..., 2:4])
    S = block_sumi(wtype, a, w).astype(np.float64)
    if wtype == 0:
        return np.einsum("nb,mnb->mn", dw, da[:, None, :] * S - 8.0 * sa[:, None, :])
    if wtype == 5:
        return np.einsum("nb,mnb->mn", dw, da[:, None, :] * S - 16.0 * sa[:, None, :])
    if wtype == 1:
        return np.einsum("nb,mb,mnb->mn", dw, da, S)
    return np.einsum("nb,mb,mnb->mn", dw, da, S) + np.einsum("nb,mb->mn", mw, sa)


def max_rel_err(y: np.ndarray, ref: np.ndarray) -> float:
    """Max of |y - ref| / max(|ref|, 1e-3 * max |ref| of the row)."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    floor = 1e-3 * np.abs(ref).max(axis=-1, keepdims=True) + 1e-30
    return float((np.abs(y - ref) / np.maximum(np.abs(ref), floor)).max())


def quantize_q8s(x: np.ndarray) -> np.ndarray:
    """fp32 [M, K] -> block_q8s bytes [M, K/32, 36], the native W8A8C8 operator's rules
    (core/operators/quant_gemm/variants/deepseek_v3/w8a8c8_q8_0_q8_1/kernel.cu:66-93):
    d = amax/127 in fp32 (1 below 1e-6), q = clamp(roundf(x / d)) by true division."""
    x = np.asarray(x, dtype=np.float32)
    M, K = x.shape
    xb = x.reshape(M, K // 32, 32)
    d = (np.abs(xb).max(axis=-1) / np.float32(127.0)).astype(np.float32)
    d = np.where(d < np.float32(1e-6), np.float32(1.0), d).astype(np.float32)
    v = (xb / d[..., None]).astype(np.float32).astype(np.float64)
    q = np.clip(np.sign(v) * np.floor(np.abs(v) + 0.5), -128, 127).astype(np.int8)
    out = np.empty((M, K // 32, 36), dtype=np.uint8)
    out[..., 0:4] = d[..., None].view(np.uint8)
    out[..., 4:] = q.view(np.uint8)
    return out


def quantize_q8f(x: np.ndarray, rule: int = 0) -> np.ndarray:
    """fp32 [M, K] -> block_q8f bytes [M, K/32, 40] (fp32 d, fp32 s, 32 int8).
    rule 0, the deepseek_v2 W4A32C8 operator (core/operators/quant_gemm/variants/deepseek_v2/
    w4a32c8_q4_0_fp32_int8/reference.py:50-73): d = amax / 127 in fp32 (1.0 when amax is 0),
    s = the left-to-right fp32 sum, q = round half to even of the fp32 quotient x / d, clamped.
    rule 1, the lm_head kernel (best_kernels_GLM-5/quant_gemm/..._lm_head_n128256_k4096/
    kernel.cu:85-107): d = amax / 127 (1.0 when amax <= 1e-10), q = lroundf(x * (127 / amax)),
    half away from zero, wrapped to int8."""
    x = np.asarray(x, dtype=np.float32)
    M, K = x.shape
    xb = x.reshape(M, K // 32, 32)
    amax = np.abs(xb).max(axis=-1)
    ssum = np.cumsum(xb, axis=-1, dtype=np.float32)[..., -1]
    if rule == 0:
        d = np.where(amax > 0, amax / np.float32(127.0), np.float32(1.0)).astype(np.float32)
        v = (xb / d[..., None]).astype(np.float32)
        q = np.clip(np.rint(v), -128, 127).astype(np.int8)
    else:
        d = np.where(amax > np.float32(1e-10), amax / np.float32(127.0), np.float32(1.0)).astype(np.float32)
        sc = (np.float32(127.0) / np.maximum(amax, np.float32(1e-10))).astype(np.float32)
        v = (xb * sc[..., None]).astype(np.float32).astype(np.float64)
        q = (np.sign(v) * np.floor(np.abs(v) + 0.5)).astype(np.int64).astype(np.uint8).view(np.int8)
    out = np.empty((M, K // 32, 40), dtype=np.uint8)
    out[..., 0:4] = d[..., None].view(np.uint8)
    out[..., 4:8] = ssum.astype(np.float32)[..., None].view(np.uint8)
    out[..., 8:] = q.view(np.uint8)
    return out


def gemm_q8s_f64(a: np.ndarray, w: np.ndarray) -> np.ndarray:
    """Q8_0 weights x block_q8s activations: sum_b d_w d_a S in fp64."""
    dw, _, _ = unpack(1, w)
    da = np.ascontiguousarray(a[..., 0:4]).view(np.float32)[..., 0].astype(np.float64)
    S = block_sumi(1, a, w).astype(np.float64)
    return np.einsum("nb,mb,mnb->mn", dw, da, S)


# ---- unit-scale exactness -------------------------------------------------------------------
# With every weight scale 1 (d = 1; Q4_K dmin = 1 with integer 6-bit mins; Q4_1 / Q5_1 integer
# offsets m) and every activation block at d_a = 1 (fp32 input: integer values whose block
# maximum is exactly 127, so d = 127 / 127 = 1 and q = x; pre-quantised input: d = 1 stored), each
# block contributes an integer to the output.  If the sum of the absolute values of all those
# contributions stays below 2^24, every partial sum of them, in any order, is an exact fp32
# integer: the fp32 output of a correct engine then equals the exact integer result bit for bit,
# and a single wrong integer block dot (or a wrong scale, nibble, sub-block or offset) changes it.

K_QUANT_BYTES = {2: 144, 3: 210}


def _kq_fields(wtype: int, w: np.ndarray):
    """K-quant super-blocks [N, nsb, bytes] -> (element multiplier [N, K], quants [N, K] int64,
    side factor per 32-element block [N, K/32]) of the public GGML layouts: Q4_K value
    d*sc_j*q - dmin*m_j (get_scale_min_k4 packing of the 12 scale bytes; the low / high nibbles of
    qs[32g .. 32g+31] are sub-blocks 2g / 2g+1); Q6_K value d*sc[k/16]*(q - 32) with
    q = ql nibble | 2 qh bits (dequantize_row_q6_K order)."""
    N, nsb, _ = w.shape
    if wtype == 2:
        d = _f16(w[..., 0:2])
        dmin = _f16(w[..., 2:4])
        s = w[..., 4:16].astype(np.int64)
        sc = np.empty((N, nsb, 8), np.int64)
        mn = np.empty((N, nsb, 8), np.int64)
        sc[..., :4] = s[..., 0:4] & 63
        mn[..., :4] = s[..., 4:8] & 63
        sc[..., 4:] = (s[..., 8:12] & 0x0F) | ((s[..., 0:4] >> 6) << 4)
        mn[..., 4:] = (s[..., 8:12] >> 4) | ((s[..., 4:8] >> 6) << 4)
        qs = w[..., 16:144].astype(np.int64).reshape(N, nsb, 4, 32)
        q = np.stack([qs & 0x0F, qs >> 4], axis=3).reshape(N, nsb * 256)      # [g][lo/hi][32]
        mult = np.repeat((d[..., None] * sc).reshape(N, nsb * 8), 32, axis=1)
        side = -(dmin[..., None] * mn).reshape(N, nsb * 8)
        return mult, q, side
    ql = w[..., 0:128].astype(np.int64).reshape(N, nsb, 2, 64)
    qh = w[..., 128:192].astype(np.int64).reshape(N, nsb, 2, 32)
    sc = w[..., 192:208].view(np.int8).astype(np.int64)
    d = _f16(w[..., 208:210])
    q = np.empty((N, nsb, 2, 4, 32), np.int64)
    q[..., 0, :] = (ql[..., 0:32] & 0x0F) | ((qh & 3) << 4)
    q[..., 1, :] = (ql[..., 32:64] & 0x0F) | (((qh >> 2) & 3) << 4)
    q[..., 2, :] = (ql[..., 0:32] >> 4) | (((qh >> 4) & 3) << 4)
    q[..., 3, :] = (ql[..., 32:64] >> 4) | (((qh >> 6) & 3) << 4)
    mult = np.repeat((d[..., None] * sc).reshape(N, nsb * 16), 16, axis=1)
    return mult, q.reshape(N, nsb * 256) - 32, np.zeros((N, nsb * 8))


def weight_terms(wtype: int, w: np.ndarray):
    """Weights [N, blocks, bytes] -> (Weff [N, K] fp64, coef [N, K/32] fp64) with
    output = sum_k A[k] * Weff[k] + sum_b s_a[b] * coef[b] for A[k] = d_a * q_a (the block
    formulas of gemm_reference.h:175-267 and the harness oracles gemm_ref.py:100-153, :274-330,
    regrouped: Q4_0 coef -8 d_w, Q5_0 -16 d_w, Q4_1 / Q5_1 m_w, Q4_K -dmin m_j, Q8_0 / Q6_K 0)."""
    if wtype in K_QUANT_BYTES:
        mult, q, side = _kq_fields(wtype, w)
        return mult * q, side
    d, m, q = unpack(wtype, w)
    N = w.shape[0]
    weff = (d[..., None] * q).reshape(N, -1)
    if wtype == 0:
        coef = -8.0 * d
    elif wtype == 5:
        coef = -16.0 * d
    elif wtype == 1:
        coef = np.zeros_like(d)
    else:
        coef = m
    return weff, coef


def act_terms(a: np.ndarray, q8s: bool = False):
    """block_q8_1 (or block_q8s) activations [M, K/32, 36], or block_q8f [M, K/32, 40] (fp32 d and s),
    -> (A [M, K] = d_a * q_a, s_a [M, K/32])."""
    M, nb, nbytes = a.shape
    if nbytes == 40:
        f = np.ascontiguousarray(a[..., 0:8]).view(np.float32).astype(np.float64)
        q = np.ascontiguousarray(a[..., 8:40]).view(np.int8).astype(np.int64)
        return (f[..., 0:1] * q).reshape(M, -1), f[..., 1]
    d = (np.ascontiguousarray(a[..., 0:4]).view(np.float32)[..., 0].astype(np.float64) if q8s
         else _f16(a[..., 0:2]))
    s = np.zeros((M, nb)) if q8s else _f16(a[..., 2:4])
    q = a[..., 4:36].view(np.int8).astype(np.int64)
    return (d[..., None] * q).reshape(M, -1), s


def exact_gemm(wtype: int, a: np.ndarray, w: np.ndarray, q8s: bool = False):
    """(y, bound): y[m, n] = the block formulas summed in fp64 as one product, and bound[m, n] =
    the same sums over absolute values.  For integer-valued inputs (unit scales) with
    bound < 2^24, y is the exact integer every correct fp32 engine must produce."""
    A, s = act_terms(a, q8s)
    weff, coef = weight_terms(wtype, w)
    y = A @ weff.T + s @ coef.T
    bound = np.abs(A) @ np.abs(weff).T + np.abs(s) @ np.abs(coef).T
    return y, bound


def _f16_bytes(v: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(v, np.float64).astype(np.float16)).view(np.uint8).reshape(*np.shape(v), 2)


def unit_weights(wtype: int, g: np.random.Generator, N: int, K: int, q6k_scale: int = 32) -> np.ndarray:
    """Random quants with every scale 1: d = 1 (and dmin = 1 for Q4_K with its 6-bit scales and
    mins drawn over the full 0..63, high bits included; Q4_1 / Q5_1 offsets m integers in
    [-8, 8]; Q6_K int8 scales in [-q6k_scale, q6k_scale - 1])."""
    if wtype in K_QUANT_BYTES:
        nsb, nbytes = K // 256, K_QUANT_BYTES[wtype]
        w = g.integers(0, 256, size=(N, nsb, nbytes), dtype=np.uint8)
        if wtype == 2:
            w[..., 0:2] = _f16_bytes(np.ones((N, nsb)))
            w[..., 2:4] = _f16_bytes(np.ones((N, nsb)))
        else:
            w[..., 192:208] = g.integers(-q6k_scale, q6k_scale, size=(N, nsb, 16)).astype(np.int8).view(np.uint8)
            w[..., 208:210] = _f16_bytes(np.ones((N, nsb)))
        return w
    nbytes, do, mo, _, _, _ = LAYOUT[wtype]
    nb = K // 32
    w = g.integers(0, 256, size=(N, nb, nbytes), dtype=np.uint8)
    w[..., do:do + 2] = _f16_bytes(np.ones((N, nb)))
    if mo is not None:
        w[..., mo:mo + 2] = _f16_bytes(g.integers(-8, 9, size=(N, nb)))
    return w


def _block_rows(M: int, nb: int, onehot) -> np.ndarray:
    """mask [M, nb]: all blocks of dense rows (onehot[m] < 0), block onehot[m] only otherwise."""
    mask = np.ones((M, nb), dtype=bool)
    if onehot is not None:
        oh = np.asarray(onehot)
        rows = oh >= 0
        mask[rows] = False
        mask[np.nonzero(rows)[0], oh[rows]] = True
    return mask


def unit_activations(g: np.random.Generator, M: int, K: int, qmax: int = 127, onehot=None) -> np.ndarray:
    """fp32 [M, K] integers: every non-zero block holds values in [-qmax, qmax] plus one element of
    +-127 at a random position (so its Q8_1 / block_q8s d is exactly 1 and q = x), and its sum
    within [-2048, 2048] (exact in fp16).  Blocks outside the mask of `onehot` are zero."""
    nb = K // 32

    def draw(n):
        v = g.integers(-qmax, qmax + 1, size=(n, 32)).astype(np.float64)
        pos = g.integers(0, 32, size=n)
        v[np.arange(n), pos] = np.where(g.integers(0, 2, size=n) == 1, 127.0, -127.0)
        return v

    x = draw(M * nb).reshape(M, nb, 32)
    while True:
        bad = np.abs(x.sum(axis=-1)) > 2048
        if not bad.any():
            break
        x[bad] = draw(int(bad.sum()))
    x *= _block_rows(M, nb, onehot)[..., None]
    return x.reshape(M, K).astype(np.float32)


def unit_q8_1(g: np.random.Generator, M: int, K: int, qmax: int = 127, onehot=None, smax: int = 2048) -> np.ndarray:
    """block_q8_1 [M, K/32, 36] with d = 1, quants uniform in [-qmax, qmax] (qmax 128 includes -128)
    and an independent integer s in [-smax, smax]; blocks outside the mask are all zero."""
    nb = K // 32
    a = np.zeros((M, nb, 36), dtype=np.uint8)
    lo = -128 if qmax >= 128 else -qmax
    q = g.integers(lo, min(qmax, 127) + 1, size=(M, nb, 32)).astype(np.int8)
    a[..., 0:2] = _f16_bytes(np.ones((M, nb)))
    a[..., 2:4] = _f16_bytes(g.integers(-smax, smax + 1, size=(M, nb)))
    a[..., 4:] = q.view(np.uint8)
    a *= _block_rows(M, nb, onehot)[..., None].astype(np.uint8)
    return a


def unit_q8s(g: np.random.Generator, M: int, K: int, qmax: int = 127, onehot=None) -> np.ndarray:
    """block_q8s [M, K/32, 36] with the fp32 d = 1 and quants in [-qmax, qmax]; masked blocks zero."""
    nb = K // 32
    a = np.zeros((M, nb, 36), dtype=np.uint8)
    a[..., 0:4] = np.ones((M, nb, 1), np.float32).view(np.uint8)
    a[..., 4:] = g.integers(-qmax, qmax + 1, size=(M, nb, 32)).astype(np.int8).view(np.uint8)
    a *= _block_rows(M, nb, onehot)[..., None].astype(np.uint8)
    return a


# mean |stored quant x scale| of unit weights per type, for sizing the activations below
_MEAN_ABS_W = {0: 7.5, 1: 64.0, 2: 236.0, 3: 256.0, 4: 9.5, 5: 15.5, 6: 17.5}


def unit_qmax(wtype: int, K: int, budget: float = 2.0 ** 23) -> int:
    """The activation quant range for unit_activations that keeps the expected magnitude sum of a
    row near `budget` (half of 2^24) at this K, counting the forced +-127 element per block."""
    wabs = _MEAN_ABS_W[wtype]
    forced = 127.0 * wabs * (K / 32)
    q = int(2.0 * (budget - forced) / (K * wabs)) if budget > forced else 1
    return max(1, min(127, q))


def onehot_pattern(M: int, nb: int, every: int = 2, seed: int = 0) -> np.ndarray:
    """Row m is dense when m % every == 0, else one-hot at a block that walks all nb positions."""
    oh = np.full(M, -1, dtype=np.int64)
    rows = np.arange(M)
    sel = rows % every != 0
    oh[sel] = (rows[sel] * 7 + seed) % nb
    return oh
