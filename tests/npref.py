"""Independent numpy formulations used to pin the C oracle.

These are written from the block layouts and the mathematics, with different
primitives from oracle/ksq_oracle.c (numpy float16 instead of the hand-written
converter, float64 floor for round-half-away, cumsum for the sequential sum,
vectorised unpacking, and *encoders* for the K-quant layouts where the oracle
has decoders), so that a dropped term, a wrong sign or index or a transposed
operand in either shows up as a mismatch.
"""
from __future__ import annotations

import numpy as np


def f16(b: np.ndarray) -> np.ndarray:
    """little-endian fp16 byte pairs [..., 2] -> float64."""
    return np.ascontiguousarray(b).view(np.float16)[..., 0].astype(np.float64)


def quantize_q8_1(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    M, K = x.shape
    xb = x.reshape(M, K // 32, 32)
    amax = np.abs(xb).max(axis=-1)
    ssum = np.cumsum(xb, axis=-1, dtype=np.float32)[..., -1]           # sequential fp32 sum
    d = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(d > 0, np.float32(1.0) / np.where(d > 0, d, np.float32(1)), np.float32(0)).astype(np.float32)
    v = (xb * idv[..., None]).astype(np.float32).astype(np.float64)
    q = np.sign(v) * np.floor(np.abs(v) + 0.5)                          # half away from zero, exact in f64
    q = np.clip(q, -128, 127).astype(np.int8)
    out = np.empty((M, K // 32, 36), dtype=np.uint8)
    out[..., 0:2] = d.astype(np.float16)[..., None].view(np.uint8)
    out[..., 2:4] = ssum.astype(np.float16)[..., None].view(np.uint8)
    out[..., 4:] = q.view(np.uint8)
    return out


def unpack_q4_0(w: np.ndarray):
    """[N, nb, 18] -> (d [N, nb] f64, q [N, nb, 32] int64 in 0..15, element order of the reference)."""
    d = f16(w[..., 0:2])
    qs = w[..., 2:18].astype(np.int64)
    q = np.concatenate([qs & 0x0F, qs >> 4], axis=-1)
    return d, q


def unpack_q8_0(w: np.ndarray):
    d = f16(w[..., 0:2])
    q = w[..., 2:34].view(np.int8).astype(np.int64)
    return d, q


def unpack_q8_1(a: np.ndarray):
    d = f16(a[..., 0:2])
    s = f16(a[..., 2:4])
    q = a[..., 4:36].view(np.int8).astype(np.int64)
    return d, s, q


def sumi(wtype: int, a: np.ndarray, w: np.ndarray) -> np.ndarray:
    """Brute-force integer block dots [M, N, nb] for Q4_0 (0) / Q8_0 (1)."""
    _, qw = unpack_q4_0(w) if wtype == 0 else unpack_q8_0(w)
    _, _, qa = unpack_q8_1(a)
    return np.einsum("mbk,nbk->mnb", qa, qw)


def gemm_f64(wtype: int, a: np.ndarray, w: np.ndarray) -> np.ndarray:
    """Block formula in fp64: Q4_0 sum_b dw*(da*sumi - 8*sa), Q8_0 sum_b sumi*da*dw."""
    dw, _ = unpack_q4_0(w) if wtype == 0 else unpack_q8_0(w)
    da, sa, _ = unpack_q8_1(a)
    S = sumi(wtype, a, w).astype(np.float64)
    if wtype == 0:
        return np.einsum("nb,mnb->mn", dw, da[:, None, :] * S - 8.0 * sa[:, None, :])
    return np.einsum("nb,mb,mnb->mn", dw, da, S)


# ---- K-quant encoders (bytes from chosen fields, written from the public GGML layout) ----

def encode_q4_K(d, dmin, sc, mn, q) -> np.ndarray:
    """d, dmin: floats; sc, mn: 8 ints in [0, 63]; q: 256 ints in [0, 15] -> 144 bytes."""
    b = np.zeros(144, dtype=np.uint8)
    b[0:2] = np.array([d], dtype=np.float16).view(np.uint8)
    b[2:4] = np.array([dmin], dtype=np.float16).view(np.uint8)
    s = np.zeros(12, dtype=np.int64)
    for j in range(4):
        s[j] = sc[j] | ((sc[j + 4] >> 4) << 6)        # low 6 bits: scale j; top 2: high bits of scale j+4
        s[j + 4] = mn[j] | ((mn[j + 4] >> 4) << 6)    # low 6 bits: min j;   top 2: high bits of min j+4
        s[j + 8] = (sc[j + 4] & 0x0F) | ((mn[j + 4] & 0x0F) << 4)
    b[4:16] = s.astype(np.uint8)
    q = np.asarray(q, dtype=np.int64).reshape(4, 2, 32)  # 64-element groups, two 32-element halves
    b[16:] = (q[:, 0, :] | (q[:, 1, :] << 4)).reshape(128).astype(np.uint8)
    return b


def encode_q6_K(d, sc, q) -> np.ndarray:
    """d: float; sc: 16 ints in [-128, 127]; q: 256 ints in [0, 63] (stored value, dequant uses q-32)."""
    b = np.zeros(210, dtype=np.uint8)
    q = np.asarray(q, dtype=np.int64).reshape(2, 4, 32)   # half, quarter, lane
    ql = np.zeros((2, 64), dtype=np.int64)
    qh = np.zeros((2, 32), dtype=np.int64)
    for n in range(2):
        ql[n, 0:32] = (q[n, 0] & 0x0F) | ((q[n, 2] & 0x0F) << 4)
        ql[n, 32:64] = (q[n, 1] & 0x0F) | ((q[n, 3] & 0x0F) << 4)
        qh[n] = (q[n, 0] >> 4) | ((q[n, 1] >> 4) << 2) | ((q[n, 2] >> 4) << 4) | ((q[n, 3] >> 4) << 6)
    b[0:128] = ql.reshape(128).astype(np.uint8)
    b[128:192] = qh.reshape(64).astype(np.uint8)
    b[192:208] = np.asarray(sc, dtype=np.int8).view(np.uint8)
    b[208:210] = np.array([d], dtype=np.float16).view(np.uint8)
    return b


# ---- Q4_1 / Q5_0 / Q5_1 (layouts of core/operators/common/types.py:94-140) ----

LEGACY_LAYOUT = {  # wtype: (bytes, offset of m or None, offset of qh or None, offset of qs)
    4: (20, 2, None, 4),
    5: (22, None, 2, 6),
    6: (24, 2, 4, 8),
}


def unpack_legacy(wtype: int, w: np.ndarray):
    """[N, nb, bytes] -> (d f64, m f64 or None, q int64 [N, nb, 32] unsigned quants).
    qh bits via numpy.unpackbits (little bit order), nibbles by shifts."""
    nbytes, mo, ho, qo = LEGACY_LAYOUT[wtype]
    d = f16(w[..., 0:2])
    m = f16(w[..., mo:mo + 2]) if mo is not None else None
    qs = w[..., qo:qo + 16].astype(np.int64)
    q = np.concatenate([qs & 0x0F, qs >> 4], axis=-1)
    if ho is not None:
        bits = np.unpackbits(np.ascontiguousarray(w[..., ho:ho + 4]), axis=-1, bitorder="little").astype(np.int64)
        q = q + 16 * bits
    return d, m, q


def encode_legacy(wtype: int, d: float, m, q) -> np.ndarray:
    """One block from chosen fields (q: 32 unsigned quants)."""
    nbytes, mo, ho, qo = LEGACY_LAYOUT[wtype]
    q = np.asarray(q, dtype=np.int64)
    b = np.zeros(nbytes, dtype=np.uint8)
    b[0:2] = np.array([d], dtype=np.float16).view(np.uint8)
    if mo is not None:
        b[mo:mo + 2] = np.array([m], dtype=np.float16).view(np.uint8)
    b[qo:qo + 16] = ((q[:16] & 0x0F) | ((q[16:] & 0x0F) << 4)).astype(np.uint8)
    if ho is not None:
        h = int(sum(((int(q[e]) >> 4) & 1) << e for e in range(32)))
        b[ho:ho + 4] = np.array([h], dtype="<u4").view(np.uint8)
    return b


def gemm_legacy_f64(wtype: int, a: np.ndarray, w: np.ndarray) -> np.ndarray:
    """Harness formula in fp64 (gemm_ref.py:274-330 for Q4_1; the same with the 5-bit
    quants for Q5_1; d_w*(d_a*sumi - 16*s_a) for Q5_0)."""
    dw, mw, qw = unpack_legacy(wtype, w)
    da, sa, qa = unpack_q8_1(a)
    S = np.einsum("mbk,nbk->mnb", qa, qw).astype(np.float64)
    if wtype == 5:
        return np.einsum("nb,mnb->mn", dw, da[:, None, :] * S - 16.0 * sa[:, None, :])
    return np.einsum("nb,mb,mnb->mn", dw, da, S) + np.einsum("nb,mb->mn", mw, sa)


def quantize_q4_1(x: np.ndarray) -> np.ndarray:
    """quantize_to_q4_1 (llm_kernel_test/reference/quantize.py:105-153) vectorised."""
    x = np.asarray(x, dtype=np.float32)
    N, K = x.shape
    xb = x.reshape(N, K // 32, 32)
    lo, hi = xb.min(axis=-1), xb.max(axis=-1)
    scale = np.where(hi > lo, (hi - lo) / np.float32(15.0), np.float32(1.0)).astype(np.float32)
    q = np.clip(np.round((xb - lo[..., None]) / scale[..., None]), 0, 15).astype(np.int64)
    out = np.zeros((N, K // 32, 20), dtype=np.uint8)
    out[..., 0:2] = scale.astype(np.float16)[..., None].view(np.uint8)
    out[..., 2:4] = lo.astype(np.float16)[..., None].view(np.uint8)
    out[..., 4:] = (q[..., :16] | (q[..., 16:] << 4)).astype(np.uint8)
    return out


def quantize_q8s(x: np.ndarray) -> np.ndarray:
    """Native W8A8C8 activation quantiser (variants/deepseek_v3/w8a8c8_q8_0_q8_1/kernel.cu:66-93):
    d = max|x| / 127 in fp32 (1 when below 1e-6), q = half-away(x / d) by true fp32 division."""
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


def quantize_q8_1_numpy_harness(x: np.ndarray) -> np.ndarray:
    """The test harness' quantize_to_q8_1 as NumPy runs it (np.max, np.where, true division,
    np.round half-even, np.sum's pairwise float32 order, np.float16 packing), for finite x."""
    M, K = x.shape
    a = x.reshape(M, K // 32, 32).astype(np.float32)
    mx = np.max(np.abs(a), axis=2)
    d = np.where(mx > 0, mx / np.float32(127.0), np.float32(1.0)).astype(np.float32)
    q = np.round(a / d[:, :, None]).clip(-128, 127).astype(np.int8)
    s = np.sum(a, axis=2)
    out = np.zeros((M, K // 32, 36), dtype=np.uint8)
    out[:, :, 0:2] = d.astype(np.float16).view(np.uint8).reshape(M, K // 32, 2)
    with np.errstate(over="ignore"):
        out[:, :, 2:4] = s.astype(np.float16).view(np.uint8).reshape(M, K // 32, 2)
    out[:, :, 4:] = q.view(np.uint8)
    return out


def quantize_q8_1_device_rint(x: np.ndarray) -> np.ndarray:
    """The reference's device quantiser (fmaxf max, sequential sum by cumsum, id = 1/d,
    np.rint half-even, clamp), for finite x."""
    M, K = x.shape
    a = x.reshape(M, K // 32, 32).astype(np.float32)
    amax = np.max(np.abs(a), axis=2)
    s = np.cumsum(a, axis=2, dtype=np.float32)[:, :, -1]
    d = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(d > 0, np.float32(1.0) / d, np.float32(0.0)).astype(np.float32)
    q = np.rint(a * idv[:, :, None]).clip(-128, 127).astype(np.int8)
    out = np.zeros((M, K // 32, 36), dtype=np.uint8)
    out[:, :, 0:2] = d.astype(np.float16).view(np.uint8).reshape(M, K // 32, 2)
    with np.errstate(over="ignore"):
        out[:, :, 2:4] = s.astype(np.float16).view(np.uint8).reshape(M, K // 32, 2)
    out[:, :, 4:] = q.view(np.uint8)
    return out
