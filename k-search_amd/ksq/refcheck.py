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


def gemm_q8s_f64(a: np.ndarray, w: np.ndarray) -> np.ndarray:
    """Q8_0 weights x block_q8s activations: sum_b d_w d_a S in fp64."""
    dw, _, _ = unpack(1, w)
    da = np.ascontiguousarray(a[..., 0:4]).view(np.float32)[..., 0].astype(np.float64)
    S = block_sumi(1, a, w).astype(np.float64)
    return np.einsum("nb,mb,mnb->mn", dw, da, S)
