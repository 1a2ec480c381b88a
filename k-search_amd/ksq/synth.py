"""Seeded synthetic inputs for the benchmark configurations (numpy, PCG64).

Distributions follow BASELINE.json's configs:
  Q4_0 weights  uniform nibbles 0..15, d = fp16(|N(0, 0.02)|)
  Q8_0 weights  qs uniform in [-127, 127], d = fp16(|N(0, 0.01)|)
  Q4_K weights  uniform nibbles, 6-bit scales and mins uniform in [0, 63],
                d, dmin = fp16(|N(0, 0.02)|)          (ranges chosen here; BASELINE leaves them open)
  Q6_K weights  uniform 6-bit quants, int8 scales uniform in [-128, 127], d = fp16(|N(0, 0.002)|)
  Q4_1 weights  uniform nibbles, d = fp16(|N(0, 0.02)|), m = fp16(-d * U(6, 9))
  Q5_0 weights  uniform 5-bit quants, d = fp16(|N(0, 0.01)|)
  Q5_1 weights  uniform 5-bit quants, d = fp16(|N(0, 0.01)|), m = fp16(-d * U(13, 18))
                (Q4_1 / Q5_x ranges chosen here: no BASELINE config uses them)
  activations   fp32 N(0, 1)
  router logits fp32 N(0, 1)
All generators return flat-per-row uint8 byte arrays in the reference layouts.
"""
from __future__ import annotations

import numpy as np


def rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def _f16_bytes(vals: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(vals.astype(np.float16)).view(np.uint8).reshape(*vals.shape, 2)


def q4_0_weights(g: np.random.Generator, N: int, K: int) -> np.ndarray:
    nb = K // 32
    out = np.empty((N, nb, 18), dtype=np.uint8)
    out[:, :, 0:2] = _f16_bytes(np.abs(g.standard_normal((N, nb), dtype=np.float32) * np.float32(0.02)))
    out[:, :, 2:] = g.integers(0, 256, size=(N, nb, 16), dtype=np.uint8)
    return out


def q8_0_weights(g: np.random.Generator, N: int, K: int) -> np.ndarray:
    nb = K // 32
    out = np.empty((N, nb, 34), dtype=np.uint8)
    out[:, :, 0:2] = _f16_bytes(np.abs(g.standard_normal((N, nb), dtype=np.float32) * np.float32(0.01)))
    out[:, :, 2:] = g.integers(-127, 128, size=(N, nb, 32), dtype=np.int16).astype(np.int8).view(np.uint8)
    return out


def q4_K_weights(g: np.random.Generator, N: int, K: int) -> np.ndarray:
    nsb = K // 256
    out = np.empty((N, nsb, 144), dtype=np.uint8)
    out[:, :, 0:2] = _f16_bytes(np.abs(g.standard_normal((N, nsb), dtype=np.float32) * np.float32(0.02)))
    out[:, :, 2:4] = _f16_bytes(np.abs(g.standard_normal((N, nsb), dtype=np.float32) * np.float32(0.02)))
    out[:, :, 4:] = g.integers(0, 256, size=(N, nsb, 140), dtype=np.uint8)  # 6-bit fields uniform
    return out


def q6_K_weights(g: np.random.Generator, N: int, K: int) -> np.ndarray:
    nsb = K // 256
    out = np.empty((N, nsb, 210), dtype=np.uint8)
    out[:, :, 0:208] = g.integers(0, 256, size=(N, nsb, 208), dtype=np.uint8)  # ql, qh, int8 scales
    out[:, :, 208:210] = _f16_bytes(np.abs(g.standard_normal((N, nsb), dtype=np.float32) * np.float32(0.002)))
    return out


def _legacy(g: np.random.Generator, N: int, K: int, nbytes: int, d_sigma: float, m_span, qh_off, qs_off):
    nb = K // 32
    out = np.empty((N, nb, nbytes), dtype=np.uint8)
    d = np.abs(g.standard_normal((N, nb), dtype=np.float32) * np.float32(d_sigma))
    out[:, :, 0:2] = _f16_bytes(d)
    if m_span is not None:   # offset near the block minimum of a centred block: m = -d * U(lo, hi)
        out[:, :, 2:4] = _f16_bytes(-d * g.uniform(*m_span, size=(N, nb)).astype(np.float32))
    if qh_off is not None:
        out[:, :, qh_off:qh_off + 4] = g.integers(0, 256, size=(N, nb, 4), dtype=np.uint8)
    out[:, :, qs_off:qs_off + 16] = g.integers(0, 256, size=(N, nb, 16), dtype=np.uint8)
    return out


def q4_1_weights(g: np.random.Generator, N: int, K: int) -> np.ndarray:
    return _legacy(g, N, K, 20, 0.02, (6.0, 9.0), None, 4)


def q5_0_weights(g: np.random.Generator, N: int, K: int) -> np.ndarray:
    return _legacy(g, N, K, 22, 0.01, None, 2, 6)


def q5_1_weights(g: np.random.Generator, N: int, K: int) -> np.ndarray:
    return _legacy(g, N, K, 24, 0.01, (13.0, 18.0), 4, 8)


WEIGHT_GENERATORS = {0: q4_0_weights, 1: q8_0_weights, 2: q4_K_weights, 3: q6_K_weights,
                     4: q4_1_weights, 5: q5_0_weights, 6: q5_1_weights}


def weights(wtype: int, g: np.random.Generator, N: int, K: int) -> np.ndarray:
    return WEIGHT_GENERATORS[wtype](g, N, K)


def activations(g: np.random.Generator, M: int, K: int) -> np.ndarray:
    return g.standard_normal((M, K), dtype=np.float32)


def router_logits(g: np.random.Generator, T: int, E: int) -> np.ndarray:
    return g.standard_normal((T, E), dtype=np.float32)
