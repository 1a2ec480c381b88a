"""ctypes front end of the CPU oracle (oracle/ksq_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker.  The product library
never imports this module.

All buffers are numpy arrays; quantised tensors are flat uint8 byte arrays in
the reference layouts (block_q4_0 18 B, block_q8_0 34 B, block_q8_1 36 B,
block_q4_1 20 B, block_q5_0 22 B, block_q5_1 24 B, block_q4_K 144 B, block_q6_K
210 B), the native W8A8C8 operator's activation block (block_q8s 36 B) or the
fp32-scale activation block of the deepseek_v2 operator and the lm_head kernel
(block_q8f 40 B: fp32 d, fp32 s, 32 int8).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libksq_oracle.so")

W_Q4_0, W_Q8_0, W_Q4_K, W_Q6_K, W_Q4_1, W_Q5_0, W_Q5_1 = 0, 1, 2, 3, 4, 5, 6
WBYTES = {W_Q4_0: 18, W_Q8_0: 34, W_Q4_K: 144, W_Q6_K: 210, W_Q4_1: 20, W_Q5_0: 22, W_Q5_1: 24}
WELEMS = {W_Q4_0: 32, W_Q8_0: 32, W_Q4_K: 256, W_Q6_K: 256, W_Q4_1: 32, W_Q5_0: 32, W_Q5_1: 32}
LEGACY = (W_Q4_1, W_Q5_0, W_Q5_1)
NAMES = {W_Q4_0: "q4_0", W_Q8_0: "q8_0", W_Q4_K: "q4_K", W_Q6_K: "q6_K", W_Q4_1: "q4_1", W_Q5_0: "q5_0",
         W_Q5_1: "q5_1"}

_lib = None


def build() -> None:
    """Compile the oracle with its Makefile (gcc)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.c_void_p
        i32, i64 = ctypes.c_int, ctypes.c_int64
        L.ksq_ref_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.ksq_ref_f16_to_f32.restype = ctypes.c_float
        L.ksq_ref_f32_to_f16.argtypes = [ctypes.c_float]
        L.ksq_ref_f32_to_f16.restype = ctypes.c_uint16
        for name in ("quantize_row_q8_1", "quantize_row_q8_0", "quantize_row_q4_0",
                     "quantize_row_q4_1", "quantize_row_q5_0", "quantize_row_q5_1", "quantize_row_q8s",
                     "dequantize_row_q4_0", "dequantize_row_q8_0", "dequantize_row_q8_1",
                     "dequantize_row_q4_K", "dequantize_row_q6_K", "quantize_q4_0_device", "quantize_q8_0_device"):
            f = getattr(L, "ksq_ref_" + name)
            f.argtypes = [P, P, i64]
            f.restype = None
        for name in ("sumi_q4_0_q8_1", "sumi_q8_0_q8_1"):
            f = getattr(L, "ksq_ref_" + name)
            f.argtypes = [P, P]
            f.restype = ctypes.c_int32
        L.ksq_ref_quantize_row_q8_1_variant.argtypes = [i32, P, P, i64]
        L.ksq_ref_quantize_row_q8_1_variant.restype = None
        L.ksq_ref_dequantize_row_legacy.argtypes = [i32, P, P, i64]
        L.ksq_ref_sumi_legacy_q8_1.argtypes = [i32, P, P]
        L.ksq_ref_sumi_legacy_q8_1.restype = ctypes.c_int32
        L.ksq_ref_gemm_legacy.argtypes = [i32, P, P, P, i32, i32, i32, i32]
        L.ksq_ref_gemm_w8a8c8.argtypes = [P, P, P, i32, i32, i32, i32]
        L.ksq_ref_gemm_q8_0_q8s_f64.argtypes = [P, P, P, i32, i32, i32, i32]
        L.ksq_ref_quantize_row_q8f.argtypes = [i32, P, P, i64]
        L.ksq_ref_gemm_w4a16.argtypes = [P, P, P, i32, i32, i32, i32]
        L.ksq_ref_gemm_w8a16.argtypes = [P, P, P, i32, i32, i32, i32]
        L.ksq_ref_gemm_q8f.argtypes = [i32, P, P, P, i32, i32, i32, i32]
        L.ksq_ref_gemm_q8f_f64.argtypes = [i32, P, P, P, i32, i32, i32, i32]
        L.ksq_ref_q4_K_scale_min.argtypes = [i32, P, P, P]
        L.ksq_ref_sumi_q4_K_q8_1.argtypes = [P, i32, P]
        L.ksq_ref_sumi_q4_K_q8_1.restype = ctypes.c_int32
        L.ksq_ref_sumi_q6_K_q8_1.argtypes = [P, i32, P]
        L.ksq_ref_sumi_q6_K_q8_1.restype = ctypes.c_int32
        for name in ("gemm_w4a8", "gemm_w8a8"):
            getattr(L, "ksq_ref_" + name).argtypes = [P, P, P, i32, i32, i32, i32]
        L.ksq_ref_gemm_f64.argtypes = [i32, P, P, P, i32, i32, i32, i32]
        L.ksq_ref_gemm_kquant.argtypes = [i32, P, P, P, i32, i32, i32, i32]
        L.ksq_ref_gemm_kquant_f64.argtypes = [i32, P, P, P, i32, i32, i32, i32]
        L.ksq_ref_block_sumi.argtypes = [i32, P, P, P, i32, i32, i32]
        L.ksq_ref_moe_route.argtypes = [P, i32, i32, i32, i32, P, P]
        L.ksq_ref_moe_q4_0_f64.argtypes = [P, P, P, P, P, i32, i32, i32, i32, i32]
        L.ksq_ref_max_threads.restype = i32
        _lib = L
    return _lib


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def max_threads() -> int:
    return lib().ksq_ref_max_threads()


def f32_to_f16_bits(x: float) -> int:
    return lib().ksq_ref_f32_to_f16(x)


def f16_bits_to_f32(h: int) -> float:
    return lib().ksq_ref_f16_to_f32(h)


def quantize_q8_1(x: np.ndarray) -> np.ndarray:
    """fp32 [M, K] -> block_q8_1 bytes [M, K/32, 36] (quantize_row_q8_1_ref per row)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    M, K = x.shape
    y = np.empty((M, K // 32, 36), dtype=np.uint8)
    lib().ksq_ref_quantize_row_q8_1(_p(x), _p(y), M * K)
    return y


def quantize_q8_1_variant(x: np.ndarray, variant: int) -> np.ndarray:
    """[M, K] -> block_q8_1 bytes [M, K/32, 36] by one of the reference's Q8_1 quantisers:
    0 quantize_row_q8_1_ref, 1 its device kernel (half-even), 2 the NumPy harness'
    quantize_to_q8_1, 3 the fused FP16-activation kernels' quantiser (x fp16)."""
    if variant == 3:
        x = np.ascontiguousarray(x, dtype=np.float16)
    else:
        x = np.ascontiguousarray(x, dtype=np.float32)
    M, K = x.shape
    y = np.empty((M, K // 32, 36), dtype=np.uint8)
    lib().ksq_ref_quantize_row_q8_1_variant(variant, _p(x), _p(y), M * K)
    return y


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    M, K = x.shape
    y = np.empty((M, K // 32, 34), dtype=np.uint8)
    lib().ksq_ref_quantize_row_q8_0(_p(x), _p(y), M * K)
    return y


def quantize_q4_0(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    M, K = x.shape
    y = np.empty((M, K // 32, 18), dtype=np.uint8)
    lib().ksq_ref_quantize_row_q4_0(_p(x), _p(y), M * K)
    return y


def quantize_weights(wtype: int, x: np.ndarray, rule: int = 0) -> np.ndarray:
    """fp32 [N, K] -> block_q4_0 (wtype 0) / block_q8_0 (wtype 1) bytes [N, K/32, 18 | 34]: rule 0
    the reference's device kernels (include/quantize.h:221-297), rule 1 its CPU references
    (quantize_row_q4_0_ref / quantize_row_q8_0_ref)."""
    if rule == 1:
        return quantize_q4_0(x) if wtype == 0 else quantize_q8_0(x)
    name = {0: "quantize_q4_0_device", 1: "quantize_q8_0_device"}[wtype]
    return _quantize_raw(name, x, 18 if wtype == 0 else 34)


def _quantize_raw(name: str, x: np.ndarray, bytes_per_block: int) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    M, K = x.shape
    y = np.empty((M, K // 32, bytes_per_block), dtype=np.uint8)
    getattr(lib(), "ksq_ref_" + name)(_p(x), _p(y), M * K)
    return y


def _quantize(name: str, x: np.ndarray, bytes_per_block: int) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    M, K = x.shape
    y = np.empty((M, K // 32, bytes_per_block), dtype=np.uint8)
    getattr(lib(), "ksq_ref_quantize_row_" + name)(_p(x), _p(y), M * K)
    return y


def quantize_q4_1(x: np.ndarray) -> np.ndarray:
    """fp32 [N, K] -> block_q4_1 bytes (quantize_to_q4_1 arithmetic)."""
    return _quantize("q4_1", x, 20)


def quantize_q5_0(x: np.ndarray) -> np.ndarray:
    return _quantize("q5_0", x, 22)


def quantize_q5_1(x: np.ndarray) -> np.ndarray:
    return _quantize("q5_1", x, 24)


def quantize_q8s(x: np.ndarray) -> np.ndarray:
    """fp32 [M, K] -> block_q8s bytes [M, K/32, 36] (the native W8A8C8 operator's rules)."""
    return _quantize("q8s", x, 36)


def dequantize(wtype_or_name, q: np.ndarray, rows: int, K: int) -> np.ndarray:
    by_name = {v: k for k, v in NAMES.items()}
    wt = by_name.get(wtype_or_name, wtype_or_name)
    q = np.ascontiguousarray(q, dtype=np.uint8)
    y = np.empty((rows, K), dtype=np.float32)
    if wt in LEGACY:
        lib().ksq_ref_dequantize_row_legacy(wt, _p(q), _p(y), rows * K)
    else:
        getattr(lib(), "ksq_ref_dequantize_row_" + NAMES.get(wt, wt))(_p(q), _p(y), rows * K)
    return y


def sumi_legacy(wtype: int, wblk: np.ndarray, ablk: np.ndarray) -> int:
    w = np.ascontiguousarray(wblk, dtype=np.uint8)
    a = np.ascontiguousarray(ablk, dtype=np.uint8)
    return lib().ksq_ref_sumi_legacy_q8_1(wtype, _p(w), _p(a))


def gemm_w8a8c8(x: np.ndarray, w: np.ndarray, M: int, N: int, K: int, nthreads: int = 1) -> np.ndarray:
    """The native W8A8C8 operator on fp32 activations (fp32 accumulation order)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    C = np.empty((M, N), dtype=np.float32)
    lib().ksq_ref_gemm_w8a8c8(_p(x), _p(w), _p(C), M, N, K, nthreads)
    return C


def gemm_q8s_f64(a_q8s: np.ndarray, w: np.ndarray, M: int, N: int, K: int, nthreads: int = 0) -> np.ndarray:
    """Q8_0 weights x block_q8s activations, fp64 accumulation (tolerance reference)."""
    a = np.ascontiguousarray(a_q8s, dtype=np.uint8)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    C = np.empty((M, N), dtype=np.float64)
    lib().ksq_ref_gemm_q8_0_q8s_f64(_p(a), _p(w), _p(C), M, N, K, nthreads or max_threads())
    return C


Q8F_RNE, Q8F_LROUND = 0, 1


def gemm_w16(wtype: int, x: np.ndarray, w: np.ndarray, M: int, N: int, K: int, nthreads: int = 0) -> np.ndarray:
    """gemm_w4a16_reference (wtype 0, Q4_0) / gemm_w8a16_reference (wtype 1, Q8_0): fp32 activations
    times dequantised weights, the reference's fp32 summation order."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    C = np.empty((M, N), dtype=np.float32)
    fn = lib().ksq_ref_gemm_w4a16 if wtype == W_Q4_0 else lib().ksq_ref_gemm_w8a16
    fn(_p(x), _p(w), _p(C), M, N, K, nthreads or max_threads())
    return C


def quantize_q8f(x: np.ndarray, rule: int) -> np.ndarray:
    """fp32 [M, K] -> block_q8f bytes [M, K/32, 40]: rule 0 the deepseek_v2 operator's
    quantiser (round half to even of x / d), 1 the lm_head kernel's (lroundf(x * 127/amax))."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    M, K = x.shape
    y = np.empty((M, K // 32, 40), dtype=np.uint8)
    lib().ksq_ref_quantize_row_q8f(rule, _p(x), _p(y), M * K)
    return y


def gemm_q8f(wtype: int, a_q8f: np.ndarray, w: np.ndarray, M: int, N: int, K: int, nthreads: int = 0,
             f64: bool = False) -> np.ndarray:
    """Q4_0 / Q5_0 / Q8_0 weights x block_q8f activations: the deepseek_v2 operator's fp32 block
    order (or fp64 accumulation of the same block terms with f64=True)."""
    a = np.ascontiguousarray(a_q8f, dtype=np.uint8)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    C = np.empty((M, N), dtype=np.float64 if f64 else np.float32)
    fn = lib().ksq_ref_gemm_q8f_f64 if f64 else lib().ksq_ref_gemm_q8f
    fn(wtype, _p(a), _p(w), _p(C), M, N, K, nthreads or max_threads())
    return C


def gemm(wtype: int, a_q8_1: np.ndarray, w: np.ndarray, M: int, N: int, K: int, nthreads: int = 1) -> np.ndarray:
    """Reference fp32 accumulation order: C[M, N]."""
    a = np.ascontiguousarray(a_q8_1, dtype=np.uint8)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    C = np.empty((M, N), dtype=np.float32)
    if wtype == W_Q4_0:
        lib().ksq_ref_gemm_w4a8(_p(a), _p(w), _p(C), M, N, K, nthreads)
    elif wtype == W_Q8_0:
        lib().ksq_ref_gemm_w8a8(_p(a), _p(w), _p(C), M, N, K, nthreads)
    elif wtype in LEGACY:
        lib().ksq_ref_gemm_legacy(wtype, _p(a), _p(w), _p(C), M, N, K, nthreads)
    else:
        lib().ksq_ref_gemm_kquant(wtype, _p(a), _p(w), _p(C), M, N, K, nthreads)
    return C


def gemm_f64(wtype: int, a_q8_1: np.ndarray, w: np.ndarray, M: int, N: int, K: int, nthreads: int = 0) -> np.ndarray:
    """The same block formulas accumulated in fp64 (tolerance reference)."""
    a = np.ascontiguousarray(a_q8_1, dtype=np.uint8)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    C = np.empty((M, N), dtype=np.float64)
    nthreads = nthreads or max_threads()
    if wtype in (W_Q4_0, W_Q8_0) + LEGACY:
        lib().ksq_ref_gemm_f64(wtype, _p(a), _p(w), _p(C), M, N, K, nthreads)
    else:
        lib().ksq_ref_gemm_kquant_f64(wtype, _p(a), _p(w), _p(C), M, N, K, nthreads)
    return C


def block_sumi(wtype: int, a_q8_1: np.ndarray, w: np.ndarray, M: int, N: int, K: int) -> np.ndarray:
    """Integer block dots [M, N, nblk] (nblk = K/16 for Q6_K, else K/32)."""
    a = np.ascontiguousarray(a_q8_1, dtype=np.uint8)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    nblk = K // 16 if wtype == W_Q6_K else K // 32
    out = np.empty((M, N, nblk), dtype=np.int32)
    lib().ksq_ref_block_sumi(wtype, _p(a), _p(w), _p(out), M, N, K)
    return out


def q4_K_scale_min(j: int, scales12: np.ndarray) -> tuple[int, int]:
    s = np.ascontiguousarray(scales12, dtype=np.uint8)
    sc, m = ctypes.c_int(), ctypes.c_int()
    lib().ksq_ref_q4_K_scale_min(j, _p(s), ctypes.byref(sc), ctypes.byref(m))
    return sc.value, m.value


def moe_route(logits: np.ndarray, top_k: int, renorm: bool = False) -> tuple[np.ndarray, np.ndarray]:
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    T, E = logits.shape
    ids = np.empty((T, top_k), dtype=np.int32)
    w = np.empty((T, top_k), dtype=np.float32)
    lib().ksq_ref_moe_route(_p(logits), T, E, top_k, int(renorm), _p(ids), _p(w))
    return ids, w


def moe_q4_0_f64(w_experts: np.ndarray, a_q8_1: np.ndarray, ids: np.ndarray, wts: np.ndarray,
                 T: int, N: int, K: int, nthreads: int = 0) -> np.ndarray:
    W = np.ascontiguousarray(w_experts, dtype=np.uint8)
    A = np.ascontiguousarray(a_q8_1, dtype=np.uint8)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    wts = np.ascontiguousarray(wts, dtype=np.float32)
    out = np.empty((T, N), dtype=np.float64)
    top_k = ids.shape[1]
    lib().ksq_ref_moe_q4_0_f64(_p(W), _p(A), _p(ids), _p(wts), _p(out), T, N, K, top_k, nthreads or max_threads())
    return out
