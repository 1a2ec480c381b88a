"""Loader for libksq.so, the HIP/gfx950 library behind the C ABI in include/ksq.h.

There is no CPU fallback: if the library is missing or fails to load, every
entry raises.  Build it with ``make -C k-search_amd`` (or
``__graft_entry__.build()``).
"""
from __future__ import annotations

import ctypes
import os
import threading

PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG_ROOT, "libksq.so")

# enum ksq_wtype / ksq_atype / ksq_status (include/ksq_blocks.h, include/ksq.h)
W_Q4_0, W_Q8_0, W_Q4_K, W_Q6_K, W_Q4_1, W_Q5_0, W_Q5_1 = 0, 1, 2, 3, 4, 5, 6
A_F32, A_Q8_1, A_F32_Q8S, A_Q8S, A_F16 = 0, 1, 2, 3, 4
A_Q8F, A_F32_Q8F_RNE, A_F32_Q8F_LROUND = 5, 6, 7
Q8F_RNE, Q8F_LROUND = 0, 1   # KSQ_Q8F_* rules of ksq_quantize_q8f
WQ_DEVICE, WQ_REF = 0, 1      # KSQ_WQ_* rules of ksq_quantize_weights
NOALLOC_SCRATCH_BYTES = 32 << 20   # KSQ_NOALLOC_SCRATCH_BYTES
# KSQ_ENG_* bits of ksq_debug_last_engines (include/ksq.h)
ENG = {"quantize": 1 << 0, "gemv_row": 1 << 1, "gemv_row_fq": 1 << 2, "gemv_direct": 1 << 3,
       "gemv_direct_fq": 1 << 4, "gemv_mr": 1 << 5, "gemv_mr_fq": 1 << 6, "gemv_kq": 1 << 7, "skinny": 1 << 8,
       **{f"mmq{c}": 1 << (8 + c) for c in range(1, 8)}, "splitk": 1 << 16, "moe_route": 1 << 17,
       "moe_group": 1 << 18, "moe_tile64": 1 << 19, "moe_tile128": 1 << 20, "moe_combine": 1 << 21,
       "transpose": 1 << 22, "w16": 1 << 23, "mmq_planar": 1 << 24, "moe_planar": 1 << 25}
STATUS = {0: "KSQ_OK", 1: "KSQ_ERR_NULL", 2: "KSQ_ERR_SHAPE", 3: "KSQ_ERR_ALIGN",
          4: "KSQ_ERR_TYPE", 5: "KSQ_ERR_WORKSPACE", 6: "KSQ_ERR_HIP"}

# Every symbol include/ksq.h declares, with its ctypes signature.
_P, _I, _SZ = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
SIGNATURES = {
    "ksq_last_error": ([], _I),
    "ksq_last_error_message": ([], ctypes.c_char_p),
    "ksq_error_string": ([_I], ctypes.c_char_p),
    "ksq_version": ([], ctypes.c_char_p),
    "ksq_release": ([], None),
    "gemm_w4a32c8_q4_0_fp32_int8": ([_P, _P, _P, _I, _I, _I], None),
    "gemm_w8a32c8_q8_0_fp32_int8": ([_P, _P, _P, _I, _I, _I], None),
    "gemm_w4a32c8_q4_k_fp32_int8": ([_P, _P, _P, _I, _I, _I], None),
    "gemm_w6a32c8_q6_k_fp32_int8": ([_P, _P, _P, _I, _I, _I], None),
    "ksq_gemm_q4_0_q8_1": ([_P, _P, _P, _I, _I, _I], None),
    "ksq_gemm_q8_0_q8_1": ([_P, _P, _P, _I, _I, _I], None),
    "ksq_gemm_q4_k_q8_1": ([_P, _P, _P, _I, _I, _I], None),
    "ksq_gemm_q6_k_q8_1": ([_P, _P, _P, _I, _I, _I], None),
    "gemm_w4a32c8_q4_1_fp32_int8": ([_P, _P, _P, _I, _I, _I], None),
    "gemm_w5a32c8_q5_0_fp32_int8": ([_P, _P, _P, _I, _I, _I], None),
    "gemm_w5a32c8_q5_1_fp32_int8": ([_P, _P, _P, _I, _I, _I], None),
    "ksq_gemm_q4_1_q8_1": ([_P, _P, _P, _I, _I, _I], None),
    "ksq_gemm_q5_0_q8_1": ([_P, _P, _P, _I, _I, _I], None),
    "ksq_gemm_q5_1_q8_1": ([_P, _P, _P, _I, _I, _I], None),
    "gemm_w8a8c8_q8_0_q8_1": ([_P, _P, _P, _I, _I, _I], None),
    "gemm_w4a32c8_q4_0_fp32_int8_deepseek_v2": ([_P, _P, _P, _I, _I, _I], None),
    "ksq_quantize_q8f": ([_I, _P, _P, _I, _I, _P], _I),
    "ksq_gemm_w16_workspace_size": ([_I, _I, _I], _SZ),
    "ksq_gemm_w16": ([_I, _P, _P, _P, _I, _I, _I, _P, _SZ, _P], _I),
    "ksq_gemm_w4a16": ([_P, _P, _P, _I, _I, _I, _P], _I),
    "ksq_gemm_w8a16": ([_P, _P, _P, _I, _I, _I, _P], _I),
    "ksq_quantize_q8_1": ([_P, _P, _I, _I, _P], _I),
    "ksq_quantize_q8s": ([_P, _P, _I, _I, _P], _I),
    "ksq_quantize_q8_1_variant": ([_I, _P, _P, _I, _I, _P], _I),
    "ksq_quantize_weights": ([_I, _I, _P, _P, ctypes.c_int64, _P], _I),
    "ksq_gemm_q4_0_fp16_fused_workspace_size": ([_I, _I, _I], _SZ),
    "ksq_gemm_q4_0_fp16_fused": ([_P, _P, _P, _I, _I, _I, _P, _SZ, _P], _I),
    "ksq_gemm_workspace_size": ([_I, _I, _I, _I, _I], _SZ),
    "ksq_gemm": ([_I, _I, _P, _P, _P, _I, _I, _I, _P, _SZ, _P], _I),
    "ksq_gemm_noalloc": ([_I, _I, _P, _P, _P, _I, _I, _I, _P], _I),
    "ksq_debug_planar_bytes": ([_I, _I], _SZ),
    "ksq_debug_quantize_planar": ([_I, _P, _P, _I, _I, _P], _I),
    "ksq_debug_gemm_planar": ([_I, _P, _P, _P, _I, _I, _I, _P], _I),
    "ksq_debug_stream_read_outputs": ([_SZ], _SZ),
    "ksq_debug_stream_read": ([_P, _SZ, _P, _P], _I),
    "ksq_debug_stream_read_wg_outputs": ([_SZ, _SZ], _SZ),
    "ksq_debug_stream_read_wg": ([_P, _SZ, _SZ, _P, _P], _I),
    "ksq_debug_block_sumi": ([_I, _P, _P, _P, _I, _I, _I, _P], _I),
    "ksq_debug_block_sumi_mfma": ([_I, _P, _P, _P, _I, _I, _I, _P], _I),
    "ksq_set_path": ([_I], _I),
    "ksq_set_mmq_config": ([_I], _I),
    "ksq_debug_last_engines": ([], ctypes.c_uint32),
    "ksq_moe_workspace_size": ([_I, _I, _I, _I, _I, _I], _SZ),
    "ksq_moe_gemm": ([_I, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P, _P, _P, _SZ, _P], _I),
    "ksq_moe_gemm_routed": ([_I, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _SZ, _P], _I),
    "moe_w4a32c8_q4_0_fp32_int8": ([_P, _P, _P, _P, _I, _I, _I, _I, _I], None),
}


class KsqError(RuntimeError):
    """A libksq call returned a non-zero ksq_status."""

    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS.get(status, status)}: {message}")
        self.status = status


_lib = None
_lock = threading.Lock()


def lib() -> ctypes.CDLL:
    """Load libksq.so once; raise if it is absent (no fallback path exists)."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise ImportError(f"libksq.so not built ({LIB_PATH}); run `make -C k-search_amd`")
                L = ctypes.CDLL(LIB_PATH)
                for name, (args, res) in SIGNATURES.items():
                    fn = getattr(L, name)
                    fn.argtypes = args
                    fn.restype = res
                _lib = L
    return _lib


def check(status: int) -> None:
    if status != 0:
        msg = lib().ksq_last_error_message().decode()
        raise KsqError(status, msg)
