"""ksq - MI355X-native quantized GGML matmul (host side of libksq.so).

The compute path is the HIP library libksq.so (k-search_amd/csrc); this
package loads it through its C ABI and offers the reference harness's
forward(weight, activation, M, N, K) convention on torch tensors.
"""
from ._lib import (A_F32, A_F32_Q8F_LROUND, A_F32_Q8F_RNE, A_F32_Q8S, A_Q8_1, A_Q8F, A_Q8S,  # noqa: F401
                   Q8F_LROUND, Q8F_RNE, W_Q4_0, W_Q4_1, W_Q4_K, W_Q5_0, W_Q5_1, W_Q6_K, W_Q8_0, WQ_DEVICE, WQ_REF,
                   KsqError, lib)
from .formats import QUANT_TYPES, WTYPE_NAMES, quant_type  # noqa: F401
from .ops import (ENTRY_POINTS, block_sumi, forward, gemm, gemm_w16, moe_gemm, moe_gemm_routed,  # noqa: F401
                  moe_workspace_size, quantize_q8_1, quantize_q8f, quantize_q8s, release, set_path,
                  workspace_size)
