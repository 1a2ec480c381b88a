"""Torch-tensor front end of libksq (PyTorch is only the device-memory / stream plumbing).

`forward` mirrors the wrapper the reference harness generates around a
quant_gemm entry point (kernelevalplus-main/llm_kernel_test/op_test_handler.py:298-349):
same arguments (weight, activation, M, N, K), same CUDA-tensor checks and
messages, output allocated as an fp32 [M, N] tensor on the weight's device.
Calls go through the C ABI on torch's current stream.
"""
from __future__ import annotations

import torch

from . import _lib
from ._lib import (A_F32, A_F32_Q8F_RNE, A_F32_Q8S, A_Q8_1, Q8F_LROUND, Q8F_RNE, W_Q4_0, W_Q4_1, W_Q4_K,
                   W_Q5_0, W_Q5_1, W_Q6_K, W_Q8_0, check, lib)

# Definition-style entry points of include/ksq.h -> (weight type, activation type)
ENTRY_POINTS = {
    "gemm_w4a32c8_q4_0_fp32_int8": (W_Q4_0, A_F32),
    "gemm_w8a32c8_q8_0_fp32_int8": (W_Q8_0, A_F32),
    "gemm_w4a32c8_q4_k_fp32_int8": (W_Q4_K, A_F32),
    "gemm_w6a32c8_q6_k_fp32_int8": (W_Q6_K, A_F32),
    "ksq_gemm_q4_0_q8_1": (W_Q4_0, A_Q8_1),
    "ksq_gemm_q8_0_q8_1": (W_Q8_0, A_Q8_1),
    "ksq_gemm_q4_k_q8_1": (W_Q4_K, A_Q8_1),
    "ksq_gemm_q6_k_q8_1": (W_Q6_K, A_Q8_1),
    "gemm_w4a32c8_q4_1_fp32_int8": (W_Q4_1, A_F32),
    "gemm_w5a32c8_q5_0_fp32_int8": (W_Q5_0, A_F32),
    "gemm_w5a32c8_q5_1_fp32_int8": (W_Q5_1, A_F32),
    "ksq_gemm_q4_1_q8_1": (W_Q4_1, A_Q8_1),
    "ksq_gemm_q5_0_q8_1": (W_Q5_0, A_Q8_1),
    "ksq_gemm_q5_1_q8_1": (W_Q5_1, A_Q8_1),
    # the native deepseek_v3 W8A8C8 operator (spec.json entry point "gemm_w8a8c8_q8_0_q8_1")
    "gemm_w8a8c8_q8_0_q8_1": (W_Q8_0, A_F32_Q8S),
    # the deepseek_v2 W4A32C8 operator (spec.json entry point "forward"): fp32 d_a and s_a
    "gemm_w4a32c8_q4_0_fp32_int8_deepseek_v2": (W_Q4_0, A_F32_Q8F_RNE),
}


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def gemm(wtype: int, atype: int, weight: torch.Tensor, activation: torch.Tensor, M: int, N: int, K: int,
         out: torch.Tensor | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """output[M, N] = activation[M, K] . weight[N, K]^T through ksq_gemm."""
    if out is None:
        out = torch.empty((M, N), dtype=torch.float32, device=weight.device)
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    check(lib().ksq_gemm(wtype, atype, _ptr(weight), _ptr(activation), _ptr(out), M, N, K,
                         _ptr(workspace), ws_bytes, _stream()))
    return out


def gemm_w16(wtype: int, activation: torch.Tensor, weight: torch.Tensor, M: int, N: int, K: int,
             out: torch.Tensor | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """The dequantise-then-fp32 GEMM (W4A16 / W8A16): output[M, N] = activation[M, K] (fp32) .
    dequant(weight)[N, K]^T for Q4_0 / Q8_0 weights, through ksq_gemm_w16."""
    if activation.dtype != torch.float32 or not activation.is_cuda or not weight.is_cuda:
        raise RuntimeError("gemm_w16 expects a CUDA float32 activation and CUDA uint8 weights")
    if out is None:
        out = torch.empty((M, N), dtype=torch.float32, device=weight.device)
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    check(lib().ksq_gemm_w16(wtype, _ptr(activation.contiguous()), _ptr(weight), _ptr(out), M, N, K,
                             _ptr(workspace), ws_bytes, _stream()))
    return out


def gemm_w16_workspace_size(M: int, N: int, K: int) -> int:
    return lib().ksq_gemm_w16_workspace_size(M, N, K)


def gemm_q4_0_fp16_fused(weight: torch.Tensor, activation: torch.Tensor, M: int, N: int, K: int,
                         out: torch.Tensor | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """The reference's gemm_q4_0_fp16_fused orientation: Q4_0 weight [M, K/32] (M weight rows),
    fp16 activation [N, K], output fp32 [M, N]."""
    if activation.dtype != torch.float16 or not activation.is_cuda or not weight.is_cuda:
        raise RuntimeError("gemm_q4_0_fp16_fused expects CUDA uint8 weights and float16 activations")
    if out is None:
        out = torch.empty((M, N), dtype=torch.float32, device=weight.device)
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    check(lib().ksq_gemm_q4_0_fp16_fused(_ptr(weight), _ptr(activation.contiguous()), _ptr(out), M, N, K,
                                         _ptr(workspace), ws_bytes, _stream()))
    return out


def gemm_q4_0_fp16_fused_workspace_size(M: int, N: int, K: int) -> int:
    return lib().ksq_gemm_q4_0_fp16_fused_workspace_size(M, N, K)


def forward(weight: torch.Tensor, activation: torch.Tensor, M: int, N: int, K: int,
            entry: str = "gemm_w4a32c8_q4_0_fp32_int8") -> torch.Tensor:
    """The harness wrapper: forward(weight, activation, M, N, K) -> fp32 [M, N]."""
    if not weight.is_cuda:
        raise RuntimeError("Weight must be CUDA tensor")
    if not activation.is_cuda:
        raise RuntimeError("Activation must be CUDA tensor")
    wtype, atype = ENTRY_POINTS[entry]
    if weight.dtype != torch.uint8:
        raise RuntimeError(f"expected scalar type Byte for weight but found {weight.dtype}")
    want = torch.float32 if atype in (A_F32, A_F32_Q8S, A_F32_Q8F_RNE) else torch.uint8
    if activation.dtype != want:
        raise RuntimeError(f"expected scalar type {want} for activation but found {activation.dtype}")
    return gemm(wtype, atype, weight, activation, int(M), int(N), int(K))


def quantize_q8_1(x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """fp32 [..., K] -> uint8 [..., K/32, 36] (quantize_row_q8_1_ref bit for bit)."""
    if x.dtype != torch.float32 or not x.is_cuda:
        raise RuntimeError("quantize_q8_1 expects a CUDA float32 tensor")
    x = x.contiguous()
    K = x.shape[-1]
    rows = x.numel() // K if K else 0
    if out is None:
        out = torch.empty((*x.shape[:-1], K // 32, 36), dtype=torch.uint8, device=x.device)
    check(lib().ksq_quantize_q8_1(_ptr(x), _ptr(out), rows, K, _stream()))
    return out


Q81_REF, Q81_CUDA, Q81_NUMPY, Q81_FUSED_F16 = 0, 1, 2, 3


def quantize_q8_1_variant(x: torch.Tensor, variant: int, out: torch.Tensor | None = None) -> torch.Tensor:
    """[..., K] -> uint8 [..., K/32, 36] block_q8_1 by one of the reference's quantisers:
    Q81_REF quantize_row_q8_1_ref, Q81_CUDA its device kernel (half-even), Q81_NUMPY the
    harness' quantize_to_q8_1, Q81_FUSED_F16 the fused FP16 kernels' quantiser (x float16)."""
    want = torch.float16 if variant == Q81_FUSED_F16 else torch.float32
    if x.dtype != want or not x.is_cuda:
        raise RuntimeError(f"quantize_q8_1_variant({variant}) expects a CUDA {want} tensor")
    x = x.contiguous()
    K = x.shape[-1]
    rows = x.numel() // K if K else 0
    if out is None:
        out = torch.empty((*x.shape[:-1], K // 32, 36), dtype=torch.uint8, device=x.device)
    check(lib().ksq_quantize_q8_1_variant(variant, _ptr(x), _ptr(out), rows, K, _stream()))
    return out


def quantize_weights(wtype: int, x: torch.Tensor, rule: int = 0, out: torch.Tensor | None = None) -> torch.Tensor:
    """fp32 [..., K] -> uint8 [..., K/32, 18 | 34] block_q4_0 (wtype W_Q4_0) / block_q8_0 (W_Q8_0) on
    the device: rule WQ_DEVICE the reference's quantize_q4_0_kernel / quantize_q8_0_kernel
    (half-to-even), WQ_REF its CPU references quantize_row_q4_0_ref / quantize_row_q8_0_ref."""
    if x.dtype != torch.float32 or not x.is_cuda:
        raise RuntimeError("quantize_weights expects a CUDA float32 tensor")
    x = x.contiguous()
    K = x.shape[-1]
    bpb = 18 if wtype == 0 else 34
    if out is None:
        out = torch.empty((*x.shape[:-1], K // 32, bpb), dtype=torch.uint8, device=x.device)
    check(lib().ksq_quantize_weights(wtype, rule, _ptr(x), _ptr(out), x.numel(), _stream()))
    return out


def quantize_q8s(x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """fp32 [..., K] -> uint8 [..., K/32, 36] block_q8s (the native W8A8C8 operator's rules)."""
    if x.dtype != torch.float32 or not x.is_cuda:
        raise RuntimeError("quantize_q8s expects a CUDA float32 tensor")
    x = x.contiguous()
    K = x.shape[-1]
    rows = x.numel() // K if K else 0
    if out is None:
        out = torch.empty((*x.shape[:-1], K // 32, 36), dtype=torch.uint8, device=x.device)
    check(lib().ksq_quantize_q8s(_ptr(x), _ptr(out), rows, K, _stream()))
    return out


def quantize_q8f(x: torch.Tensor, rule: int = Q8F_RNE, out: torch.Tensor | None = None) -> torch.Tensor:
    """fp32 [..., K] -> uint8 [..., K/32, 40] block_q8f (fp32 d and s): rule Q8F_RNE the deepseek_v2
    operator's quantiser, Q8F_LROUND the lm_head kernel's."""
    if x.dtype != torch.float32 or not x.is_cuda:
        raise RuntimeError("quantize_q8f expects a CUDA float32 tensor")
    x = x.contiguous()
    K = x.shape[-1]
    rows = x.numel() // K if K else 0
    if out is None:
        out = torch.empty((*x.shape[:-1], K // 32, 40), dtype=torch.uint8, device=x.device)
    check(lib().ksq_quantize_q8f(rule, _ptr(x), _ptr(out), rows, K, _stream()))
    return out


def block_sumi(wtype: int, weight: torch.Tensor, act_q8_1: torch.Tensor, M: int, N: int, K: int,
               mfma: bool = False) -> torch.Tensor:
    """Per-block integer dots [M, N, nblk] from the device block-dot code (debug): the v_dot4
    decode helpers, or the int8 MFMA GEMM's tiles (mfma=True)."""
    nblk = K // 16 if wtype == W_Q6_K else K // 32
    out = torch.empty((M, N, nblk), dtype=torch.int32, device=weight.device)
    fn = lib().ksq_debug_block_sumi_mfma if mfma else lib().ksq_debug_block_sumi
    check(fn(wtype, _ptr(weight), _ptr(act_q8_1), _ptr(out), M, N, K, _stream()))
    return out


def quantize_planar(wtype: int, x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """The planar block_q8_1 activations the LDS-DMA GEMM reads (debug / measurement): a uint8
    buffer of ksq_debug_planar_bytes(M, K) bytes holding the int8 quant plane [M][K], the
    (d, -12582912 d) fp32 pairs [K/32][Mp] and the -s fp16 bits [K/128][Mp][4], each plane
    256-byte aligned (Mp = M rounded up to 128)."""
    if not (x.is_cuda and x.dtype == torch.float32):
        raise RuntimeError("quantize_planar expects a CUDA float32 tensor")
    x = x.contiguous()
    M, K = x.shape
    if out is None:
        out = torch.empty(max(1, lib().ksq_debug_planar_bytes(M, K)), dtype=torch.uint8, device=x.device)
    check(lib().ksq_debug_quantize_planar(wtype, _ptr(x), _ptr(out), M, K, _stream()))
    return out


def gemm_planar(wtype: int, weight: torch.Tensor, planar: torch.Tensor, M: int, N: int, K: int,
                out: torch.Tensor | None = None) -> torch.Tensor:
    """The LDS-DMA GEMM alone on quantize_planar's output (debug / measurement)."""
    if out is None:
        out = torch.empty((M, N), dtype=torch.float32, device=weight.device)
    check(lib().ksq_debug_gemm_planar(wtype, _ptr(weight), _ptr(planar), _ptr(out), M, N, K, _stream()))
    return out


def stream_read(buf: torch.Tensor, out: torch.Tensor | None = None, wg_bytes: int | None = None) -> torch.Tensor:
    """Calibration read of every byte of buf (ksq_debug_stream_read, or ksq_debug_stream_read_wg
    with wg_bytes per workgroup); returns the XOR words, one per workgroup."""
    nbytes = buf.numel() * buf.element_size()
    if wg_bytes is None:
        if out is None:
            out = torch.empty(max(1, lib().ksq_debug_stream_read_outputs(nbytes)), dtype=torch.int32,
                              device=buf.device)
        check(lib().ksq_debug_stream_read(_ptr(buf), nbytes, _ptr(out), _stream()))
        return out
    if out is None:
        out = torch.empty(max(1, lib().ksq_debug_stream_read_wg_outputs(nbytes, wg_bytes)), dtype=torch.int32,
                          device=buf.device)
    check(lib().ksq_debug_stream_read_wg(_ptr(buf), nbytes, wg_bytes, _ptr(out), _stream()))
    return out


def last_engines() -> set[str]:
    """Kernel families the calling thread's last libksq call launched (ksq_debug_last_engines)."""
    bits = lib().ksq_debug_last_engines()
    return {k for k, v in _lib.ENG.items() if bits & v}


def moe_gemm(wtype: int, weights: torch.Tensor, activation: torch.Tensor, router_logits: torch.Tensor,
             T: int, N: int, K: int, E: int, top_k: int, renorm: bool = False,
             out: torch.Tensor | None = None, workspace: torch.Tensor | None = None,
             return_routing: bool = False):
    """Expert-grouped MoE: fp32 activations [T, K], logits [T, E] -> fp32 [T, N]."""
    dev = activation.device
    if out is None:
        out = torch.empty((T, N), dtype=torch.float32, device=dev)
    ids = torch.empty((T, top_k), dtype=torch.int32, device=dev) if return_routing else None
    wts = torch.empty((T, top_k), dtype=torch.float32, device=dev) if return_routing else None
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    check(lib().ksq_moe_gemm(wtype, _ptr(weights), _ptr(activation), _ptr(router_logits), _ptr(out), T, N, K, E,
                             top_k, int(renorm), _ptr(ids), _ptr(wts), _ptr(workspace), ws_bytes, _stream()))
    return (out, ids, wts) if return_routing else out


def moe_gemm_routed(wtype: int, weights: torch.Tensor, activation: torch.Tensor, topk_ids: torch.Tensor,
                    topk_weights: torch.Tensor, T: int, N: int, K: int, E: int,
                    out: torch.Tensor | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    dev = activation.device
    top_k = topk_ids.shape[1]
    if out is None:
        out = torch.empty((T, N), dtype=torch.float32, device=dev)
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    check(lib().ksq_moe_gemm_routed(wtype, _ptr(weights), _ptr(activation), _ptr(topk_ids), _ptr(topk_weights),
                                    _ptr(out), T, N, K, E, top_k, _ptr(workspace), ws_bytes, _stream()))
    return out


def moe_workspace_size(wtype: int, T: int, N: int, K: int, E: int, top_k: int) -> int:
    return lib().ksq_moe_workspace_size(wtype, T, N, K, E, top_k)


def set_path(path: int) -> None:
    """Routing override for calls from this thread: 0 automatic, 1 v_dot4 decode kernels only,
    2 int8 MFMA GEMM where it applies, 3 the 4x4x4-MFMA small-batch kernel where it applies
    (M <= 8; M <= 32 with K % 128 == 0 and 16-byte aligned activations)."""
    check(lib().ksq_set_path(path))


def workspace_size(wtype: int, atype: int, M: int, N: int, K: int) -> int:
    return lib().ksq_gemm_workspace_size(wtype, atype, M, N, K)


def release() -> None:
    lib().ksq_release()


__all__ = ["ENTRY_POINTS", "gemm", "gemm_w16", "gemm_w16_workspace_size", "forward", "quantize_q8_1", "quantize_q8s", "quantize_q8f", "block_sumi", "last_engines", "set_path",
           "workspace_size", "moe_gemm", "moe_gemm_routed", "moe_workspace_size", "release", "_lib"]
