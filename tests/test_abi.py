"""C-ABI checks that need no GPU: the library loads, exports every symbol
include/ksq.h declares, and rejects bad arguments on the host before any launch
(the reference entries never validate; ksq records a status instead of launching)."""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_symbols():
    txt = open(os.path.join(ROOT, "include", "ksq.h")).read()
    return re.findall(r"^KSQ_API\s+[\w\s\*]+?\b(\w+)\(", txt, flags=re.M)


def test_header_declarations_found():
    syms = _declared_symbols()
    assert "gemm_w4a32c8_q4_0_fp32_int8" in syms and "ksq_gemm" in syms
    assert len(syms) >= 19


def test_library_exports_every_declared_symbol():
    from ksq import _lib
    L = _lib.lib()
    for s in _declared_symbols():
        assert hasattr(L, s), s
        assert s in _lib.SIGNATURES, f"{s} has no ctypes signature"


def test_block_layout_header_matches_formats():
    from ksq.formats import QUANT_TYPES
    hdr = open(os.path.join(ROOT, "include", "ksq_blocks.h")).read()
    for name, size in (("q4_0", 18), ("q8_0", 34), ("q8_1", 36), ("q4_K", 144), ("q6_K", 210)):
        assert f"sizeof(ksq_block_{name}) == {size}" in hdr
        assert QUANT_TYPES["block_" + name].size_bytes == size


def test_version_and_error_strings():
    from ksq import _lib
    L = _lib.lib()
    assert b"gfx950" in L.ksq_version()
    assert L.ksq_error_string(0) == b"ok"
    assert L.ksq_error_string(3) == b"misaligned pointer"


FAKE = 1 << 20  # a 16-byte aligned non-null address; never dereferenced by the failing paths below


@pytest.mark.parametrize("args,status", [
    ((9, 0, FAKE, FAKE, FAKE, 1, 1, 32), 4),          # unknown weight type
    ((0, 8, FAKE, FAKE, FAKE, 1, 1, 32), 4),          # unknown activation type
    ((0, 0, FAKE, FAKE, FAKE, -1, 1, 32), 2),         # negative M
    ((0, 0, FAKE, FAKE, FAKE, 1, 1, 48), 2),          # K % 32
    ((2, 0, FAKE, FAKE, FAKE, 1, 1, 288), 2),         # K-quant needs K % 256
    ((0, 0, None, FAKE, FAKE, 1, 1, 32), 1),          # null weight
    ((0, 0, FAKE, FAKE, None, 1, 1, 32), 1),          # null output
    ((0, 0, FAKE + 1, FAKE, FAKE, 1, 1, 32), 3),      # odd weight address
    ((2, 0, FAKE + 2, FAKE, FAKE, 1, 1, 256), 3),     # K-quant weight not 4-byte aligned
    ((0, 0, FAKE, FAKE + 4, FAKE, 1, 1, 32), 3),      # fp32 activation not 16-byte aligned
    ((0, 1, FAKE, FAKE + 2, FAKE, 1, 1, 32), 3),      # Q8_1 activation not 4-byte aligned
    ((0, 0, FAKE, FAKE, FAKE + 2, 1, 1, 32), 3),      # output not 4-byte aligned
    ((0, 9, FAKE, FAKE, FAKE, 1, 1, 32), 4),          # activation type past KSQ_A_F32_Q8F_LROUND
    ((0, 4, FAKE, FAKE + 8, FAKE, 1, 1, 32), 3),      # fp16 activation not 16-byte aligned
    ((4, 5, FAKE, FAKE, FAKE, 1, 1, 256), 4),         # block_q8f with Q4_1 weights
    ((3, 6, FAKE, FAKE, FAKE, 1, 1, 256), 4),         # block_q8f with Q6_K weights
    ((0, 5, FAKE, FAKE, FAKE, 1, 1, 32), 2),          # block_q8f needs K % 256
    ((0, 7, FAKE, FAKE, FAKE, 1, 1, 224), 2),
    ((0, 5, FAKE, FAKE + 4, FAKE, 1, 1, 256), 3),     # block_q8f activation not 16-byte aligned
    ((1, 6, FAKE + 2, FAKE, FAKE, 1, 1, 256), 3),     # weight not 16-byte aligned with block_q8f
])
def test_gemm_rejects_bad_arguments(args, status):
    from ksq import _lib
    L = _lib.lib()
    st = L.ksq_gemm(*args, None, 0, None)
    assert st == status
    assert L.ksq_last_error() == status
    assert L.ksq_last_error_message()


def test_empty_calls_are_noops():
    from ksq import _lib
    L = _lib.lib()
    assert L.ksq_gemm(0, 0, None, None, None, 0, 5, 64, None, 0, None) == 0
    assert L.ksq_gemm(0, 0, None, None, None, 5, 0, 64, None, 0, None) == 0
    assert L.ksq_quantize_q8_1(None, None, 0, 64, None) == 0
    assert L.ksq_quantize_q8_1_variant(2, None, None, 0, 64, None) == 0


def test_fp16_fused_entry_rejects_bad_arguments():
    """ksq_gemm_q4_0_fp16_fused validates like ksq_gemm, in its own (M weight rows) orientation."""
    from ksq import _lib
    L = _lib.lib()
    assert L.ksq_gemm_q4_0_fp16_fused(FAKE, FAKE + 8, FAKE, 4, 2, 64, None, 0, None) == 3   # activation alignment
    assert L.ksq_gemm_q4_0_fp16_fused(FAKE, FAKE, FAKE, 4, 2, 48, None, 0, None) == 2       # K % 32
    assert L.ksq_gemm_q4_0_fp16_fused(None, FAKE, FAKE, 4, 2, 64, None, 0, None) == 1       # null weight
    assert L.ksq_gemm_q4_0_fp16_fused(FAKE, FAKE, FAKE, 0, 2, 64, None, 0, None) == 0       # empty: no-op


def test_quantize_variant_rejects_unknown_variant():
    from ksq import _lib
    L = _lib.lib()
    assert L.ksq_quantize_q8_1_variant(4, None, None, 1, 64, None) == 4      # KSQ_ERR_TYPE
    assert L.ksq_quantize_q8_1_variant(-1, None, None, 1, 64, None) == 4
    assert L.ksq_quantize_q8_1_variant(1, None, None, 1, 48, None) == 2      # KSQ_ERR_SHAPE


def test_quantize_q8f_rejects_bad_arguments():
    from ksq import _lib
    L = _lib.lib()
    assert L.ksq_quantize_q8f(2, FAKE, FAKE, 1, 64, None) == 4       # unknown rule
    assert L.ksq_quantize_q8f(0, FAKE, FAKE, 1, 48, None) == 2       # K % 32
    assert L.ksq_quantize_q8f(1, FAKE + 4, FAKE, 1, 64, None) == 3   # x alignment
    assert L.ksq_quantize_q8f(1, None, None, 0, 64, None) == 0       # empty: no-op


def test_workspace_size():
    """fp32 input needs its block_q8_1 copy, quantised input none (M = 2048: no split-K).  Q4_0 / Q4_1
    at this shape take the LDS-DMA GEMM, whose activations are planar: [M][K] int8 quants, d and nc
    as [K/32][Mp] floats, -s_a as [K/128][Mp][4] fp16 (Mp = M rounded up to 128)."""
    from ksq import _lib
    L = _lib.lib()
    planar = 2048 * 4096 + 2 * 128 * 2048 * 4 + 32 * 2048 * 8
    assert L.ksq_gemm_workspace_size(0, 0, 2048, 4096, 4096) == planar
    assert L.ksq_gemm_workspace_size(4, 0, 2048, 4096, 4096) == planar
    # M = 1100 (Mp = 1152; each plane 256-byte aligned), split in two along K: the partial sums follow
    assert L.ksq_gemm_workspace_size(0, 0, 1100, 4096, 4096) == (1100 * 4096 + 2 * 128 * 1152 * 4 + 32 * 1152 * 8
                                                                 + 2 * 1100 * 4096 * 4)
    assert L.ksq_gemm_workspace_size(0, 1, 2048, 4096, 4096) == 0
    assert L.ksq_gemm_workspace_size(1, 0, 2048, 4096, 4096) == 2048 * 128 * 36
    # block_q8f (fp32 d and s): 40-byte blocks
    assert L.ksq_gemm_workspace_size(0, 6, 2048, 4096, 4096) == 2048 * 128 * 40
    assert L.ksq_gemm_workspace_size(0, 5, 2048, 4096, 4096) == 0
    # the fused FP16 orientation: the quantised copy of its N x K activations plus an M x N
    # transposition buffer, each 256-byte aligned
    assert L.ksq_gemm_q4_0_fp16_fused_workspace_size(4096, 8, 4096) == 8 * 128 * 36 + 4096 * 8 * 4
    assert L.ksq_gemm_q4_0_fp16_fused_workspace_size(4096, 3, 4096) == 13824 + 49152


def test_void_entry_records_error():
    """The drop-in void entry validates too (the reference's would launch blindly)."""
    from ksq import _lib
    L = _lib.lib()
    L.gemm_w4a32c8_q4_0_fp32_int8(FAKE, FAKE, FAKE, 1, 1, 33)
    assert L.ksq_last_error() == 2


def test_forward_mirrors_harness_checks():
    import torch
    from ksq import forward
    w = torch.zeros(8, dtype=torch.uint8)
    a = torch.zeros(32, dtype=torch.float32)
    with pytest.raises(RuntimeError, match="Weight must be CUDA tensor"):
        forward(w, a, 1, 1, 32)


def test_set_path_validation():
    from ksq import _lib
    L = _lib.lib()
    assert L.ksq_set_path(5) == 4
    assert L.ksq_set_path(-1) == 4
    assert L.ksq_set_path(4) == 4
    assert L.ksq_set_path(3) == 0
    assert L.ksq_set_path(0) == 0
