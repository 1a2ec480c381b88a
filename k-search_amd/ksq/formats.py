"""Block formats of the quantised matmul path (byte layouts of include/ksq_blocks.h).

The table mirrors the reference's quant-type registry
(kernelevalplus-main/core/operators/common/types.py:78-195) for the formats on
this path, plus the two K-quant super-blocks the reference lacks and the
fp32-scale activation block of the native W8A8C8 operator.
"""
from __future__ import annotations

from dataclasses import dataclass, field

from ._lib import W_Q4_0, W_Q4_1, W_Q4_K, W_Q5_0, W_Q5_1, W_Q6_K, W_Q8_0


@dataclass(frozen=True)
class QuantType:
    name: str
    size_bytes: int
    block_size: int
    wtype: int | None = None
    fields: tuple = field(default_factory=tuple)

    def nbytes(self, rows: int, K: int) -> int:
        if K % self.block_size:
            raise ValueError(f"K={K} is not a multiple of {self.block_size} for {self.name}")
        return rows * (K // self.block_size) * self.size_bytes


QUANT_TYPES = {
    "block_q4_0": QuantType("block_q4_0", 18, 32, W_Q4_0, (("d", "half", 0), ("qs", "uint8[16]", 2))),
    "block_q8_0": QuantType("block_q8_0", 34, 32, W_Q8_0, (("d", "half", 0), ("qs", "int8[32]", 2))),
    "block_q8_1": QuantType("block_q8_1", 36, 32, None, (("ds", "half2", 0), ("qs", "int8[32]", 4))),
    "block_q4_1": QuantType("block_q4_1", 20, 32, W_Q4_1,
                            (("d", "half", 0), ("m", "half", 2), ("qs", "uint8[16]", 4))),
    "block_q5_0": QuantType("block_q5_0", 22, 32, W_Q5_0,
                            (("d", "half", 0), ("qh", "uint8[4]", 2), ("qs", "uint8[16]", 6))),
    "block_q5_1": QuantType("block_q5_1", 24, 32, W_Q5_1,
                            (("d", "half", 0), ("m", "half", 2), ("qh", "uint8[4]", 4), ("qs", "uint8[16]", 8))),
    # activation block of the native W8A8C8 operator: fp32 scale, no sum
    "block_q8s": QuantType("block_q8s", 36, 32, None, (("d", "float", 0), ("qs", "int8[32]", 4))),
    "block_q4_K": QuantType("block_q4_K", 144, 256, W_Q4_K,
                            (("d", "half", 0), ("dmin", "half", 2), ("scales", "uint8[12]", 4), ("qs", "uint8[128]", 16))),
    "block_q6_K": QuantType("block_q6_K", 210, 256, W_Q6_K,
                            (("ql", "uint8[128]", 0), ("qh", "uint8[64]", 128), ("scales", "int8[16]", 192), ("d", "half", 208))),
}

# weight-type code -> block type name
WTYPE_NAMES = {W_Q4_0: "block_q4_0", W_Q8_0: "block_q8_0", W_Q4_K: "block_q4_K", W_Q6_K: "block_q6_K",
               W_Q4_1: "block_q4_1", W_Q5_0: "block_q5_0", W_Q5_1: "block_q5_1"}


def quant_type(name: str) -> QuantType:
    key = name if name.startswith("block_") else "block_" + name
    key = key.replace("_k", "_K") if key.endswith("_k") else key
    return QUANT_TYPES[key]
