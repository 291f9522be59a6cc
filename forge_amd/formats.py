"""Block-format table for the quantized-matmul hot path.

Mirrors forge::DataType (include/forge/types.h:7-26) and the block geometry of
QuantTraits / data_type_traits (include/forge/quant_traits.h:19-95,
src/operators/cpu/quant_traits.cpp:33-52) for the ten formats this library
implements: the five of the decode benchmarks (Q4_0, Q4_1, Q8_0, Q4_K, Q6_K)
and the five other formats a Q4_K_M/Q5_K_M model file mixes in (Q5_0, Q5_1,
Q3_K, Q5_K, IQ4_NL).  The numeric dtype values are the reference's, so a caller can pass
``static_cast<uint32_t>(tensor->dtype())`` straight through the C ABI.
"""
from __future__ import annotations

from dataclasses import dataclass

FP32 = 0
Q4_0 = 2
Q4_1 = 3
Q4_K = 4
Q8_0 = 7
Q5_0 = 8
Q5_1 = 9
Q3_K = 11
Q5_K = 12
Q6_K = 13
IQ4_NL = 17


@dataclass(frozen=True)
class BlockFormat:
    dtype: int
    name: str
    block_elems: int
    block_bytes: int

    @property
    def bytes_per_weight(self) -> float:
        return self.block_bytes / self.block_elems

    def row_bytes(self, K: int) -> int:
        return -(-K // self.block_elems) * self.block_bytes

    def matrix_bytes(self, N: int, K: int) -> int:
        return N * self.row_bytes(K)


FORMATS = {
    Q4_0: BlockFormat(Q4_0, "q4_0", 32, 18),
    Q4_1: BlockFormat(Q4_1, "q4_1", 32, 20),
    Q8_0: BlockFormat(Q8_0, "q8_0", 32, 34),
    Q4_K: BlockFormat(Q4_K, "q4_k", 256, 144),
    Q6_K: BlockFormat(Q6_K, "q6_k", 256, 210),
    Q5_0: BlockFormat(Q5_0, "q5_0", 32, 22),
    Q5_1: BlockFormat(Q5_1, "q5_1", 32, 24),
    Q3_K: BlockFormat(Q3_K, "q3_k", 256, 110),
    Q5_K: BlockFormat(Q5_K, "q5_k", 256, 176),
    IQ4_NL: BlockFormat(IQ4_NL, "iq4_nl", 32, 18),
}

# Formats with an aligned (repacked) device layout; the others run from
# their GGUF bytes only.
PACKED = (Q4_0, Q4_1, Q8_0, Q4_K, Q6_K)

BY_NAME = {f.name: f for f in FORMATS.values()}


def fmt(dtype) -> BlockFormat:
    """Look a format up by DataType value or by name ('q4_0', 'Q4_K', ...)."""
    if isinstance(dtype, str):
        return BY_NAME[dtype.lower()]
    return FORMATS[int(dtype)]
