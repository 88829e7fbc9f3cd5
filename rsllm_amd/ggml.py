"""GGUF tensor-type ids and block geometry.

Mirrors ``GgmlType`` and its ``block_elements`` / ``block_bytes`` /
``byte_size`` (rsllm-gguf/src/tensor.rs:26-194) for the types this backend
handles, plus the ones ``matmul_quant_f32`` names in its dtype guard.
"""
from __future__ import annotations

import enum


class GgmlType(enum.IntEnum):
    """GGUF on-disk type ids (rsllm-gguf/src/tensor.rs:26-85)."""

    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q4_1 = 3
    Q8_0 = 8
    Q2_K = 10
    Q3_K = 11
    Q4_K = 12
    Q5_K = 13
    Q6_K = 14
    Q8_K = 15
    IQ2_XXS = 16
    BF16 = 30

    def block_elements(self) -> int:  # tensor.rs:128-150
        if self in (GgmlType.F32, GgmlType.F16, GgmlType.BF16):
            return 1
        if self in (GgmlType.Q4_0, GgmlType.Q4_1, GgmlType.Q8_0):
            return 32
        return 256

    def block_bytes(self) -> int:  # tensor.rs:153-184
        return {
            GgmlType.F32: 4, GgmlType.F16: 2, GgmlType.BF16: 2,
            GgmlType.Q4_0: 18, GgmlType.Q4_1: 20, GgmlType.Q8_0: 34,
            GgmlType.Q2_K: 84, GgmlType.Q3_K: 110, GgmlType.Q4_K: 144,
            GgmlType.Q5_K: 176, GgmlType.Q6_K: 210, GgmlType.Q8_K: 292,
            GgmlType.IQ2_XXS: 66,
        }[self]

    def byte_size(self, elements: int) -> int:  # tensor.rs:188-194
        be = self.block_elements()
        return (elements + be - 1) // be * self.block_bytes()

    def row_bytes(self, in_dim: int) -> int:
        """Bytes of one weight row of ``in_dim`` elements (quant_matmul.rs:75-76)."""
        return in_dim // self.block_elements() * self.block_bytes()

    def gguf_name(self) -> str:
        return self.name.lower()
