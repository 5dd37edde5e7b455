"""Precision modes of a quantized leaf.

Mirrors the mode set of mtc/core/types.py:9-28 (PrecisionMode). A mode value
is also the code width in bits; P0 marks a dropped leaf (no payload, all zeros).
"""

from enum import IntEnum


class PrecisionMode(IntEnum):
    P0 = 0     # dropped leaf: zero payload, reconstructs to +0.0
    P2 = 2     # signed codes in [-2, 1]
    P3 = 3     # signed codes in [-4, 3]
    P4 = 4     # signed codes in [-8, 7]
    P5 = 5     # signed codes in [-16, 15]
    P6 = 6     # signed codes in [-32, 31]
    P8 = 8     # signed codes in [-128, 127]
    P16 = 16   # signed codes in [-32768, 32767]

    @property
    def values_per_byte(self) -> float:
        return float("inf") if self.value == 0 else 8.0 / self.value

    @property
    def bytes_per_value(self) -> float:
        return self.value / 8.0
