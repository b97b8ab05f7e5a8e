"""float32 -> bfloat16 rounding on the CPU -- test infrastructure only.

The bf16-KV tolerance of the data path is stated against the reference attention run on K and V
rounded to bfloat16. This module supplies that rounding: bfloat16 is
the upper 16 bits of a binary32, and rounding to nearest with ties to even adds 0x7FFF plus the
lowest kept bit before truncating. NaN maps to the canonical quiet NaN 0x7FC0.
"""

from __future__ import annotations

import numpy as np

__all__ = ["bf16_bits", "bf16_round", "bits_to_f32"]


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round float32 values to bfloat16 bit patterns (uint16), nearest-even."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return np.where(nan, 0x7FC0, rounded).astype(np.uint16)


def bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """Widen bfloat16 bit patterns to float32 (exact)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 values rounded to the nearest bfloat16, returned as float32."""
    return bits_to_f32(bf16_bits(x))
