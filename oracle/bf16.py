"""bfloat16 rounding on numpy float32 arrays (round-to-nearest-even).

The reference rounds with MLX's ``astype(mx.bfloat16)``, which is IEEE
round-to-nearest-even on the top 16 bits of an fp32 value.  Pinned against
torch's bfloat16 cast in tests/test_oracle_bf16.py.
"""

from __future__ import annotations

import numpy as np


def bf16r(a) -> np.ndarray:
    """Round to the nearest bf16 (ties to even); returns float32 values."""
    a = np.array(a, dtype=np.float32, order="C")  # keeps 0-d inputs 0-d
    bits = a.view(np.uint32).astype(np.uint64)
    lsb = (bits >> 16) & 1
    rounded = (bits + 0x7FFF + lsb) & 0xFFFF0000
    nan = np.isnan(a)
    if nan.any():
        rounded = np.where(nan, (bits | 0x00400000) & 0xFFFF0000, rounded)
    return rounded.astype(np.uint32).view(np.float32).reshape(a.shape)


def to_bf16_bits(a) -> np.ndarray:
    """bf16 bit patterns (uint16) of the bf16-rounded values of ``a``."""
    return (bf16r(a).view(np.uint32) >> 16).astype(np.uint16)


def from_bf16_bits(bits) -> np.ndarray:
    """float32 values of uint16 bf16 bit patterns."""
    b = np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16
    return b.view(np.float32)


def ulp_bf16(a) -> np.ndarray:
    """Spacing of bf16 numbers at |a| (for tolerance statements)."""
    a = np.abs(np.asarray(a, dtype=np.float32))
    e = np.floor(np.log2(np.maximum(a, np.float32(2.0 ** -126))))
    return np.exp2(e - 7).astype(np.float32)
