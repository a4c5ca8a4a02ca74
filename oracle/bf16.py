"""bf16 bit helpers (NumPy) for the oracle -- test infrastructure only.

bf16 values travel as their uint16 bit patterns so that the oracle and the HIP
path see identical bits.  Rounding is round-to-nearest-even, as torch's
``.to(torch.bfloat16)`` (h3/htrc_flat.py:211-212) and Triton's
``.to(tl.bfloat16)`` (h3/htrc_flat_triton.py:154, 183).
"""
from __future__ import annotations

import numpy as np


def to_f32(bits: np.ndarray) -> np.ndarray:
    """bf16 bit patterns (uint16) -> float32 (exact)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def from_f32(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns, round to nearest even; NaN stays quiet NaN."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    if nan.any():
        r = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)
    return r


def round_f32(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bf16 value, returned as float32."""
    return to_f32(from_f32(x))
