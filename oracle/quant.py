"""bfloat16 / float16 round-to-nearest-even in NumPy (test infrastructure).

bfloat16 is the upper 16 bits of an IEEE binary32.  Rounding a float32 to
bfloat16 with ties-to-even adds 0x7FFF plus the lowest kept bit to the
32-bit pattern and truncates; NaNs are mapped to a quiet NaN with the sign
kept (adding to a NaN payload could carry into the exponent and turn it
into an infinity).  The reference has no bfloat16 storage at all
(reference dtype.py:31 maps bfloat16 to float32), so this convention is the
device path's own and is pinned by IEEE known answers.
"""
from __future__ import annotations

import numpy as np


def bf16_bits(x) -> np.ndarray:
    """float32 values -> uint16 bfloat16 bit patterns (RNE)."""
    f = np.ascontiguousarray(x, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    lsb = (u >> np.uint64(16)) & np.uint64(1)
    rounded = ((u + np.uint64(0x7FFF) + lsb) >> np.uint64(16)).astype(np.uint16)
    nan = np.isnan(f)
    if nan.any():
        sign = ((u >> np.uint64(16)) & np.uint64(0x8000)).astype(np.uint16)
        rounded = np.where(nan, sign | np.uint16(0x7FC0), rounded)
    return rounded


def bf16_to_f32(bits) -> np.ndarray:
    """uint16 bfloat16 bit patterns -> float32 (exact)."""
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    return (b.astype(np.uint32) << np.uint32(16)).view(np.float32)


def round_bf16(x) -> np.ndarray:
    """float32 values rounded to the nearest bfloat16, returned as float32."""
    return bf16_to_f32(bf16_bits(x))


def round_f16(x) -> np.ndarray:
    """float32 values rounded to the nearest float16 (IEEE RNE, NumPy's
    cast), returned as float32."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def quantize(x, dtype: str) -> np.ndarray:
    """Rounds float32 data to `dtype` ('float32', 'float16', 'bfloat16') and
    returns it as float32 values."""
    if dtype == "float32":
        return np.asarray(x, dtype=np.float32)
    if dtype == "float16":
        return round_f16(x)
    if dtype == "bfloat16":
        return round_bf16(x)
    raise ValueError(dtype)
