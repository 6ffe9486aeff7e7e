"""BF16 bit-pattern helpers (numpy; ml_dtypes is not available).

BF16 tensors are carried as uint16 arrays holding the high half of an IEEE
float32. Conversion from float32 rounds to nearest even; NaNs stay NaN.
"""

from __future__ import annotations

import numpy as np


def f32_to_bf16_bits(x) -> np.ndarray:
    f = np.ascontiguousarray(x, dtype=np.float32)
    u = f.view(np.uint32)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    with np.errstate(over="ignore"):
        r = ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16))
    r = r.astype(np.uint16)
    if nan.any():
        r[nan] = ((u[nan] >> np.uint32(16)) | np.uint32(0x40)).astype(np.uint16)
    return r


def bf16_bits_to_f32(b) -> np.ndarray:
    u = np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)
    return u.view(np.float32)


def round_f32(x) -> np.ndarray:
    """float32 values rounded to the nearest BF16 (returned as float32)."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x))
