"""bfloat16 helpers on numpy arrays (bit-exact, round to nearest even).

bf16 is the upper half of an IEEE f32; rounding adds 0x7FFF plus the lowest
kept bit before truncating, which is round-half-to-even (NaNs become the
canonical quiet NaN 0x7FC0).
"""
from __future__ import annotations

import numpy as np


def f32_to_bf16_bits(x) -> np.ndarray:
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        r = np.where(nan, np.uint16(0x7FC0), r)
    return r


def bf16_bits_to_f32(b) -> np.ndarray:
    b = np.asarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def round_bf16(x) -> np.ndarray:
    """f32 -> nearest bf16, returned as f32 values."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


def f64_to_bf16_bits(x) -> np.ndarray:
    """f64 -> f32 (nearest even) -> bf16 (nearest even); the two-step rule
    the GPU selection kernels use."""
    return f32_to_bf16_bits(np.asarray(x, dtype=np.float64).astype(np.float32))
