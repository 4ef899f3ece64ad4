"""NeoX rotary embedding (dllmserve/layers/rotary_embedding.py:6-57).

inv_freq[i] = 1 / base**(2i/D) (f32), angle = pos * inv_freq, cos/sin in f32;
with x = [x1 | x2] split in halves:  y1 = x1 cos - x2 sin,  y2 = x2 cos + x1 sin.
Computed in f32 like the reference.  ``apply`` prepares inputs (C1);
``rotate_table`` gives the expected results of the K7 kernel: the reference's table
lookup (rotary_embedding.py:47-49) and its f32 expression evaluated op by op
(each product, sum and difference rounded to f32; :12-16), rounded to bf16.
"""
from __future__ import annotations

import numpy as np


def cos_sin(positions, head_dim: int, base: float):
    inv_freq = (1.0 / (np.float32(base) ** (np.arange(0, head_dim, 2, dtype=np.float32) / np.float32(head_dim))))
    inv_freq = inv_freq.astype(np.float32)
    t = np.asarray(positions, dtype=np.float32)
    freqs = np.outer(t, inv_freq).astype(np.float32)
    return np.cos(freqs).astype(np.float32), np.sin(freqs).astype(np.float32)


def apply(x: np.ndarray, positions, base: float) -> np.ndarray:
    """x: [N, H, D] -> rotated copy (f32 math, returned as f32)."""
    D = x.shape[-1]
    cos, sin = cos_sin(positions, D, base)
    cos = cos[:, None, :]
    sin = sin[:, None, :]
    xf = x.astype(np.float32)
    x1, x2 = xf[..., : D // 2], xf[..., D // 2:]
    return np.concatenate([x1 * cos - x2 * sin, x2 * cos + x1 * sin], axis=-1).astype(np.float32)


def rotate_table(x: np.ndarray, positions, table: np.ndarray) -> np.ndarray:
    """x: [N, H, D] f32 (bf16 values), table: [P, D] f32 = [cos | sin] rows
    (rotary_embedding.py:30-38).  Returns the rotated tensor as bf16 bits
    [N, H, D] (uint16): y1 = x1*c - x2*s, y2 = x2*c + x1*s with every
    operation rounded to f32 (rotary_embedding.py:6-17,47-56)."""
    from .bf16 import f32_to_bf16_bits

    D = x.shape[-1]
    h = D // 2
    rows = np.asarray(table, dtype=np.float32)[np.asarray(positions, dtype=np.int64)]
    c = rows[:, None, :h]
    s = rows[:, None, h:]
    xf = np.asarray(x, dtype=np.float32)
    x1, x2 = xf[..., :h], xf[..., h:]
    y1 = np.subtract(np.multiply(x1, c, dtype=np.float32), np.multiply(x2, s, dtype=np.float32), dtype=np.float32)
    y2 = np.add(np.multiply(x2, c, dtype=np.float32), np.multiply(x1, s, dtype=np.float32), dtype=np.float32)
    return f32_to_bf16_bits(np.concatenate([y1, y2], axis=-1))
