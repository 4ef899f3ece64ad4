"""NeoX rotary embedding (dllmserve/layers/rotary_embedding.py:6-57).

inv_freq[i] = 1 / base**(2i/D) (f32), angle = pos * inv_freq, cos/sin in f32;
with x = [x1 | x2] split in halves:  y1 = x1 cos - x2 sin,  y2 = x2 cos + x1 sin.
Computed in f32 like the reference; used only to prepare inputs.
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
