"""Shared helpers of the GPU parity tests (tolerances live in the tests)."""
from __future__ import annotations

import numpy as np
import torch

# bf16 attention output vs fp32 reference on the same bf16 inputs
MAX_ABS = 2e-2
MEAN_ABS = 2e-3


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def bits(t: torch.Tensor) -> np.ndarray:
    """bf16 tensor -> uint16 bit patterns."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def assert_attn_close(out: torch.Tensor, ref: np.ndarray, what: str = "") -> tuple[float, float]:
    o = to_np(out).astype(np.float64)
    err = np.abs(o - ref.astype(np.float64))
    mx, mean = float(err.max()) if err.size else 0.0, float(err.mean()) if err.size else 0.0
    assert np.isfinite(o).all(), f"{what}: non-finite output"
    assert mx <= MAX_ABS and mean <= MEAN_ABS, f"{what}: max-abs {mx:.3e} mean-abs {mean:.3e}"
    return mx, mean
