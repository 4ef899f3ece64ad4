"""Drop-in ``RotaryEmbedding`` / ``get_rope`` on the gfx950 RoPE kernel (K7).

Interface of dllmserve/layers/rotary_embedding.py:19-69:
``RotaryEmbedding(head_size, rotary_dim, max_position_embeddings, base)``
builds the same f32 table ``cos_sin_cache`` [max_position, head_size]
(cos of the head_size/2 frequencies, then their sin; :30-38), and
``forward(positions, query, key)`` returns the NeoX-rotated (query, key)
(:41-57).  One kernel launch rotates both; the result is bit-exact against
the reference's f32 expression ``x1*cos - x2*sin`` / ``x2*cos + x1*sin``
evaluated op by op and rounded to bf16 (the kernel does not fuse the
multiply-adds).  There is no CPU path: tensors must be bf16 on the GPU.
"""
from __future__ import annotations

from functools import lru_cache

import torch
from torch import nn

from .. import _capi


def _rows(x: torch.Tensor, n: int, head_size: int, name: str) -> torch.Tensor:
    """[n, H*D] or [n, H, D] with a contiguous last dim -> [n, H, D] view."""
    if x.dtype != torch.bfloat16:
        raise ValueError(f"{name} must be bfloat16 (got {x.dtype})")
    if x.shape[0] != n or x.stride(-1) != 1:
        raise ValueError(f"{name} must be [num_tokens, ...] with a contiguous last dim; got shape "
                         f"{tuple(x.shape)} strides {x.stride()}")
    v = x.view(n, -1, head_size)
    if v.stride(1) != head_size:
        raise ValueError(f"{name}: heads must be contiguous inside a token row")
    return v


class RotaryEmbedding(nn.Module):
    """NeoX rotary embedding (rotary_embedding.py:19-57).

    ``inplace=True`` rotates query / key in their own storage (they are
    usually views of the QKV projection output that nothing else reads);
    the default returns new tensors, as the reference does."""

    def __init__(self, head_size: int, rotary_dim: int, max_position_embeddings: int, base: float,
                 inplace: bool = False) -> None:
        super().__init__()
        self.head_size = head_size
        assert rotary_dim == head_size
        # Same table construction as rotary_embedding.py:30-38 (f32 ops on the
        # default device), so the kernel reads the same cos / sin values.
        inv_freq = 1.0 / (base ** (torch.arange(0, rotary_dim, 2, dtype=torch.float) / rotary_dim))
        t = torch.arange(max_position_embeddings, dtype=torch.float)
        freqs = torch.einsum("i,j -> ij", t, inv_freq)
        cache = torch.cat((freqs.cos(), freqs.sin()), dim=-1)
        self.register_buffer("cos_sin_cache", cache, persistent=False)
        self.inplace = inplace

    def forward(self, positions: torch.Tensor, query: torch.Tensor,
                key: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        n = positions.size(0)
        D = self.head_size
        if self.cos_sin_cache.device != query.device:
            self.cos_sin_cache = self.cos_sin_cache.to(query.device)
        pos = positions if positions.dtype == torch.int64 else positions.to(torch.int64)
        pos = pos.contiguous()
        q_in = _rows(query, n, D, "query")
        k_in = _rows(key, n, D, "key")
        if self.inplace:
            q_out, k_out, q_ret, k_ret = q_in, k_in, query, key
        else:
            q_ret = torch.empty(query.shape, dtype=query.dtype, device=query.device)
            k_ret = torch.empty(key.shape, dtype=key.dtype, device=key.device)
            q_out, k_out = q_ret.view(n, -1, D), k_ret.view(n, -1, D)
        _capi.rope_neox(q_in, q_out, k_in, k_out, pos, self.cos_sin_cache, n, q_in.shape[1], k_in.shape[1], D)
        return q_ret, k_ret


@lru_cache(1)
def get_rope(head_size: int, rotary_dim: int, max_position: int, base: float, rope_scaling: dict | None = None):
    """rotary_embedding.py:60-69."""
    assert rope_scaling is None
    return RotaryEmbedding(head_size, rotary_dim, max_position, base)
