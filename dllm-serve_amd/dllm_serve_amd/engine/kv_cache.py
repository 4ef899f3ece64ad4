"""Paged KV-cache sizing and binding (ModelRunner.allocate_kv_cache,
dllmserve/engine/model_runner.py:152-206).

The cache is one bf16 tensor [2, num_layers, num_blocks, 256, Hkv / world,
head_dim]: K then V, per layer, 256-row pages, rows of Hkv*head_dim elements
-- the layout the attention kernels address by slot (slot = page * 256 +
row).  Its page count is what the reference computes from the device's
memory after the model is loaded:

    num_blocks = int(total * utilization - used - peak + current) // block_bytes
    block_bytes = 2 * num_layers * 256 * (Hkv / world) * head_dim * 2

and every module with ``k_cache`` / ``v_cache`` attributes gets the views of
its layer, in module order.  On MI355X's 288 GB the default utilisation
leaves room for several hundred thousand pages of an 8B model.
"""
from __future__ import annotations

import torch
from torch import nn

BLOCK_SIZE = 256


def block_bytes(num_layers: int, num_kv_heads: int, head_dim: int, world_size: int = 1,
                block_size: int = BLOCK_SIZE) -> int:
    return 2 * num_layers * block_size * (num_kv_heads // world_size) * head_dim * torch.bfloat16.itemsize


def kv_cache_blocks(total: int, used: int, peak: int, current: int, utilization: float, num_layers: int,
                    num_kv_heads: int, head_dim: int, world_size: int = 1, block_size: int = BLOCK_SIZE) -> int:
    """Page count of model_runner.py:168-185 from the device memory figures."""
    return int(total * utilization - used - peak + current) // block_bytes(num_layers, num_kv_heads, head_dim,
                                                                          world_size, block_size)


def allocate_kv_cache(model: nn.Module, num_layers: int, num_kv_heads: int, head_dim: int,
                      gpu_memory_utilization: float = 0.9, world_size: int = 1, device=None,
                      num_blocks: int | None = None) -> torch.Tensor:
    """Size (unless num_blocks is given), allocate and bind the paged cache."""
    device = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    if num_blocks is None:
        free, total = torch.cuda.mem_get_info(device)
        stats = torch.cuda.memory_stats(device)
        num_blocks = kv_cache_blocks(total, total - free, stats["allocated_bytes.all.peak"],
                                     stats["allocated_bytes.all.current"], gpu_memory_utilization,
                                     num_layers, num_kv_heads, head_dim, world_size)
    if num_blocks <= 0:
        raise RuntimeError(f"no memory left for the KV cache ({num_blocks} pages)")
    cache = torch.zeros(2, num_layers, num_blocks, BLOCK_SIZE, num_kv_heads // world_size, head_dim,
                        dtype=torch.bfloat16, device=device)
    bind_kv_cache(model, cache)
    return cache


def bind_kv_cache(model: nn.Module, cache: torch.Tensor) -> int:
    """Give each module with k_cache / v_cache its layer's views (module
    order, model_runner.py:201-206); returns the number of layers bound."""
    layer = 0
    for m in model.modules():
        if hasattr(m, "k_cache") and hasattr(m, "v_cache"):
            if layer >= cache.shape[1]:
                raise ValueError(f"the model has more attention layers than the cache's {cache.shape[1]}")
            m.k_cache = cache[0, layer]
            m.v_cache = cache[1, layer]
            layer += 1
    return layer
