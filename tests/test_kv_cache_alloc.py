"""Paged KV-cache sizing and binding (model_runner.py:152-206), on the CPU."""
import torch
from torch import nn

from dllm_serve_amd.engine.kv_cache import allocate_kv_cache, bind_kv_cache, block_bytes, kv_cache_blocks
from dllm_serve_amd.layers.attention import Attention


def test_block_bytes_and_page_count():
    # LLaDA-8B: one 256-row page across 32 layers of K and V = 128 MiB
    assert block_bytes(32, 32, 128) == 128 << 20
    # Dream-7B, 4 KV heads: 16 MiB; under tensor parallelism 2 the heads halve
    assert block_bytes(28, 4, 128) == 2 * 28 * 256 * 4 * 128 * 2
    assert block_bytes(28, 4, 128, world_size=2) == block_bytes(28, 4, 128) // 2
    GiB = 1 << 30
    # 288 GB device, 16 GB of weights resident (used = current = peak), 0.9 utilisation
    total, used, peak, cur = 288 * 10 ** 9, 17 * GiB, 16 * GiB, 16 * GiB
    n = kv_cache_blocks(total, used, peak, cur, 0.9, 32, 32, 128)
    assert n == int(total * 0.9 - used - peak + cur) // (128 << 20)
    assert 1500 < n < 2000
    # a transient peak above the current allocation is held back
    assert kv_cache_blocks(total, used, peak + 4 * GiB, cur, 0.9, 32, 32, 128) == n - 32


class _Model(nn.Module):
    def __init__(self, layers):
        super().__init__()
        self.attn = nn.ModuleList([Attention(4, 128, 128 ** -0.5, 2, causal=False) for _ in range(layers)])
        self.proj = nn.Linear(8, 8)


def test_bind_in_module_order():
    m = _Model(3)
    cache = allocate_kv_cache(m, 3, 2, 128, device="cpu", num_blocks=5)
    assert cache.shape == (2, 3, 5, 256, 2, 128) and cache.dtype == torch.bfloat16
    for i, a in enumerate(m.attn):
        assert a.k_cache.data_ptr() == cache[0, i].data_ptr()
        assert a.v_cache.data_ptr() == cache[1, i].data_ptr()
        assert a.k_cache.shape == (5, 256, 2, 128)
    assert bind_kv_cache(_Model(2), cache) == 2
    try:
        bind_kv_cache(_Model(4), cache)
    except ValueError:
        pass
    else:
        raise AssertionError("more layers than the cache holds must raise")
