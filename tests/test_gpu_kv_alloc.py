"""Paged KV cache sized from the MI355X's live memory figures
(ModelRunner.allocate_kv_cache, dllmserve/engine/model_runner.py:152-206):
allocate_kv_cache with no page count reads torch.cuda.mem_get_info and the
allocator's peak / current bytes, sizes [2, L, pages, 256, Hkv, D], binds the
layer views in module order, and the kernels then run on those views: one
state-1 step (selection + store) and one state-2 step against the oracle."""
import numpy as np
import pytest
import torch
from torch import nn

from helpers import assert_attn_close, bits, to_np
from oracle.bf16 import f32_to_bf16_bits

from oracle import attention as oatt
from dllm_serve_amd.engine.kv_cache import allocate_kv_cache, block_bytes, kv_cache_blocks
from dllm_serve_amd.engine.sequence import PageAllocator, Sequence, prepare_step, slot_mapping_for
from dllm_serve_amd.layers.attention import Attention
from dllm_serve_amd.sparse.state import SparseConfig, keep_count
from dllm_serve_amd.utils.context import reset_context

pytestmark = pytest.mark.gpu

D = 128
MASK = 126336


class _TwoLayers(nn.Module):
    def __init__(self, Hq, Hkv):
        super().__init__()
        self.layers = nn.ModuleList([Attention(Hq, D, D ** -0.5, Hkv, causal=False) for _ in range(2)])


def test_allocate_from_device_memory_and_run(dev, monkeypatch):
    Hq, Hkv, L = 16, 8, 2
    model = _TwoLayers(Hq, Hkv)
    torch.cuda.empty_cache()
    free, total = torch.cuda.mem_get_info(dev)
    st = torch.cuda.memory_stats(dev)
    used, peak, cur = total - free, st["allocated_bytes.all.peak"], st["allocated_bytes.all.current"]
    want_pages = 64
    bb = block_bytes(L, Hkv, D)
    # a utilisation that leaves room for about 64 pages beyond what is held now
    util = (used + peak - cur + want_pages * bb + bb // 2) / total
    print(f"kv alloc: total {total / 2**30:.1f} GiB, used {used / 2**30:.2f} GiB, peak {peak}, current {cur}, "
          f"utilisation {util:.6f}", flush=True)
    # record the figures allocate_kv_cache itself reads
    seen = {}
    real_info, real_stats = torch.cuda.mem_get_info, torch.cuda.memory_stats

    def info(d=None):
        seen["info"] = real_info(d)
        return seen["info"]

    def stats(d=None):
        seen["stats"] = real_stats(d)
        return seen["stats"]

    monkeypatch.setattr(torch.cuda, "mem_get_info", info)
    monkeypatch.setattr(torch.cuda, "memory_stats", stats)
    cache = allocate_kv_cache(model, L, Hkv, D, gpu_memory_utilization=util, device=dev)
    monkeypatch.undo()
    f2, t2 = seen["info"]
    s2 = seen["stats"]
    expect = kv_cache_blocks(t2, t2 - f2, s2["allocated_bytes.all.peak"], s2["allocated_bytes.all.current"], util,
                             L, Hkv, D)
    assert cache.shape == (2, L, expect, 256, Hkv, D)
    assert abs(expect - want_pages) <= 1, expect
    assert cache.dtype == torch.bfloat16 and cache.device.type == "cuda"
    for i, a in enumerate(model.layers):
        assert a.k_cache.data_ptr() == cache[0, i].data_ptr() and a.v_cache.data_ptr() == cache[1, i].data_ptr()

    # a sparse sequence: step 0 full, step 1 select + store, step 2 block vs cache, on both layers' views
    cfg = SparseConfig(enabled=True, default_block_len=32, retention_ratio=0.5, pool_kernel=3, delay_step=1,
                       head_select=True)
    seq = Sequence([1] * 500, 64, MASK, cfg, device=dev)
    PageAllocator(range(expect - 1, expect - 1 - seq.num_blocks, -1)).allocate(seq)
    ref = np.zeros((L, 2, expect * 256, Hkv, D), dtype=np.float32)
    g = torch.Generator().manual_seed(9)
    n_keep = keep_count(564 - 32, 0.5)
    for step in range(3):
        prepare_step([seq], dev)
        rows = 32 if step == 2 else 564
        desc = [dict(mode=0, rows=rows)] if step == 0 else (
            [dict(mode=1, rows=rows, blk_start=500, blk_len=32, n_keep=n_keep, head_select=True, pool_k=3)]
            if step == 1 else [dict(mode=2, rows=rows)])
        slots = [slot_mapping_for(seq)] if step else [[]]
        for li, a in enumerate(model.layers):
            q = torch.randn(rows, Hq, D, generator=g).to(torch.bfloat16)
            k = torch.randn(rows, Hkv, D, generator=g).to(torch.bfloat16)
            v = torch.randn(rows, Hkv, D, generator=g).to(torch.bfloat16)
            out = a(q.to(dev).view(rows, -1), k.to(dev).view(rows, -1), v.to(dev).view(rows, -1))
            torch.cuda.synchronize()
            want, _ = oatt.mixed_step(to_np(q), to_np(k), to_np(v), desc, ref[li, 0], ref[li, 1], slots,
                                      D ** -0.5, dtype=np.float32)
            assert_attn_close(out.view(rows, Hq, D), want, f"layer {li} step {step}")
            for kv in range(2):
                assert np.array_equal(bits(cache[kv, li]).reshape(-1, Hkv * D),
                                      f32_to_bf16_bits(ref[li, kv]).reshape(-1, Hkv * D)), (li, kv, step)
        reset_context()
        seq.advance()
    del cache
    torch.cuda.empty_cache()
