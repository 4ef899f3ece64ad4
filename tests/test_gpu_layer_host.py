"""The layer's host path: q/k/v layouts it takes without a view, the stream it
launches on, and the re-check of a rebound cache.

One reuse step (cache state 2) of two sparse sequences next to a dense one,
as in test_gpu_layer: the outputs of 2-D inputs, 3-D inputs, row-strided
slices of one fused qkv buffer and a call on a side stream are bit-identical."""
import pytest
import torch

from dllm_serve_amd import _capi
from dllm_serve_amd.engine.sequence import PageAllocator, Sequence, prepare_step
from dllm_serve_amd.layers.attention import Attention
from dllm_serve_amd.sparse.state import SparseConfig
from dllm_serve_amd.utils.context import get_context, reset_context

pytestmark = pytest.mark.gpu

MASK = 126336


def _reuse_step(dev, Hq, Hkv, D):
    attn = Attention(Hq, D, D ** -0.5, Hkv, causal=False)
    cache = torch.randn(2, 8, 256, Hkv, D, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).to(dev)
    attn.k_cache, attn.v_cache = cache[0], cache[1]
    cfg = SparseConfig(enabled=True, default_block_len=32, retention_ratio=0.5, pool_kernel=3, delay_step=1,
                       head_select=True)
    seqs = [Sequence([1] * 100, 64, MASK, None, device=dev), Sequence([2] * 200, 64, MASK, cfg, device=dev),
            Sequence([3] * 150, 64, MASK, cfg, device=dev)]
    alloc = PageAllocator(range(8))
    for s in seqs[1:]:
        alloc.allocate(s)
    for _ in range(2):  # steps 0 and 1 only advance the state machine here
        prepare_step(seqs, dev)
        reset_context()
        for s in seqs:
            s.advance()
    prepare_step(seqs, dev)
    assert get_context().is_diffusion
    return attn, cache


def test_layouts_and_side_stream(dev):
    print("layer host path: layouts and streams", flush=True)
    Hq, Hkv, D = 32, 8, 128
    try:
        attn, _ = _reuse_step(dev, Hq, Hkv, D)
        n = 164 + 32 + 32
        g = torch.Generator().manual_seed(11)
        qkv = torch.randn(n, (Hq + 2 * Hkv) * D, generator=g).to(torch.bfloat16).to(dev)
        q2, k2, v2 = (t.contiguous() for t in qkv.split([Hq * D, Hkv * D, Hkv * D], dim=1))
        base = attn(q2, k2, v2)
        assert base.shape == (n, Hq * D)
        out3 = attn(q2.view(n, Hq, D), k2.view(n, Hkv, D), v2.view(n, Hkv, D))
        qs, ks, vs = qkv.split([Hq * D, Hkv * D, Hkv * D], dim=1)  # row stride (Hq + 2 Hkv) D
        assert qs.stride(0) == (Hq + 2 * Hkv) * D
        out_s = attn(qs, ks, vs)
        out_flat = attn(q2.reshape(-1), k2.reshape(-1), v2.reshape(-1))  # through the reference's view
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            assert _capi._stream(dev) == side.cuda_stream
            out_side = attn(q2, k2, v2)
        torch.cuda.current_stream(dev).wait_stream(side)
        assert _capi._stream(dev) == torch.cuda.current_stream(dev).cuda_stream
        torch.cuda.synchronize()
        for name, o in (("3-D", out3), ("strided", out_s), ("flat", out_flat), ("side stream", out_side)):
            assert o.shape == (n, Hq * D), name
            assert torch.equal(o.view(torch.int16), base.view(torch.int16)), name
        with pytest.raises(ValueError):  # heads not contiguous
            attn(q2.view(n, Hq, D).transpose(1, 2).contiguous().transpose(1, 2), k2, v2)
    finally:
        reset_context()


def test_rebound_cache_is_checked_again(dev):
    print("layer host path: rebound cache", flush=True)
    Hq, Hkv, D = 32, 8, 128
    try:
        attn, cache = _reuse_step(dev, Hq, Hkv, D)
        n = 164 + 32 + 32
        q = torch.randn(n, Hq * D, device=dev).to(torch.bfloat16)
        k = torch.randn(n, Hkv * D, device=dev).to(torch.bfloat16)
        attn(q, k, k)
        attn.k_cache = cache[0].float()  # same layer, a cache the kernels cannot use
        with pytest.raises(ValueError, match="k_cache"):
            attn(q, k, k)
        attn.k_cache = cache[0]
        attn.v_cache = cache[1][:, :, : Hkv // 2]  # wrong head count
        with pytest.raises(ValueError, match="v_cache"):
            attn(q, k, k)
        attn.v_cache = cache[1]
        attn(q, k, k)
        torch.cuda.synchronize()
    finally:
        reset_context()


def test_layers_of_two_head_shapes_share_one_step(dev):
    """Two Attention layers of different head shapes in one context, the
    smaller first.  Each layer's K3b launch splits its keys and so needs the
    step's partial-record workspace; the larger shape asks for more bytes.
    The smaller layer's workspace must stay its own when the larger one
    allocates: buffers of the smaller workspace's size allocated in between
    (the caching allocator hands freed blocks out again) keep their sentinel
    through the smaller layer's next call, and every output matches the
    oracle, over two reuse steps."""
    import numpy as np

    from helpers import assert_attn_close, to_np
    from oracle import attention as oatt
    from dllm_serve_amd.engine.sequence import slot_mapping_for

    print("layer host path: two head shapes in one step", flush=True)
    D = 128
    shapes = [(8, 2), (32, 8)]  # (Hq, Hkv), the smaller workspace first
    n_pages = 16
    gen = torch.Generator().manual_seed(21)
    layers, caches = [], []
    for Hq, Hkv in shapes:
        attn = Attention(Hq, D, D ** -0.5, Hkv, causal=False)
        cache = torch.randn(2, n_pages, 256, Hkv, D, generator=gen).to(torch.bfloat16).to(dev)
        attn.k_cache, attn.v_cache = cache[0], cache[1]
        layers.append(attn)
        caches.append(cache)
    cfg = SparseConfig(enabled=True, default_block_len=32, retention_ratio=0.5, pool_kernel=3, delay_step=1,
                       head_select=True)
    seqs = [Sequence([2] * 2000, 64, MASK, cfg, device=dev), Sequence([3] * 1800, 64, MASK, cfg, device=dev)]
    alloc = PageAllocator(range(n_pages))
    for s in seqs:
        alloc.allocate(s)
    try:
        for _ in range(2):  # steps 0 and 1 only advance the state machine here
            prepare_step(seqs, dev)
            reset_context()
            for s in seqs:
                s.advance()
        slot_lists = [slot_mapping_for(s) for s in seqs]
        assert [len(x) for x in slot_lists] == [1016, 916]
        for step in range(2):
            prepare_step(seqs, dev)
            n = 64
            ins = []
            for Hq, Hkv in shapes:
                q = torch.randn(n, Hq, D, generator=gen).to(torch.bfloat16)
                k = torch.randn(n, Hkv, D, generator=gen).to(torch.bfloat16)
                v = torch.randn(n, Hkv, D, generator=gen).to(torch.bfloat16)
                ins.append((q, k, v, q.to(dev), k.to(dev), v.to(dev)))
            ws_small = _capi.block_cached_workspace_size(2, 32, 32 + 1016, 8, 2, D)
            ws_large = _capi.block_cached_workspace_size(2, 32, 32 + 1016, 32, 8, D)
            assert 0 < ws_small < ws_large, (ws_small, ws_large)
            outs = [layers[0](*ins[0][3:]), layers[1](*ins[1][3:])]
            plan = get_context()._dllm_plan  # built by the first layer call of the step
            sentinels = [torch.full((ws_small,), 0x5A, dtype=torch.uint8, device=dev) for _ in range(4)]
            outs.append(layers[0](*ins[0][3:]))
            torch.cuda.synchronize()
            for t in sentinels:
                assert bool((t == 0x5A).all()), "a freed workspace was written after the allocator handed it out"
            assert plan.launch_args(8, 2, D)["ws_tensor"] is not None
            for li, out in zip((0, 1, 0), outs):
                Hq, Hkv = shapes[li]
                q, k, v = ins[li][:3]
                kc = to_np(caches[li][0]).reshape(-1, Hkv, D)
                vc = to_np(caches[li][1]).reshape(-1, Hkv, D)
                ref = np.concatenate([
                    oatt.block_cached(to_np(q[32 * i:32 * i + 32]), to_np(k[32 * i:32 * i + 32]),
                                      to_np(v[32 * i:32 * i + 32]), kc, vc, slot_lists[i], D ** -0.5,
                                      dtype=np.float32) for i in range(2)])
                assert_attn_close(out.view(n, Hq, D), ref, f"step {step} layer shape {shapes[li]}")
            reset_context()
            for s in seqs:
                s.advance()
    finally:
        reset_context()
