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
