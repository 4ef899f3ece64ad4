"""Attention.forward end to end (Context + SparseConfig state machine + all
kernels) over three denoising steps of a mixed batch, vs the oracle.

Batch: A dense (no SparseConfig), B and C sparse (head_select, block 32,
delay_step 1).  Step 0: all full attention.  Step 1: B and C select and
store their KV (cache state 1).  Step 2: B and C attend from their block to
the cache (state 2).  Outputs within the bf16 tolerance, cache bit-exact."""
import numpy as np
import pytest
import torch

from helpers import assert_attn_close, bits, to_np
from oracle.bf16 import f32_to_bf16_bits

from oracle import attention as oatt
from dllm_serve_amd.engine.sequence import PageAllocator, Sequence, prepare_step, slot_mapping_for
from dllm_serve_amd.layers.attention import Attention
from dllm_serve_amd.sparse.state import SparseConfig
from dllm_serve_amd.utils.context import get_context, reset_context

pytestmark = pytest.mark.gpu

MASK = 126336


@pytest.mark.parametrize("Hq,Hkv", [(32, 32), (28, 4)])
def test_three_steps_mixed_batch(dev, Hq, Hkv):
    print(f"layer three steps Hq={Hq} Hkv={Hkv}", flush=True)
    D = 128
    scale = D ** -0.5
    attn = Attention(Hq, D, scale, Hkv, causal=False)
    n_pages = 8
    cache = torch.zeros(2, n_pages, 256, Hkv, D, dtype=torch.bfloat16, device=dev)
    attn.k_cache, attn.v_cache = cache[0], cache[1]
    ref_cache = np.zeros((2, n_pages * 256, Hkv * D), dtype=np.float32)

    cfg_b = SparseConfig(enabled=True, default_block_len=32, retention_ratio=0.5, pool_kernel=3,
                         delay_step=1, head_select=True)
    cfg_c = SparseConfig(enabled=True, default_block_len=32, retention_ratio=0.25, pool_kernel=3,
                         delay_step=1, head_select=True)
    A = Sequence([1] * 100, 64, MASK, None, device=dev)
    B = Sequence([2] * 200, 64, MASK, cfg_b, device=dev)
    C = Sequence([3] * 150, 64, MASK, cfg_c, device=dev)
    seqs = [A, B, C]
    alloc = PageAllocator([5, 2, 7, 0, 3, 6, 1, 4])
    for s in (B, C):
        alloc.allocate(s)
    assert B.block_table == [5] and C.block_table == [2]

    # Literal schedule (P = 100/200/150, gen 64, block 32):
    #   B: block rows [200, 232), Kc 232, n_keep int(232*0.5) = 116
    #   C: block rows [150, 182), Kc 182, n_keep int(182*0.25) = 45
    plan_rows = {0: [164, 264, 214], 1: [164, 264, 214], 2: [164, 32, 32]}
    g = torch.Generator().manual_seed(2024)
    for step in range(3):
        prepare_step(seqs, dev)
        ctx = get_context()
        n = sum(plan_rows[step])
        q = torch.randn(n, Hq, D, generator=g).to(torch.bfloat16)
        k = torch.randn(n, Hkv, D, generator=g).to(torch.bfloat16)
        v = torch.randn(n, Hkv, D, generator=g).to(torch.bfloat16)
        out = attn(q.to(dev).view(n, Hq * D), k.to(dev).view(n, Hkv * D), v.to(dev).view(n, Hkv * D))
        torch.cuda.synchronize()
        assert out.shape == (n, Hq * D)

        if step == 0:
            desc = [dict(mode=0, rows=r) for r in plan_rows[0]]
            slots = [[], [], []]
        elif step == 1:
            desc = [dict(mode=0, rows=164),
                    dict(mode=1, rows=264, blk_start=200, blk_len=32, n_keep=116, head_select=True, pool_k=3),
                    dict(mode=1, rows=214, blk_start=150, blk_len=32, n_keep=45, head_select=True, pool_k=3)]
            slots = [[], list(range(5 * 256, 5 * 256 + 116)), list(range(2 * 256, 2 * 256 + 45))]
        else:
            desc = [dict(mode=0, rows=164), dict(mode=2, rows=32), dict(mode=2, rows=32)]
            slots = [[], list(range(5 * 256, 5 * 256 + 116)), list(range(2 * 256, 2 * 256 + 45))]
        if step > 0:
            assert slot_mapping_for(B) == slots[1] and slot_mapping_for(C) == slots[2]
        ref, _ = oatt.mixed_step(to_np(q), to_np(k), to_np(v), desc,
                                 ref_cache[0].reshape(-1, Hkv, D), ref_cache[1].reshape(-1, Hkv, D),
                                 slots, scale, dtype=np.float32)
        assert_attn_close(out.view(n, Hq, D), ref, f"step {step}")
        kc_bits = bits(cache[0]).reshape(-1, Hkv * D)
        assert np.array_equal(kc_bits, f32_to_bf16_bits(ref_cache[0])), f"k cache differs after step {step}"
        assert np.array_equal(bits(cache[1]).reshape(-1, Hkv * D), f32_to_bf16_bits(ref_cache[1]))
        reset_context()
        for s in seqs:
            s.advance()
