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


def test_dream_reference_batch_three_steps(dev):
    """The batch of the reference's Dream sparse test
    (tests/unit/test_dream_sparse.py:49): [dense, SparseConfig(enabled=True,
    retention_ratio=0.5, default_block_len=16), dense] -- token selection
    (head_select False, the SparseConfig default), pool 3, delay 1 -- at
    Dream-7B's 28 query / 4 KV heads, gen 64.  Step 0 all full attention,
    step 1 the middle sequence selects and stores (cache state 1), step 2 it
    attends from its 16-token block to the cache (state 2).  Outputs within
    the bf16 tolerance of the fp32 oracle, the cache bit-exact."""
    Hq, Hkv, D = 28, 4, 128
    print("layer: Dream reference batch [None, SparseConfig(0.5, block 16), None], three steps", flush=True)
    scale = D ** -0.5
    attn = Attention(Hq, D, scale, Hkv, causal=False)
    n_pages = 4
    cache = torch.zeros(2, n_pages, 256, Hkv, D, dtype=torch.bfloat16, device=dev)
    attn.k_cache, attn.v_cache = cache[0], cache[1]
    ref_cache = np.zeros((2, n_pages * 256, Hkv * D), dtype=np.float32)
    cfg = SparseConfig(enabled=True, retention_ratio=0.5, default_block_len=16)
    assert cfg.head_select is False and cfg.pool_kernel == 3 and cfg.delay_step == 1
    P = [57, 130, 96]
    seqs = [Sequence([5] * P[0], 64, MASK, None, device=dev), Sequence([6] * P[1], 64, MASK, cfg, device=dev),
            Sequence([7] * P[2], 64, MASK, None, device=dev)]
    PageAllocator([3, 1, 0, 2]).allocate(seqs[1])
    N = [p + 64 for p in P]
    n_keep = int((N[1] - 16) * 0.5)   # candidates: every row but the 16-token block
    slots = list(range(3 * 256, 3 * 256 + 89))
    rows = {0: N, 1: N, 2: [N[0], 16, N[2]]}
    g = torch.Generator().manual_seed(49)
    for step in range(3):
        prepare_step(seqs, dev)
        if step > 0:  # slot lists exist in cache states 1 and 2 (the reference raises otherwise)
            assert n_keep == 89 and slot_mapping_for(seqs[1]) == slots
        n = sum(rows[step])
        q = torch.randn(n, Hq, D, generator=g).to(torch.bfloat16)
        k = torch.randn(n, Hkv, D, generator=g).to(torch.bfloat16)
        v = torch.randn(n, Hkv, D, generator=g).to(torch.bfloat16)
        out = attn(q.to(dev), k.to(dev), v.to(dev))
        torch.cuda.synchronize()
        mid = (dict(mode=0, rows=N[1]) if step == 0 else
               dict(mode=1, rows=N[1], blk_start=P[1], blk_len=16, n_keep=n_keep, head_select=False, pool_k=3)
               if step == 1 else dict(mode=2, rows=16))
        desc = [dict(mode=0, rows=N[0]), mid, dict(mode=0, rows=N[2])]
        ref, _ = oatt.mixed_step(to_np(q), to_np(k), to_np(v), desc,
                                 ref_cache[0].reshape(-1, Hkv, D), ref_cache[1].reshape(-1, Hkv, D),
                                 [[], slots, []], scale, dtype=np.float32)
        assert_attn_close(out.view(n, Hq, D), ref, f"Dream reference batch, step {step}")
        assert np.array_equal(bits(cache[0]).reshape(-1, Hkv * D), f32_to_bf16_bits(ref_cache[0]))
        assert np.array_equal(bits(cache[1]).reshape(-1, Hkv * D), f32_to_bf16_bits(ref_cache[1]))
        reset_context()
        for s in seqs:
            s.advance()
