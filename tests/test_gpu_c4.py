"""The head-sparse C4 workload (LLaDA-8B shape: 32 heads x 128, B = 4 prompts of
1024 tokens, gen 256, block 64, retention 0.5, head_select, pool 3, delay 1)
at full size against the oracle, and a step mixing SparseConfigs.

- The dense full step (4 x 1280 tokens) of the varlen kernel vs the fp32
  oracle.
- Steps 0-2 of the first generation block through Attention.forward: step 0
  full attention, step 1 full attention + selection and store of 608 rows per
  KV head into each sequence's pages, step 2 the 64 block rows against the
  cached rows.  Outputs within max-abs 2e-2 / mean-abs 2e-3 of the fp32 oracle
  (oracle.attention.mixed_step), the whole cache bit-exact after every step.
- One step whose state-1 sequences use head_select True / False and pool
  1 / 3 / 5, next to a dense sequence, through Attention.forward.
- A Dream-shaped batch (28 query / 4 KV heads, 16 ragged sequences, block
  32): its reuse step runs the paired-row-block launch, once with every
  sequence cached (no id table) and once next to a dense sequence."""
import numpy as np
import pytest
import torch

from helpers import assert_attn_close, bits, to_np
from oracle.bf16 import f32_to_bf16_bits

from oracle import attention as oatt
from oracle import configs
from dllm_serve_amd import _capi
from dllm_serve_amd.engine.sequence import PageAllocator, Sequence, prepare_step, slot_mapping_for
from dllm_serve_amd.layers.attention import Attention
from dllm_serve_amd.sparse.state import SparseConfig, keep_count
from dllm_serve_amd.utils.context import reset_context

pytestmark = pytest.mark.gpu

MASK = 126336
D = 128


def test_c4_dense_full_step(dev):
    print("C4 dense full step: 4 x 1280 tokens, 32 heads", flush=True)
    lens = [1280] * 4
    q, k, v, cu = configs.packed_qkv(lens, 32, 32, D, seed=41)
    o = torch.full(q.shape, float("nan"), dtype=torch.bfloat16, device=dev)
    cud = cu.to(dev)
    _capi.attn_varlen_fwd(q.to(dev), k.to(dev), v.to(dev), o, cud, cud, None, 4, 1280, D ** -0.5)
    torch.cuda.synchronize()
    ref = oatt.varlen(to_np(q), to_np(k), to_np(v), cu.numpy(), cu.numpy(), D ** -0.5, dtype=np.float32)
    assert_attn_close(o, ref, "C4 4 x 1280")


def _run_steps(dev, seqs, attn, cache, n_steps, descs_for, seed):
    """Runs n_steps forwards; descs_for(step) gives the oracle's per-sequence
    description.  The whole cache is compared bit for bit after each step."""
    Hq, Hkv = attn.num_heads, attn.num_kv_heads
    scale = attn.scale
    ref_cache = np.zeros((2, cache.shape[1] * cache.shape[2], Hkv, D), dtype=np.float32)
    g = torch.Generator().manual_seed(seed)
    for step in range(n_steps):
        prepare_step(seqs, dev)
        desc, slots = descs_for(step)
        n = sum(d["rows"] for d in desc)
        q = torch.randn(n, Hq, D, generator=g).to(torch.bfloat16)
        k = torch.randn(n, Hkv, D, generator=g).to(torch.bfloat16)
        v = torch.randn(n, Hkv, D, generator=g).to(torch.bfloat16)
        print(f"  step {step}: {n} rows, modes {[d['mode'] for d in desc]}", flush=True)
        out = attn(q.to(dev).view(n, Hq * D), k.to(dev).view(n, Hkv * D), v.to(dev).view(n, Hkv * D))
        torch.cuda.synchronize()
        ref, _ = oatt.mixed_step(to_np(q), to_np(k), to_np(v), desc, ref_cache[0], ref_cache[1], slots, scale,
                                 dtype=np.float32)
        assert_attn_close(out.view(n, Hq, D), ref, f"step {step}")
        assert np.array_equal(bits(cache[0]).reshape(-1, Hkv * D),
                              f32_to_bf16_bits(ref_cache[0]).reshape(-1, Hkv * D)), f"k cache after step {step}"
        assert np.array_equal(bits(cache[1]).reshape(-1, Hkv * D),
                              f32_to_bf16_bits(ref_cache[1]).reshape(-1, Hkv * D)), f"v cache after step {step}"
        reset_context()
        for s in seqs:
            s.advance()


def test_c4_block_steps_through_the_layer(dev):
    print("C4 block: B=4, P=1024, gen 256, block 64, steps 0-2 through Attention.forward", flush=True)
    Hq = Hkv = 32
    attn = Attention(Hq, D, D ** -0.5, Hkv, causal=False)
    cfg = SparseConfig(enabled=True, default_block_len=64, retention_ratio=0.5, pool_kernel=3, delay_step=1,
                       head_select=True)
    seqs = [Sequence([1] * 1024, 256, MASK, cfg, device=dev, steps=256) for _ in range(4)]
    n_pages = sum(s.num_blocks for s in seqs) + 2
    alloc = PageAllocator(torch.randperm(n_pages, generator=torch.Generator().manual_seed(8)).tolist())
    for s in seqs:
        alloc.allocate(s)
    cache = torch.zeros(2, n_pages, 256, Hkv, D, dtype=torch.bfloat16, device=dev)
    attn.k_cache, attn.v_cache = cache[0], cache[1]
    n_keep = keep_count(1280 - 64, 0.5)
    assert n_keep == 608

    def descs(step):
        if step == 0:
            return [dict(mode=0, rows=1280)] * 4, [[]] * 4
        slots = [slot_mapping_for(s) for s in seqs]
        assert all(len(x) == n_keep for x in slots)
        if step == 1:
            return [dict(mode=1, rows=1280, blk_start=1024, blk_len=64, n_keep=n_keep, head_select=True, pool_k=3)
                    ] * 4, slots
        return [dict(mode=2, rows=64)] * 4, slots

    _run_steps(dev, seqs, attn, cache, 3, descs, seed=1024)


def test_step_mixing_sparse_configs_through_the_layer(dev):
    """State-1 sequences with head_select True / False and pool 1 / 3 / 5 in
    one step, next to a dense sequence; then their state-2 step."""
    print("layer: one step mixing head_select / pool_kernel", flush=True)
    Hq, Hkv = 16, 4
    attn = Attention(Hq, D, D ** -0.5, Hkv, causal=False)
    cfgs = [SparseConfig(enabled=True, default_block_len=32, retention_ratio=0.5, pool_kernel=1, head_select=True),
            SparseConfig(enabled=True, default_block_len=32, retention_ratio=0.3, pool_kernel=3, head_select=False),
            SparseConfig(enabled=True, default_block_len=32, retention_ratio=0.75, pool_kernel=5, head_select=True)]
    prompts = [300, 180, 420]
    seqs = [Sequence([i + 1] * p, 64, MASK, c, device=dev) for i, (p, c) in enumerate(zip(prompts, cfgs))]
    seqs.append(Sequence([9] * 90, 64, MASK, None, device=dev))
    n_pages = sum(s.num_blocks for s in seqs[:3]) + 1
    alloc = PageAllocator(list(range(n_pages))[::-1])
    for s in seqs[:3]:
        alloc.allocate(s)
    cache = torch.zeros(2, n_pages, 256, Hkv, D, dtype=torch.bfloat16, device=dev)
    attn.k_cache, attn.v_cache = cache[0], cache[1]

    def descs(step):
        N = [p + 64 for p in prompts]
        if step == 0:
            return [dict(mode=0, rows=n) for n in N] + [dict(mode=0, rows=154)], [[]] * 4
        slots = [slot_mapping_for(s) for s in seqs[:3]] + [[]]
        if step == 1:
            d = [dict(mode=1, rows=n, blk_start=p, blk_len=32, n_keep=keep_count(n - 32, c.retention_ratio),
                      head_select=c.head_select, pool_k=c.pool_kernel) for n, p, c in zip(N, prompts, cfgs)]
            return d + [dict(mode=0, rows=154)], slots
        return [dict(mode=2, rows=32)] * 3 + [dict(mode=0, rows=154)], slots

    _run_steps(dev, seqs, attn, cache, 3, descs, seed=77)


@pytest.mark.parametrize("with_dense", [False, True])
def test_dream_batch_paired_row_blocks_through_the_layer(dev, with_dense):
    print(f"Dream batch: 16 ragged sequences, 28/4 heads, block 32, dense neighbour {with_dense}", flush=True)
    Hq, Hkv = 28, 4
    attn = Attention(Hq, D, D ** -0.5, Hkv, causal=False)
    cfg = SparseConfig(enabled=True, default_block_len=32, retention_ratio=0.5, pool_kernel=3, delay_step=1,
                       head_select=True)
    prompts = [200 + (i * 53) % 300 for i in range(16)]
    seqs = [Sequence([i + 1] * p, 64, MASK, cfg, device=dev) for i, p in enumerate(prompts)]
    if with_dense:
        seqs.append(Sequence([99] * 120, 32, MASK, None, device=dev))
    n_pages = sum(s.num_blocks for s in seqs[:16]) + 1
    alloc = PageAllocator(torch.randperm(n_pages, generator=torch.Generator().manual_seed(5)).tolist())
    for s in seqs[:16]:
        alloc.allocate(s)
    cache = torch.zeros(2, n_pages, 256, Hkv, D, dtype=torch.bfloat16, device=dev)
    attn.k_cache, attn.v_cache = cache[0], cache[1]
    N = [p + 64 for p in prompts]
    # 16 x 4 KV heads x 7 M tiles: more than one generation of single-block workgroups
    assert 16 * Hkv * (32 * (Hq // Hkv) // 32) > 256
    dense = [dict(mode=0, rows=152)] if with_dense else []

    def descs(step):
        if step == 0:
            return [dict(mode=0, rows=n) for n in N] + dense, [[]] * len(seqs)
        slots = [slot_mapping_for(s) for s in seqs[:16]] + ([[]] if with_dense else [])
        if step == 1:
            return [dict(mode=1, rows=n, blk_start=p, blk_len=32, n_keep=keep_count(n - 32, 0.5), head_select=True,
                         pool_k=3) for n, p in zip(N, prompts)] + dense, slots
        return [dict(mode=2, rows=32)] * 16 + dense, slots

    _run_steps(dev, seqs, attn, cache, 3, descs, seed=33 + int(with_dense))
