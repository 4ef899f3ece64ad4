"""Seeded synthetic inputs of the benchmark configurations (CPU tensors).

One torch.Generator per configuration, seeded with 0, draws in the order
listed in each function.  Shapes follow the LLaDA-8B (32 heads x 128) and
Dream-7B (28 query / 4 KV heads x 128) attention layers.
"""
from __future__ import annotations

import math

import torch

LLADA = dict(Hq=32, Hkv=32, D=128, theta=500000.0)
DREAM = dict(Hq=28, Hkv=4, D=128, theta=1000000.0)


def rope_torch(x: torch.Tensor, positions: torch.Tensor, base: float) -> torch.Tensor:
    """NeoX RoPE as dllmserve/layers/rotary_embedding.py:6-57 computes it (f32)."""
    D = x.shape[-1]
    inv_freq = 1.0 / (base ** (torch.arange(0, D, 2, dtype=torch.float) / D))
    freqs = torch.einsum("i,j -> ij", positions.to(torch.float), inv_freq)
    cos, sin = freqs.cos().unsqueeze(-2), freqs.sin().unsqueeze(-2)
    x1, x2 = torch.chunk(x.to(torch.float32), 2, dim=-1)
    return torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), dim=-1).to(x.dtype)


def c1_single_layer(n: int = 512, seed: int = 0):
    """C1: one LLaDA-8B attention layer, one sequence of n=512 tokens, fp32.
    Q, K, V ~ N(0,1) (drawn in that order), RoPE theta 5e5 on Q and K at
    positions 0..n-1.  Returns q, k, v [n, 32, 128] f32, cu, scale."""
    g = torch.Generator().manual_seed(seed)
    H, D = LLADA["Hq"], LLADA["D"]
    q = torch.randn(n, H, D, generator=g)
    k = torch.randn(n, H, D, generator=g)
    v = torch.randn(n, H, D, generator=g)
    pos = torch.arange(n)
    q = rope_torch(q, pos, LLADA["theta"])
    k = rope_torch(k, pos, LLADA["theta"])
    return q, k, v, torch.tensor([0, n], dtype=torch.int32), D ** -0.5


def packed_qkv(lens, Hq, Hkv, D, seed=0, dtype=torch.bfloat16):
    """Packed q [sum(lens), Hq, D], k/v [sum(lens), Hkv, D] ~ N(0,1), cu."""
    g = torch.Generator().manual_seed(seed)
    n = int(sum(lens))
    q = torch.randn(n, Hq, D, generator=g).to(dtype)
    k = torch.randn(n, Hkv, D, generator=g).to(dtype)
    v = torch.randn(n, Hkv, D, generator=g).to(dtype)
    cu = torch.zeros(len(lens) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(lens, dtype=torch.int32), 0)
    return q, k, v, cu


def c2_dense_lens(batch=8, prompt=256, gen=128):
    """C2 dense step: every sequence feeds prompt+gen rows (LLaDA shape)."""
    return [prompt + gen] * batch


def c3_lens(n_seq=16, lo=128, hi=1024, gen=256, seed=0):
    """C3: prompt lengths ~ U{lo..hi} (drawn first from seed), + gen rows."""
    g = torch.Generator().manual_seed(seed)
    p = torch.randint(lo, hi + 1, (n_seq,), generator=g)
    return [int(x) + gen for x in p]


def c5_cached(batch=32, lo=2048, hi=4096, blk=32, page=256, seed=0, Hkv=32, D=128, Hq=32):
    """C5: prefix lengths ~ U{lo..hi}; pages from a seeded shuffled free list;
    cached prefix K/V and block q/k/v ~ N(0,1) bf16.  Returns a dict with
    prefix lengths, per-sequence slot lists, page count, block q/k/v and the
    prefix K/V rows (to be written to the cache with store_kvcache)."""
    g = torch.Generator().manual_seed(seed)
    prefix = [int(x) for x in torch.randint(lo, hi + 1, (batch,), generator=g)]
    pages_per = [math.ceil(p / page) for p in prefix]
    num_pages = sum(pages_per)
    free = torch.randperm(num_pages, generator=g).tolist()
    slots, at = [], 0
    for p, npg in zip(prefix, pages_per):
        pg = free[at:at + npg]
        at += npg
        s = []
        for j, pid in enumerate(pg):
            fill = page if j < npg - 1 else p - page * (npg - 1)
            s.extend(range(pid * page, pid * page + fill))
        slots.append(s)
    total_prefix = sum(prefix)
    k_pre = torch.randn(total_prefix, Hkv, D, generator=g).to(torch.bfloat16)
    v_pre = torch.randn(total_prefix, Hkv, D, generator=g).to(torch.bfloat16)
    q = torch.randn(batch * blk, Hq, D, generator=g).to(torch.bfloat16)
    k = torch.randn(batch * blk, Hkv, D, generator=g).to(torch.bfloat16)
    v = torch.randn(batch * blk, Hkv, D, generator=g).to(torch.bfloat16)
    return dict(prefix=prefix, slots=slots, num_pages=num_pages, page=page, k_pre=k_pre, v_pre=v_pre,
                q=q, k=k, v=v, blk=blk)


def attention_flops(seg_q, seg_k, Hq, D) -> float:
    """4 * sum Lq*Lk*Hq*D (QK^T and PV multiply-adds, softmax not counted)."""
    return float(sum(4.0 * a * b * Hq * D for a, b in zip(seg_q, seg_k)))


def attention_bytes(seg_q, seg_k, Hq, Hkv, D, elem=2) -> float:
    """Minimum HBM bytes: read Q and K/V once, write O once."""
    return float(sum(elem * (2 * a * Hq * D + 2 * b * Hkv * D) for a, b in zip(seg_q, seg_k)))
