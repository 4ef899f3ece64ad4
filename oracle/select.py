"""Sparse KV selection (mode 1) with a defined rounding and tie-break rule.

Follows dllmserve/layers/attention.py:344-413 (_select_important_head_kv,
head_select=True) and attention.py:308-342 (_select_important_kv,
head_select=False).  The reference computes the scores with bf16 torch ops
(mean -> bf16, einsum -> bf16, division by sqrt(D) -> bf16, max over the GQA
group, max_pool1d, topk); its accumulation order and topk tie order are
those of the device libraries and are not specified.  The build fixes them:

  qbar[h,d]   = bf16( f32( (sum_t q[t,h,d]) / Lb ) ), sum in f64, t ascending
  dot[h,j]    = sum_d qbar[h,d] * k[j, h//g, d]   in f64, d ascending
  raw[h,j]    = bf16( f32( dot[h,j] ) )                       (head_select=True)
  raw[j]      = bf16( f32( sum_kv ( sum_{h in group kv} dot[h,j] ) ) )
                f64, groups kv ascending, heads ascending inside a group
                (head_select=False)
  score[kv,j] = bf16( f32(max_{h in group kv} raw[h,j]) / f32(sqrt(D)) )
  pooled[j]   = max score over [j - p//2, j - p//2 + p - 1] within [0, Kc)
                (p = pool_kernel; none when p <= 1)
  top n_keep by pooled descending, ties to the lower candidate index.

Rounded division by a positive constant is monotone, so taking the group
max and the pool max before or after it gives the same value; the order
above is the reference's order up to that identity.  Products of two bf16
values are exact in f64, so the sums depend only on the fixed order.
"""
from __future__ import annotations

import numpy as np

from .bf16 import bf16_bits_to_f32, f32_to_bf16_bits, f64_to_bf16_bits


def qbar(q_blk: np.ndarray) -> np.ndarray:
    """q_blk [Lb, Hq, D] (bf16 values) -> [Hq, D] bf16 values (as f32)."""
    Lb = q_blk.shape[0]
    acc = np.zeros(q_blk.shape[1:], dtype=np.float64)
    for t in range(Lb):
        acc = acc + q_blk[t].astype(np.float64)
    return bf16_bits_to_f32(f64_to_bf16_bits(acc / np.float64(Lb)))


def dots(qb: np.ndarray, k_cand: np.ndarray) -> np.ndarray:
    """dot[h, j] = sum_d qb[h, d] * k_cand[j, h // g, d] in f64, d ascending
    ([Hq, Kc]).  Products of two bf16 values are exact in f64, so only the
    order of the additions is a choice."""
    Hq, D = qb.shape
    Kc, Hkv, _ = k_cand.shape
    g = Hq // Hkv
    q64 = qb.astype(np.float64)
    k64 = k_cand.astype(np.float64)
    out = np.empty((Hq, Kc), dtype=np.float64)
    for h in range(Hq):
        acc = np.zeros(Kc, dtype=np.float64)
        kh = k64[:, h // g, :]
        for d in range(D):
            acc = acc + q64[h, d] * kh[:, d]
        out[h] = acc
    return out


def raw_scores(qb: np.ndarray, k_cand: np.ndarray, head_select: bool) -> np.ndarray:
    """qb [Hq, D], k_cand [Kc, Hkv, D] -> head_select: [Hq, Kc]; else [Kc]
    (bf16 values as f32) before the division by sqrt(D)."""
    Hq = qb.shape[0]
    Kc, Hkv, _ = k_cand.shape
    g = Hq // Hkv
    dt = dots(qb, k_cand)
    if head_select:
        return bf16_bits_to_f32(f64_to_bf16_bits(dt)).reshape(Hq, Kc)
    total = np.zeros(Kc, dtype=np.float64)
    for kv in range(Hkv):
        part = np.zeros(Kc, dtype=np.float64)
        for gi in range(g):
            part = part + dt[kv * g + gi]
        total = total + part
    return bf16_bits_to_f32(f64_to_bf16_bits(total))


def pool(s: np.ndarray, pool_k: int) -> np.ndarray:
    """max_pool1d(kernel=pool_k, stride=1, padding=pool_k//2)[..., :Kc] with
    -inf padding, along the last axis."""
    if pool_k <= 1 or s.shape[-1] == 0:
        return s
    Kc = s.shape[-1]
    p = pool_k // 2
    padded = np.concatenate(
        [np.full(s.shape[:-1] + (p,), -np.inf, np.float32), s,
         np.full(s.shape[:-1] + (pool_k,), -np.inf, np.float32)], axis=-1)
    out = np.full(s.shape, -np.inf, dtype=np.float32)
    for w in range(pool_k):
        out = np.maximum(out, padded[..., w:w + Kc])
    return out


def scale_scores(raw: np.ndarray, sqrt_d) -> np.ndarray:
    """bf16(f32(raw) / f32(sqrt_d)) elementwise (IEEE f32 division)."""
    q = (raw.astype(np.float32) / np.float32(sqrt_d)).astype(np.float32)
    return bf16_bits_to_f32(f32_to_bf16_bits(q))


def topk_desc(s: np.ndarray, n_keep: int) -> np.ndarray:
    """Indices of the n_keep largest entries of each row of s, descending,
    ties to the lower index (-0.0 equals +0.0)."""
    s = np.where(s == 0, np.float32(0), s)
    idx = np.arange(s.shape[-1])
    order = np.lexsort((np.broadcast_to(idx, s.shape), -s), axis=-1)
    return order[..., :n_keep].astype(np.int64)


def select(q_blk: np.ndarray, k_cand: np.ndarray, n_keep: int, head_select: bool, pool_k: int,
           sqrt_d) -> np.ndarray:
    """Selected candidate indices: head_select -> [Hkv, n_keep]; else [n_keep]."""
    Kc, Hkv, _ = k_cand.shape
    Hq = q_blk.shape[1]
    if Kc == 0:
        return np.zeros((Hkv, 0) if head_select else (0,), dtype=np.int64)
    qb = qbar(q_blk)
    raw = raw_scores(qb, k_cand, head_select)
    if head_select:
        g = Hq // Hkv
        raw = raw.reshape(Hkv, g, Kc).max(axis=1)
    s = pool(scale_scores(raw, sqrt_d), pool_k)
    return topk_desc(s, n_keep)
