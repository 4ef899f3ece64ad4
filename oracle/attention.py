"""Attention restated on numpy (fp32 or fp64 math).

varlen(...)      flash_attn_varlen_func(causal=False) as called at
                 dllmserve/layers/attention.py:289-299: per segment
                 O[t,h] = softmax_u(scale * q[t,h] . k[u, h//g]) @ v[u, h//g]
block_cached(...) the mode-2 branch, attention.py:235-265: block rows attend
                 to [cache rows (by slot) ; block rows]
mixed_step(...)  _mixed_sparse_dense_attention, attention.py:150-306, per
                 sequence mode 0 / 1 / 2 including the mode-1 selection and
                 cache store (select.py, kvcache.py)
"""
from __future__ import annotations

import numpy as np

from . import kvcache as _kv
from . import select as _sel


def segment(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float, dtype=np.float64) -> np.ndarray:
    """q [Lq,Hq,D], k/v [Lk,Hkv,D] -> o [Lq,Hq,D] (math in `dtype`).  With no
    keys the softmax is empty; the rows are zero (the C ABI's convention)."""
    Lq, Hq, D = q.shape
    Lk, Hkv, _ = k.shape
    if Lk == 0:
        return np.zeros((Lq, Hq, D), dtype=dtype)
    g = Hq // Hkv
    qd = q.astype(dtype)
    kd = np.repeat(k.astype(dtype), g, axis=1)  # head h reads KV head h // g
    vd = np.repeat(v.astype(dtype), g, axis=1)
    s = np.matmul(qd.transpose(1, 0, 2), kd.transpose(1, 2, 0)) * dtype(scale)  # [H, Lq, Lk]
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p = p / p.sum(axis=-1, keepdims=True)
    return np.matmul(p, vd.transpose(1, 0, 2)).transpose(1, 0, 2).astype(dtype)  # [Lq, H, D]


def varlen(q, k, v, cu_q, cu_k, scale: float, dtype=np.float64, seg_ids=None, out=None) -> np.ndarray:
    """Segments s: q rows [cu_q[s], cu_q[s+1]), k/v rows [cu_k[s], cu_k[s+1])."""
    cu_q = np.asarray(cu_q)
    cu_k = np.asarray(cu_k)
    if out is None:
        out = np.zeros(q.shape, dtype=dtype)
    ids = range(len(cu_q) - 1) if seg_ids is None else seg_ids
    for s in ids:
        q0, q1, k0, k1 = int(cu_q[s]), int(cu_q[s + 1]), int(cu_k[s]), int(cu_k[s + 1])
        if q1 > q0:
            out[q0:q1] = segment(q[q0:q1], k[k0:k1], v[k0:k1], scale, dtype)
    return out


def block_cached(q_blk, k_blk, v_blk, k_cache, v_cache, slots, scale: float, dtype=np.float64) -> np.ndarray:
    """Mode 2: keys/values = [cache rows slots[0..n_c) ; block rows].  Slots
    outside the cache are left out (the kernels' documented rule; the
    reference would read out of bounds)."""
    Hkv, D = k_blk.shape[1], k_blk.shape[2]
    slots = np.asarray(slots, dtype=np.int64)
    slots = slots[(slots >= 0) & (slots < k_cache.shape[0])]
    kc = np.zeros((slots.size, Hkv, D), dtype=k_cache.dtype)
    vc = np.zeros((slots.size, Hkv, D), dtype=v_cache.dtype)
    _kv.load(kc, vc, k_cache, v_cache, slots)
    return segment(q_blk, np.concatenate([kc, k_blk]), np.concatenate([vc, v_blk]), scale, dtype)


def mixed_step(q, k, v, seqs_desc, k_cache, v_cache, slot_lists, scale: float, D_sqrt=None,
               dtype=np.float64):
    """One diffusion forward of the attention layer.

    q/k/v: packed rows as the runner feeds them; values are the bf16 inputs
    given as float arrays.  seqs_desc: per sequence a dict with keys
      mode (0/1/2), rows (fed rows), and for modes 1/2: blk_start, blk_len,
      n_keep, head_select, pool_k.
    k_cache / v_cache: [slots, Hkv, D] arrays updated in place by mode 1
    (bf16 bit patterns as uint16 or float values; copies are exact).
    Returns (out [rows,Hq,D] in dtype, {seq index: selected indices}).
    """
    Hq, D = q.shape[1], q.shape[2]
    out = np.zeros(q.shape, dtype=dtype)
    chosen = {}
    row = 0
    sqrt_d = np.float32(D ** 0.5) if D_sqrt is None else np.float32(D_sqrt)
    for i, sd in enumerate(seqs_desc):
        n = sd["rows"]
        r0, r1 = row, row + n
        row = r1
        mode = sd["mode"]
        if mode in (0, 1):
            out[r0:r1] = segment(q[r0:r1], k[r0:r1], v[r0:r1], scale, dtype)
        if mode == 1:
            bs, bl = sd["blk_start"], sd["blk_len"]
            cand = np.concatenate([np.arange(0, bs), np.arange(bs + bl, n)]).astype(np.int64)
            idx = _sel.select(q[r0 + bs:r0 + bs + bl], k[r0:r1][cand], sd["n_keep"],
                              sd["head_select"], sd["pool_k"], sqrt_d)
            chosen[i] = idx
            kk = k[r0:r1][cand]
            vv = v[r0:r1][cand]
            if sd["head_select"]:
                hk = np.arange(k.shape[1])[None, :]
                ksel = kk[idx.T, hk]  # [n_keep, Hkv, D]
                vsel = vv[idx.T, hk]
            else:
                ksel, vsel = kk[idx], vv[idx]
            _kv.store(ksel, vsel, k_cache, v_cache, slot_lists[i])
        elif mode == 2:
            out[r0:r1] = block_cached(q[r0:r1], k[r0:r1], v[r0:r1], k_cache, v_cache, slot_lists[i], scale, dtype)
    return out, chosen
