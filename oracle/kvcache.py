"""store_kvcache / load_kvcache restated on numpy arrays.

dllmserve/layers/attention.py:11-50 (store): for i < N,
    k_cache.flat_rows[slot[i]] = key[i]   (rows of Hkv*D elements; same for v)
attention.py:53-92 (load): key[i] = k_cache.flat_rows[slot[i]].
The cache is [num_slots, Hkv*D] here (the reference views
[num_blocks, 256, Hkv, D] as flat rows, attention.py:44).  Slots outside the
cache are skipped, matching the kernels' documented bounds rule.
"""
from __future__ import annotations

import numpy as np


def store(key: np.ndarray, value: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray, slots) -> None:
    n = key.shape[0]
    row = int(np.prod(k_cache.shape[1:]))
    kc = k_cache.reshape(k_cache.shape[0], row)
    vc = v_cache.reshape(v_cache.shape[0], row)
    slots = np.asarray(slots, dtype=np.int64).reshape(-1)
    assert slots.size == n
    ok = (slots >= 0) & (slots < kc.shape[0])
    kc[slots[ok]] = key.reshape(n, row)[ok]
    vc[slots[ok]] = value.reshape(n, row)[ok]


def load(key: np.ndarray, value: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray, slots) -> None:
    n = key.shape[0]
    row = int(np.prod(k_cache.shape[1:]))
    kc = k_cache.reshape(k_cache.shape[0], row)
    vc = v_cache.reshape(v_cache.shape[0], row)
    slots = np.asarray(slots, dtype=np.int64).reshape(-1)
    assert slots.size == n
    ok = (slots >= 0) & (slots < kc.shape[0])
    kf = key.reshape(n, row)
    vf = value.reshape(n, row)
    kf[ok] = kc[slots[ok]]
    vf[ok] = vc[slots[ok]]
