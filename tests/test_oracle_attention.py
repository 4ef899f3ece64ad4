"""Oracle pins for attention: library routine, fp64, invariants (CPU only)."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as oatt
from oracle import configs


def _sdpa(q, k, v, scale):
    """torch scaled_dot_product_attention (CPU fp32), GQA by repeating KV."""
    g = q.shape[1] // k.shape[1]
    qt = torch.from_numpy(q).float().transpose(0, 1)
    kt = torch.from_numpy(np.repeat(k, g, axis=1)).float().transpose(0, 1)
    vt = torch.from_numpy(np.repeat(v, g, axis=1)).float().transpose(0, 1)
    return F.scaled_dot_product_attention(qt, kt, vt, scale=scale).transpose(0, 1).numpy()


@pytest.mark.parametrize("Lq,Lk,Hq,Hkv", [(17, 17, 4, 4), (33, 70, 8, 2), (5, 1, 6, 3), (64, 64, 7, 1)])
def test_segment_matches_sdpa(Lq, Lk, Hq, Hkv):
    rng = np.random.default_rng(Lq * 100 + Lk)
    D = 128
    q = rng.standard_normal((Lq, Hq, D)).astype(np.float32)
    k = rng.standard_normal((Lk, Hkv, D)).astype(np.float32)
    v = rng.standard_normal((Lk, Hkv, D)).astype(np.float32)
    ref = _sdpa(q, k, v, D ** -0.5)
    assert np.abs(oatt.segment(q, k, v, D ** -0.5, np.float64) - ref).max() < 1e-5
    assert np.abs(oatt.segment(q, k, v, D ** -0.5, np.float32) - ref).max() < 1e-5


def test_mutated_oracle_is_caught():
    """A plausible mistake (GQA mapping h % Hkv instead of h // g, or a
    missing scale) fails the library comparison."""
    rng = np.random.default_rng(9)
    q = rng.standard_normal((9, 8, 128)).astype(np.float32)
    k = rng.standard_normal((12, 2, 128)).astype(np.float32)
    v = rng.standard_normal((12, 2, 128)).astype(np.float32)
    ref = _sdpa(q, k, v, 128 ** -0.5)
    kk = np.tile(k, (1, 4, 1))  # head h reads KV head h % 2
    vv = np.tile(v, (1, 4, 1))
    wrong_map = oatt.segment(q, kk, vv, 128 ** -0.5)
    assert np.abs(wrong_map - ref).max() > 1e-2
    assert np.abs(oatt.segment(q, k, v, 1.0) - ref).max() > 1e-2


def test_invariants():
    rng = np.random.default_rng(3)
    D = 128
    q = rng.standard_normal((20, 4, D)).astype(np.float32)
    k = rng.standard_normal((30, 2, D)).astype(np.float32)
    v = rng.standard_normal((30, 2, D)).astype(np.float32)
    base = oatt.segment(q, k, v, 0.1)
    perm = rng.permutation(30)
    assert np.allclose(oatt.segment(q, k[perm], v[perm], 0.1), base, atol=1e-12)   # key order
    assert np.allclose(oatt.segment(q, k[:1], v[:1], 0.1), np.repeat(v[:1], 2, 1), atol=1e-12)  # Lk = 1
    mean_v = np.repeat(v.mean(0, keepdims=True), 2, 1)
    assert np.allclose(oatt.segment(np.zeros_like(q), k, v, 0.1), mean_v, atol=1e-12)  # constant scores
    gq = oatt.segment(q, np.repeat(k, 2, 1), np.repeat(v, 2, 1), 0.1)  # GQA == repeated KV
    assert np.allclose(gq, base, atol=1e-12)


def test_varlen_segments_are_independent():
    lens = [5, 17, 1, 40]
    q, k, v, cu = configs.packed_qkv(lens, 4, 2, 128, seed=4, dtype=torch.float32)
    qn, kn, vn, cun = q.numpy(), k.numpy(), v.numpy(), cu.numpy()
    packed = oatt.varlen(qn, kn, vn, cun, cun, 0.1)
    for s in range(len(lens)):
        a, b = cun[s], cun[s + 1]
        assert np.allclose(packed[a:b], oatt.segment(qn[a:b], kn[a:b], vn[a:b], 0.1), atol=1e-12)


def test_block_cached_is_attention_over_gathered_rows():
    rng = np.random.default_rng(5)
    D, Hq, Hkv = 128, 4, 4
    kc = rng.standard_normal((300, Hkv, D)).astype(np.float32)
    vc = rng.standard_normal((300, Hkv, D)).astype(np.float32)
    slots = rng.permutation(300)[:57]
    qb = rng.standard_normal((9, Hq, D)).astype(np.float32)
    kb = rng.standard_normal((9, Hkv, D)).astype(np.float32)
    vb = rng.standard_normal((9, Hkv, D)).astype(np.float32)
    got = oatt.block_cached(qb, kb, vb, kc, vc, slots, 0.2)
    want = oatt.segment(qb, np.concatenate([kc[slots], kb]), np.concatenate([vc[slots], vb]), 0.2)
    assert np.allclose(got, want, atol=1e-12)


def test_retention_one_reuse_equals_full_attention_rows():
    """With every candidate kept and fresh K/V, the mode-2 block output equals
    the block rows of full attention (attention is key-order invariant)."""
    rng = np.random.default_rng(6)
    N, bs, bl, H, D = 48, 16, 8, 2, 128
    q = rng.standard_normal((N, H, D)).astype(np.float32)
    k = rng.standard_normal((N, H, D)).astype(np.float32)
    v = rng.standard_normal((N, H, D)).astype(np.float32)
    kc = np.zeros((64, H, D), np.float32)
    vc = np.zeros((64, H, D), np.float32)
    slots = list(range(N - bl))
    desc1 = [dict(mode=1, rows=N, blk_start=bs, blk_len=bl, n_keep=N - bl, head_select=True, pool_k=3)]
    full, _ = oatt.mixed_step(q, k, v, desc1, kc, vc, [slots], 0.1)
    blk = slice(bs, bs + bl)
    out2, _ = oatt.mixed_step(q[blk], k[blk], v[blk], [dict(mode=2, rows=bl)], kc, vc, [slots], 0.1)
    assert np.allclose(out2, full[blk], atol=1e-10)


def test_c1_config_shapes():
    q, k, v, cu, scale = configs.c1_single_layer()
    assert q.shape == (512, 32, 128) and q.dtype == torch.float32
    assert cu.tolist() == [0, 512] and abs(scale - 128 ** -0.5) < 1e-15
