"""K7 (NeoX RoPE of q and k) on the GPU: bit-exact against the oracle's
op-by-op f32 evaluation (oracle.rope.rotate_table) and against the
reference's f32 tensor expression run eagerly by torch on the same device."""
import numpy as np
import pytest
import torch

from helpers import bits, to_np

from oracle import rope as orope
from dllm_serve_amd import _capi
from dllm_serve_amd.layers.rotary_embedding import RotaryEmbedding

pytestmark = pytest.mark.gpu


def _oracle_bits(x, pos, table):
    return orope.rotate_table(to_np(x), pos.cpu().numpy(), table.cpu().numpy())


def _torch_expr(x, pos, table):
    """rotary_embedding.py:6-17,47-56 as eager torch ops."""
    D = x.shape[-1]
    cs = table[pos]
    cos, sin = cs[:, None, :D // 2], cs[:, None, D // 2:]
    x1, x2 = torch.chunk(x.to(torch.float32), 2, dim=-1)
    return torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), dim=-1).to(x.dtype)


@pytest.mark.parametrize("n,Hq,Hkv,D,theta", [
    (768, 32, 32, 128, 500000.0),      # LLaDA-8B
    (333, 28, 4, 128, 1000000.0),      # Dream-7B GQA
    (65, 8, 2, 64, 10000.0),           # head_dim 64
])
def test_rope_module_bit_exact(dev, n, Hq, Hkv, D, theta):
    print(f"rope n={n} Hq={Hq} Hkv={Hkv} D={D}", flush=True)
    g = torch.Generator().manual_seed(n + Hq)
    rope = RotaryEmbedding(D, D, 8192, theta).to(dev)
    q = torch.randn(n, Hq * D, generator=g).to(torch.bfloat16).to(dev)
    k = torch.randn(n, Hkv * D, generator=g).to(torch.bfloat16).to(dev)
    pos = torch.randint(0, 8192, (n,), generator=g).to(dev)
    q0, k0 = q.clone(), k.clone()
    qr, kr = rope(pos, q, k)
    torch.cuda.synchronize()
    assert torch.equal(q, q0) and torch.equal(k, k0)          # out of place by default
    assert qr.shape == q.shape and kr.shape == k.shape
    table = rope.cos_sin_cache
    q3, k3 = q.view(n, Hq, D), k.view(n, Hkv, D)
    assert np.array_equal(bits(qr.view(n, Hq, D)), _oracle_bits(q3, pos, table))
    assert np.array_equal(bits(kr.view(n, Hkv, D)), _oracle_bits(k3, pos, table))
    assert torch.equal(qr.view(n, Hq, D), _torch_expr(q3, pos, table))
    assert torch.equal(kr.view(n, Hkv, D), _torch_expr(k3, pos, table))


def test_rope_in_place_on_merged_qkv_views(dev):
    """q / k as column slices of one QKV projection (token stride > H*D),
    rotated in place; the v columns are untouched."""
    print("rope in place, merged qkv", flush=True)
    n, Hq, Hkv, D = 200, 28, 4, 128
    g = torch.Generator().manual_seed(7)
    qkv = torch.randn(n, (Hq + 2 * Hkv) * D, generator=g).to(torch.bfloat16).to(dev)
    ref = qkv.clone()
    q, k = qkv[:, :Hq * D], qkv[:, Hq * D:(Hq + Hkv) * D]
    pos = torch.arange(n, device=dev) * 3
    rope = RotaryEmbedding(D, D, 4096, 1000000.0, inplace=True).to(dev)
    qr, kr = rope(pos, q, k)
    torch.cuda.synchronize()
    assert qr.data_ptr() == q.data_ptr() and kr.data_ptr() == k.data_ptr()
    table = rope.cos_sin_cache
    assert np.array_equal(bits(qkv[:, :Hq * D].reshape(n, Hq, D)),
                          _oracle_bits(ref[:, :Hq * D].reshape(n, Hq, D), pos, table))
    assert np.array_equal(bits(qkv[:, Hq * D:(Hq + Hkv) * D].reshape(n, Hkv, D)),
                          _oracle_bits(ref[:, Hq * D:(Hq + Hkv) * D].reshape(n, Hkv, D), pos, table))
    assert torch.equal(qkv[:, (Hq + Hkv) * D:], ref[:, (Hq + Hkv) * D:])


def test_rope_out_of_range_positions_not_written(dev):
    print("rope out-of-range positions", flush=True)
    n, H, D = 16, 4, 128
    rope = RotaryEmbedding(D, D, 64, 10000.0).to(dev)
    g = torch.Generator().manual_seed(9)
    q = torch.randn(n, H, D, generator=g).to(torch.bfloat16).to(dev)
    k = torch.randn(n, H, D, generator=g).to(torch.bfloat16).to(dev)
    pos = torch.arange(n, device=dev)
    pos[3] = -1
    pos[7] = 64
    qo = torch.full_like(q, 7.0)
    ko = torch.full_like(k, 7.0)
    _capi.rope_neox(q, qo, k, ko, pos, rope.cos_sin_cache, n, H, H, D)
    torch.cuda.synchronize()
    ok = torch.ones(n, dtype=torch.bool)
    ok[3] = ok[7] = False
    assert torch.all(qo[~ok.to(dev)] == 7.0) and torch.all(ko[~ok.to(dev)] == 7.0)
    want = _oracle_bits(q[ok.to(dev)], pos[ok.to(dev)], rope.cos_sin_cache)
    assert np.array_equal(bits(qo[ok.to(dev)]), want)
