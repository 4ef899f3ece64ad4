"""K1 / K2 (store_kvcache / load_kvcache) on the GPU vs the oracle: bit-exact."""
import numpy as np
import pytest
import torch

from helpers import bits

from oracle import kvcache as okv
from dllm_serve_amd.layers.attention import load_kvcache, store_kvcache

pytestmark = pytest.mark.gpu

SENTINEL = 0x7E7E  # bf16 pattern of untouched cache entries


def _case(n_tok, Hkv, D, n_slots, seed, stride_pad=0, dev="cuda"):
    g = torch.Generator().manual_seed(seed)
    row = Hkv * D
    key_full = torch.randn(n_tok, Hkv * D + stride_pad, generator=g).to(torch.bfloat16)
    val_full = torch.randn(n_tok, Hkv * D + stride_pad, generator=g).to(torch.bfloat16)
    slots = torch.randperm(n_slots, generator=g)[:n_tok].to(torch.int32)
    kc = torch.full((n_slots // 256, 256, Hkv, D), 0, dtype=torch.int16)
    kc.fill_(SENTINEL - 65536 if SENTINEL > 32767 else SENTINEL)
    kc = kc.view(torch.bfloat16)
    vc = kc.clone()
    key = key_full[:, :row].view(n_tok, Hkv, D)
    val = val_full[:, :row].view(n_tok, Hkv, D)
    return key, val, kc, vc, slots, key_full, val_full


@pytest.mark.parametrize("n_tok,Hkv,D,n_slots,pad", [
    (608, 32, 128, 1024, 0),    # head-sparse C4 store: 608 rows of 8 KiB
    (300, 4, 128, 512, 0),      # Dream GQA rows of 1 KiB
    (97, 32, 128, 512, 4096),   # key is a view with token stride 2x the row
    (1, 8, 128, 256, 0),
])
def test_store_load_bit_exact(dev, n_tok, Hkv, D, n_slots, pad):
    print(f"store/load n_tok={n_tok} Hkv={Hkv} pad={pad}", flush=True)
    key, val, kc, vc, slots, kf, vf = _case(n_tok, Hkv, D, n_slots, seed=n_tok, stride_pad=pad)
    ref_k = bits(kc).reshape(n_slots, -1).copy()
    ref_v = bits(vc).reshape(n_slots, -1).copy()
    okv.store(bits(key).reshape(n_tok, -1), bits(val).reshape(n_tok, -1), ref_k, ref_v, slots.numpy())

    kc_d, vc_d = kc.to(dev), vc.to(dev)
    key_d = kf.to(dev)[:, :Hkv * D].view(n_tok, Hkv, D)
    val_d = vf.to(dev)[:, :Hkv * D].view(n_tok, Hkv, D)
    store_kvcache(key_d, val_d, kc_d, vc_d, slots.to(dev))
    torch.cuda.synchronize()
    assert np.array_equal(bits(kc_d).reshape(n_slots, -1), ref_k)
    assert np.array_equal(bits(vc_d).reshape(n_slots, -1), ref_v)

    # round trip: load(store(x)) == x
    k2 = torch.zeros(n_tok, Hkv, D, dtype=torch.bfloat16, device=dev)
    v2 = torch.zeros_like(k2)
    load_kvcache(k2, v2, kc_d, vc_d, slots.to(dev))
    torch.cuda.synchronize()
    assert np.array_equal(bits(k2), bits(key))
    assert np.array_equal(bits(v2), bits(val))


def test_out_of_range_slots_skipped(dev):
    print("store/load out-of-range slots", flush=True)
    key, val, kc, vc, slots, kf, vf = _case(64, 8, 128, 256, seed=7)
    slots[3] = -1
    slots[10] = 256  # == capacity
    kc_d, vc_d = kc.to(dev), vc.to(dev)
    store_kvcache(key.to(dev), val.to(dev), kc_d, vc_d, slots.to(dev))
    torch.cuda.synchronize()
    ref_k = bits(kc).reshape(256, -1).copy()
    ref_v = bits(vc).reshape(256, -1).copy()
    okv.store(bits(key).reshape(64, -1), bits(val).reshape(64, -1), ref_k, ref_v, slots.numpy())
    assert np.array_equal(bits(kc_d).reshape(256, -1), ref_k)
    assert np.array_equal(bits(vc_d).reshape(256, -1), ref_v)


def test_slot_count_mismatch_asserts(dev):
    key, val, kc, vc, slots, _, _ = _case(16, 8, 128, 256, seed=3)
    with pytest.raises(AssertionError):
        store_kvcache(key.to(dev), val.to(dev), kc.to(dev), vc.to(dev), slots[:15].to(dev))


def test_empty_store_is_noop(dev):
    key, val, kc, vc, slots, _, _ = _case(1, 8, 128, 256, seed=4)
    kc_d = kc.to(dev)
    vc_d = vc.to(dev)
    store_kvcache(key[:0].to(dev), val[:0].to(dev), kc_d, vc_d, slots[:0].to(dev))
    torch.cuda.synchronize()
    assert np.array_equal(bits(kc_d), bits(kc))
