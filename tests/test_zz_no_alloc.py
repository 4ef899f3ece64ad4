"""The allocation-free block-cached entry point (dllm_attn_block_cached_fwd_noalloc)
against the workspace entry point it mirrors, through the C ABI.

Both run the same kernels with the same launch plan, so their outputs must be
bit-identical.  Two calls in a row, the second on a smaller input, so the
static scratch keeps the first call's partial records when the second runs;
a launch that splits its keys (few segments) is used so that the scratch is
really written and read."""
import numpy as np
import pytest
import torch

from helpers import assert_attn_close, bits, to_np

from oracle import attention as oatt
from oracle import configs
from dllm_serve_amd import _capi

pytestmark = pytest.mark.gpu


def _case(prefix, blk, Hq, Hkv, seed, page=256):
    g = torch.Generator().manual_seed(seed)
    D = 128
    pages_per = [-(-p // page) for p in prefix]
    n_pages = sum(pages_per) + 2
    perm = torch.randperm(n_pages, generator=g).tolist()
    kc = torch.randn(n_pages * page, Hkv, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(n_pages * page, Hkv, D, generator=g).to(torch.bfloat16)
    slots, at = [], 0
    for p, npg in zip(prefix, pages_per):
        s = []
        for j in range(npg):
            pid = perm[at + j]
            fill = page if j < npg - 1 else p - page * (npg - 1)
            s.extend(range(pid * page, pid * page + fill))
        at += npg
        slots.append(s)
    q, k, v, cu = configs.packed_qkv(blk, Hq, Hkv, D, seed=seed + 1)
    return q, k, v, cu, kc, vc, slots


def _run_both(dev, prefix, blk, Hq, Hkv, seed):
    q, k, v, cu, kc, vc, slots = _case(prefix, blk, Hq, Hkv, seed)
    D = 128
    off = [0]
    for s in slots:
        off.append(off[-1] + len(s))
    flat = torch.tensor([x for s in slots for x in s], dtype=torch.int32, device=dev)
    slot_off = torch.tensor(off, dtype=torch.int32, device=dev)
    qd, kd, vd, kcd, vcd, cud = q.to(dev), k.to(dev), v.to(dev), kc.to(dev), vc.to(dev), cu.to(dev)
    max_keys = max(p + b for p, b in zip(prefix, blk))
    ws_bytes = _capi.block_cached_workspace_size(len(blk), max(blk), max_keys, Hq, Hkv, D)
    assert 0 < ws_bytes <= _capi.block_cached_noalloc_max_workspace(), ws_bytes
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    o_ws = torch.full_like(qd, float("nan"))
    o_na = torch.full_like(qd, float("nan"))
    _capi.attn_block_cached_fwd(qd, kd, vd, o_ws, cud, None, len(blk), max(blk), max_keys, kcd, vcd, flat, slot_off,
                                D ** -0.5, ws)
    _capi.attn_block_cached_fwd_noalloc(qd, kd, vd, o_na, cud, None, len(blk), max(blk), max_keys, kcd, vcd, flat,
                                        slot_off, D ** -0.5)
    torch.cuda.synchronize()
    assert np.array_equal(bits(o_na), bits(o_ws)), "no-alloc output differs from the workspace entry point"
    cul = cu.tolist()
    for i in range(len(blk)):
        r0, r1 = cul[i], cul[i + 1]
        ref = oatt.block_cached(to_np(q)[r0:r1], to_np(k)[r0:r1], to_np(v)[r0:r1], to_np(kc), to_np(vc), slots[i],
                                D ** -0.5, dtype=np.float32)
        assert_attn_close(o_na[r0:r1], ref, f"seq {i}")


def test_noalloc_matches_workspace_entry_twice(dev):
    print("no-alloc block-cached: 3 segments x 8 heads, 1200-3000 cached rows (key split)", flush=True)
    _run_both(dev, [1200, 3000, 2100], [32, 32, 20], 8, 8, seed=5)
    print("no-alloc block-cached: second, smaller call (1 segment, 700 cached rows)", flush=True)
    _run_both(dev, [700], [16], 8, 8, seed=9)


def test_noalloc_rejects_bad_head_dim(dev):
    q = torch.zeros(8, 4, 128, dtype=torch.bfloat16, device=dev)
    cu = torch.tensor([0, 8], dtype=torch.int32, device=dev)
    off = torch.tensor([0, 0], dtype=torch.int32, device=dev)
    with pytest.raises(RuntimeError, match="head_dim"):
        _capi.attn_block_cached_fwd_noalloc(q[..., :64], q[..., :64], q[..., :64], q[..., :64], cu, None, 1, 8, 8,
                                            None, None, None, off, 0.125)
