"""K3b, page-table form (dllm_attn_block_cached_paged_fwd) on the GPU: the
same outputs, bit for bit, as the slot-list form over the equivalent slot
lists (cached row r of segment s at page_table[s, r // 256] * 256 + r % 256),
and within the bf16 tolerance (max-abs 2e-2, mean-abs 2e-3) of the fp32
oracle's mode-2 attention (oracle.attention.block_cached).  Rows whose page id
is outside the cache, or whose page index is past the table's width, are left
out of the softmax, as the slot-list form does with slots outside the cache.
The rows are those the reference's state-2 slot lists address
(dllmserve/engine/model_runner.py:257-273)."""
import numpy as np
import pytest
import torch

from helpers import assert_attn_close, to_np
from oracle import attention as oatt
from dllm_serve_amd import _capi

pytestmark = pytest.mark.gpu

D = 128
PAGE = 256


def _case(dev, blk, cached, Hq, Hkv, num_pages, seed, bad_pages=(), max_pages=None, seg_ids=None):
    """blk[s] block rows and cached[s] cached rows per segment; pages dealt from
    a shuffled list of num_pages; (s, j, id) in bad_pages overrides page j of
    segment s.  Returns outputs of both forms and the oracle."""
    rng = np.random.default_rng(seed)
    n = len(blk)
    need = [-(-c // PAGE) for c in cached]
    width = max(need + [1]) if max_pages is None else max_pages
    free = rng.permutation(max(num_pages, 1)).tolist() * 4
    table = np.full((n, width), -7, dtype=np.int32)
    at = 0
    for s in range(n):
        for j in range(min(need[s], width)):
            table[s, j] = free[at]
            at += 1
    for s, j, pid in bad_pages:
        table[s, j] = pid
    # the equivalent slot lists (-1 where the page is invalid or past the table)
    slots = []
    for s in range(n):
        for r in range(cached[s]):
            j = r // PAGE
            pid = int(table[s, j]) if j < width else -1
            slots.append(pid * PAGE + r % PAGE if 0 <= pid < num_pages else -1)
    slot_off = np.concatenate([[0], np.cumsum(cached)]).astype(np.int32)
    g = torch.Generator().manual_seed(seed)
    rows = sum(blk)
    q = torch.randn(rows, Hq, D, generator=g).to(torch.bfloat16)
    k = torch.randn(rows, Hkv, D, generator=g).to(torch.bfloat16)
    v = torch.randn(rows, Hkv, D, generator=g).to(torch.bfloat16)
    kc = torch.randn(max(num_pages, 1) * PAGE, Hkv, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(max(num_pages, 1) * PAGE, Hkv, D, generator=g).to(torch.bfloat16)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(blk)]), dtype=torch.int32)
    ids = list(range(n)) if seg_ids is None else list(seg_ids)
    # launch segment i = sequence ids[i]: its page-table row / cached length / slot range by position
    pt_l = table[ids]
    len_l = np.array([cached[i] for i in ids], dtype=np.int32)
    sl_l = np.concatenate([slots[slot_off[i]:slot_off[i + 1]] for i in ids] + [[]]).astype(np.int32)
    off_l = np.concatenate([[0], np.cumsum(len_l)]).astype(np.int32)
    max_q, max_keys = max(blk[i] for i in ids), max(blk[i] + cached[i] for i in ids)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    kcd, vcd = (kc.to(dev), vc.to(dev)) if num_pages else (kc[:0].to(dev), vc[:0].to(dev))
    ws_b = _capi.block_cached_workspace_size(len(ids), max_q, max_keys, Hq, Hkv, D)
    ws = torch.empty(max(ws_b, 16), dtype=torch.uint8, device=dev) if ws_b else None
    idd = None if seg_ids is None else torch.tensor(ids, dtype=torch.int32, device=dev)
    o_pg = torch.full_like(qd, float("nan")) if seg_ids is None else torch.full_like(qd, 5.0)
    o_sl = o_pg.clone()
    _capi.attn_block_cached_paged_fwd(qd, kd, vd, o_pg, cu.to(dev), idd, len(ids), max_q, max_keys, kcd, vcd,
                                      torch.from_numpy(pt_l.copy()).to(dev), torch.from_numpy(len_l).to(dev),
                                      D ** -0.5, ws)
    sl_t = torch.from_numpy(sl_l if sl_l.size else np.zeros(1, np.int32)).to(dev)
    _capi.attn_block_cached_fwd(qd, kd, vd, o_sl, cu.to(dev), idd, len(ids), max_q, max_keys,
                                kcd if num_pages else None, vcd if num_pages else None, sl_t,
                                torch.from_numpy(off_l).to(dev), D ** -0.5, ws)
    torch.cuda.synchronize()
    ref = np.full(q.shape, 5.0, dtype=np.float32)
    kn, vn = to_np(kc), to_np(vc)
    for i in ids:
        r = slice(int(cu[i]), int(cu[i + 1]))
        sl = slots[slot_off[i]:slot_off[i + 1]] if num_pages else [-1] * cached[i]
        ref[r] = oatt.block_cached(to_np(q[r]), to_np(k[r]), to_np(v[r]), kn, vn, sl, D ** -0.5, dtype=np.float32)
    return o_pg, o_sl, ref, ids, cu


@pytest.mark.parametrize("blk,cached,Hq,Hkv,num_pages", [
    ([64] * 4, [608] * 4, 32, 32, 16),                       # C4 reuse shape, one row block per workgroup
    ([32] * 16, [700] * 16, 28, 4, 48),                      # Dream GQA shape, paired row blocks
    ([32, 16], [3000, 2900], 32, 32, 30),                    # few segments: keys split over workgroups
    ([1, 7, 32, 20, 9], [0, 255, 256, 257, 513], 16, 4, 8),  # ragged blocks, page edges, no cache rows
])
def test_paged_matches_slot_lists_and_oracle(dev, blk, cached, Hq, Hkv, num_pages):
    print(f"paged K3b blk={blk[:4]}.. cached={cached[:4]}.. Hq={Hq} Hkv={Hkv} pages={num_pages}", flush=True)
    o_pg, o_sl, ref, _, _ = _case(dev, blk, cached, Hq, Hkv, num_pages, seed=sum(cached) + Hq)
    assert torch.equal(o_pg.view(torch.int16), o_sl.view(torch.int16)), "page-table form differs from slot lists"
    assert_attn_close(o_pg, ref, "paged")


def test_paged_invalid_pages_and_short_table(dev):
    """Page ids -1 and >= num_pages, and cached lengths past the table's width:
    those rows are left out; the rest attend as usual."""
    print("paged K3b: invalid page ids, short page table", flush=True)
    blk, cached = [32, 32, 32], [700, 600, 900]
    o_pg, o_sl, ref, _, _ = _case(dev, blk, cached, 32, 8, 12, seed=77,
                                  bad_pages=[(0, 1, -1), (1, 0, 12), (1, 2, 1 << 30)], max_pages=3)
    assert torch.equal(o_pg.view(torch.int16), o_sl.view(torch.int16))
    assert_attn_close(o_pg, ref, "paged invalid")


def test_paged_without_cache_and_subset(dev):
    """num_pages = 0 (every cached row left out), and a launch over a subset
    of the batch through seg_ids (other rows untouched)."""
    print("paged K3b: no cache; seg-id subset", flush=True)
    o_pg, o_sl, ref, _, _ = _case(dev, [32, 8], [300, 40], 8, 2, 0, seed=5)
    assert_attn_close(o_pg, ref, "paged no cache")
    o_pg, o_sl, ref, ids, cu = _case(dev, [32, 16, 24, 32], [500, 0, 256, 1000], 32, 32, 16, seed=6, seg_ids=[3, 0])
    assert torch.equal(o_pg.view(torch.int16), o_sl.view(torch.int16))
    assert_attn_close(o_pg, ref, "paged subset")
    for i in (1, 2):
        assert bool((o_pg[int(cu[i]):int(cu[i + 1])].float() == 5.0).all()), f"segment {i} outside the launch written"
