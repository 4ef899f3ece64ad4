"""K5 / K6 selection + fused cache scatter on the GPU vs the oracle.

Bar: selected indices and the whole KV cache bit-exact."""
import numpy as np
import pytest
import torch

from helpers import bits, to_np

from oracle import select as osel
from oracle import kvcache as okv
from dllm_serve_amd import _capi
from dllm_serve_amd.engine.sequence import PageAllocator, Sequence, slot_mapping_for
from dllm_serve_amd.sparse.state import SparseConfig, keep_count

pytestmark = pytest.mark.gpu

D = 128


def _run_jobs(dev, q, k, v, specs, kc_cache, vc_cache, slots, max_kc=None, max_keep=None, ws_extra=0):
    """specs: per job (row0, n_tok, bs, bl, n_keep, slot_off, head_select, pool_k).
    Returns idx [n_job, Hkv, max_keep] (int64, -1 where unwritten) and the workspace."""
    Hq, Hkv = q.shape[1], k.shape[1]
    n_job = len(specs)
    max_kc = max_kc if max_kc is not None else max(s[1] - s[3] for s in specs)
    max_keep = max_keep if max_keep is not None else max(s[4] for s in specs)
    jobs = torch.tensor(specs, dtype=torch.int32, device=dev)
    idx = torch.full((n_job, Hkv, max_keep), -1, dtype=torch.int64, device=dev)
    need = _capi.select_workspace_size(n_job, max_kc, Hq, Hkv, D)
    ws = torch.empty(need + ws_extra, dtype=torch.uint8, device=dev)
    if ws_extra:
        ws[need:] = 0xA5
    _capi.select_kv_store(q, k, v, jobs, n_job, max_kc, max_keep, np.float32(D ** 0.5), kc_cache, vc_cache,
                          slots, idx, ws)
    torch.cuda.synchronize()
    return idx.cpu().numpy(), ws, need


def _expected(q, k, v, spec, ref_kc, ref_vc, slots_np):
    """Oracle selection of one job; stores the selected rows into the reference
    caches (bit patterns) in place; returns the indices ([Hkv, n] or [n])."""
    row0, n_tok, bs, bl, n_keep, soff, hs, pk = spec
    qn, kn = to_np(q[row0:row0 + n_tok]), to_np(k[row0:row0 + n_tok])
    Hkv = k.shape[1]
    cand = np.concatenate([np.arange(0, bs), np.arange(bs + bl, n_tok)])
    idx = osel.select(qn[bs:bs + bl], kn[cand], n_keep, bool(hs), pk, np.float32(D ** 0.5))
    kb = bits(k[row0:row0 + n_tok]).reshape(n_tok, Hkv, D)
    vb = bits(v[row0:row0 + n_tok]).reshape(n_tok, Hkv, D)
    if hs:
        hk = np.arange(Hkv)[None, :]
        ksel, vsel = kb[cand][idx.T, hk], vb[cand][idx.T, hk]
    else:
        ksel, vsel = kb[cand][idx], vb[cand][idx]
    okv.store(ksel.reshape(n_keep, -1), vsel.reshape(n_keep, -1), ref_kc, ref_vc, slots_np[soff:soff + n_keep])
    return idx


def _check(got, idx_ref, spec, what):
    n_keep, hs = spec[4], spec[6]
    g = got[:, :n_keep] if hs else got[:1, :n_keep]
    want = idx_ref if hs else idx_ref[None, :]
    mism = int((g != want).sum())
    assert mism == 0, f"{what}: {mism} of {want.size} selected indices differ"


def _inputs(n_tok, Hq, Hkv, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(n_tok, Hq, D, generator=g).to(torch.bfloat16)
    k = torch.randn(n_tok, Hkv, D, generator=g).to(torch.bfloat16)
    v = torch.randn(n_tok, Hkv, D, generator=g).to(torch.bfloat16)
    return q, k, v


def _one_job(dev, n_tok, bs, bl, Hq, Hkv, ratio, head_select, pool_k, seed):
    Kc = n_tok - bl
    n_keep = keep_count(Kc, ratio)
    pages = -(-n_keep // 256) + 2
    q, k, v = _inputs(n_tok, Hq, Hkv, seed)
    g = torch.Generator().manual_seed(seed + 99)
    kc = torch.randn(pages * 256, Hkv, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(pages * 256, Hkv, D, generator=g).to(torch.bfloat16)
    slots = torch.randperm(pages * 256, generator=g)[:n_keep].to(torch.int32)
    spec = (0, n_tok, bs, bl, n_keep, 0, int(head_select), pool_k)
    ref_kc, ref_vc = bits(kc).reshape(-1, Hkv * D).copy(), bits(vc).reshape(-1, Hkv * D).copy()
    idx_ref = _expected(q, k, v, spec, ref_kc, ref_vc, slots.numpy())
    kcd, vcd = kc.to(dev), vc.to(dev)
    got, _, _ = _run_jobs(dev, q.to(dev), k.to(dev), v.to(dev), [spec], kcd, vcd, slots.to(dev))
    _check(got[0], idx_ref, spec, f"n_tok={n_tok}")
    assert np.array_equal(bits(kcd).reshape(-1, Hkv * D), ref_kc)
    assert np.array_equal(bits(vcd).reshape(-1, Hkv * D), ref_vc)


CASES = [
    # n_tok, bs, bl, Hq, Hkv, ratio, head_select, pool_k
    (1280, 1024, 64, 32, 32, 0.5, True, 3),    # C4: LLaDA shape, head_select, 608 kept of 1216
    (1280, 1088, 64, 32, 32, 0.5, False, 3),   # token selection, block in the middle
    (400, 300, 32, 28, 4, 0.5, True, 3),       # Dream GQA (max over the 7 heads of a group)
    (400, 300, 32, 28, 4, 0.25, False, 2),     # GQA token selection, even pool kernel
    (96, 40, 16, 8, 8, 1.0, True, 1),          # keep everything, no pooling
    (50, 0, 17, 4, 4, 0.0, True, 5),           # ratio 0 keeps one row; block at the start
    (4128, 4000, 32, 32, 32, 0.5, True, 3),    # long sequence, 4096 candidates
]


@pytest.mark.parametrize("n_tok,bs,bl,Hq,Hkv,ratio,head_select,pool_k", CASES)
def test_select_store_bit_exact(dev, n_tok, bs, bl, Hq, Hkv, ratio, head_select, pool_k):
    print(f"select n_tok={n_tok} bs={bs} bl={bl} Hq={Hq} Hkv={Hkv} r={ratio} hs={head_select} p={pool_k}",
          flush=True)
    _one_job(dev, n_tok, bs, bl, Hq, Hkv, ratio, head_select, pool_k, seed=n_tok + bs)


@pytest.mark.parametrize("n_tok,bs,bl,Hq,Hkv,ratio,head_select,pool_k", [
    (12352, 12288, 64, 8, 8, 0.5, True, 3),    # 12288 candidates, 6144 kept: compaction, then the LDS sort
    (12352, 6000, 64, 8, 4, 0.5, False, 3),    # the same with GQA token selection
    (20032, 20000, 32, 4, 4, 0.9, True, 3),    # 18000 kept: the two-pass radix sort in the workspace
    (20032, 5000, 32, 4, 4, 0.3, True, 3),     # keys in the workspace, 6000 kept: 64-bit keys sorted in LDS
    (20032, 100, 32, 4, 2, 0.75, False, 1),    # 15000 kept, token selection, no pooling
])
def test_select_beyond_8192_candidates(dev, n_tok, bs, bl, Hq, Hkv, ratio, head_select, pool_k):
    """No candidate cap: the reference's torch.topk has none (attention.py:341,402-404)."""
    print(f"select long n_tok={n_tok} Hq={Hq} Hkv={Hkv} r={ratio} hs={head_select} p={pool_k}", flush=True)
    _one_job(dev, n_tok, bs, bl, Hq, Hkv, ratio, head_select, pool_k, seed=n_tok + Hkv)


@pytest.mark.parametrize("Hq,Hkv", [(6, 2), (10, 2), (12, 2), (24, 3), (16, 1), (64, 1)])
@pytest.mark.parametrize("head_select", [True, False])
def test_select_group_sizes(dev, Hq, Hkv, head_select):
    """Query heads per KV head g = 3 (one padded group of four), 5, 6 and 8 (one group of eight),
    16 (two groups) and 64 (the largest group the launch takes): the score kernel's head groups and
    the qbar padding, bit-exact in both selection modes."""
    print(f"select group size g={Hq // Hkv} Hq={Hq} Hkv={Hkv} hs={head_select}", flush=True)
    _one_job(dev, 360, 200, 24, Hq, Hkv, 0.5, head_select, 3, seed=Hq * 7 + Hkv)


def test_select_summation_order(dev):
    """Scores whose f64 sums are inexact, so the order of the additions decides
    the result: q rows of one token (qbar = q exactly) hold +-2^60 at
    d = 0 / 2 and ordinary values elsewhere, K holds 1 at those positions.
    Summed d ascending, the ordinary term at d = 1 vanishes in 2^60; token
    selection also adds KV-head partials of +-2^60 in head order.  The kernel
    must follow the stated order exactly (oracle.select.dots / raw_scores)."""
    print("select summation order (cancelling 2^60 terms)", flush=True)
    for hs, Hq, Hkv in ((True, 4, 4), (False, 4, 4), (False, 8, 2)):
        n_tok, bl = 300, 1
        q, k, v = _inputs(n_tok, Hq, Hkv, seed=31 + Hq)
        big = 2.0 ** 60
        q[0, :, 0] = big
        q[0, :, 2] = -big
        if not hs:
            # heads 0 / 1 end at +2^60 / -2^60: added in head order they cancel
            # before the other heads' sums arrive, which then survive whole
            q[0, 0, 3] = big
            q[0, 1, 3] = -big
        k[:, :, 0] = 1.0
        k[:, :, 2] = 1.0
        k[:, :, 3] = 1.0
        Kc = n_tok - bl
        spec = (0, n_tok, 0, bl, keep_count(Kc, 0.5), 0, int(hs), 3)
        cache = torch.zeros(2, 256, Hkv, D, dtype=torch.bfloat16)
        slots = torch.arange(spec[4], dtype=torch.int32)
        ref_kc, ref_vc = bits(cache[0]).reshape(-1, Hkv * D).copy(), bits(cache[1]).reshape(-1, Hkv * D).copy()
        idx_ref = _expected(q, k, v, spec, ref_kc, ref_vc, slots.numpy())
        cd = cache.to(dev)
        got, _, _ = _run_jobs(dev, q.to(dev), k.to(dev), v.to(dev), [spec], cd[0], cd[1], slots.to(dev))
        _check(got[0], idx_ref, spec, f"hs={hs} Hq={Hq} Hkv={Hkv}")
        assert np.array_equal(bits(cd[0]).reshape(-1, Hkv * D), ref_kc)


def test_select_c4_four_jobs(dev):
    """C4: B=4 sequences of 1024 prompt + 256 generated tokens, block 0 of the
    generation (rows 1024..1087), retention 0.5, head_select, pool 3; slots
    from slot_mapping_for over a shuffled page table; one launch."""
    print("select C4 4 jobs x 1280 tokens, 32 heads", flush=True)
    Hq = Hkv = 32
    cfg = SparseConfig(enabled=True, default_block_len=64, retention_ratio=0.5, pool_kernel=3, head_select=True)
    seqs = [Sequence([1] * 1024, 256, 126336, cfg, device="cpu") for _ in range(4)]
    n_pages = sum(s.num_blocks for s in seqs) + 3
    perm = torch.randperm(n_pages, generator=torch.Generator().manual_seed(4)).tolist()
    alloc = PageAllocator(perm)
    for s in seqs:
        alloc.allocate(s)
    q, k, v = _inputs(4 * 1280, Hq, Hkv, seed=1280)
    specs, slot_list = [], []
    for b, s in enumerate(seqs):
        n_keep = keep_count(1280 - 64, 0.5)
        s.sparse_state.cache_state = 1   # the block's selection step (delay_step 1, step 1)
        sl = slot_mapping_for(s)
        assert len(sl) == n_keep == 608
        specs.append((b * 1280, 1280, 1024, 64, n_keep, b * n_keep, 1, 3))
        slot_list.extend(sl)
    slots = torch.tensor(slot_list, dtype=torch.int32)
    cache = torch.zeros(2, n_pages * 256, Hkv, D, dtype=torch.bfloat16)
    ref_kc, ref_vc = bits(cache[0]).reshape(-1, Hkv * D).copy(), bits(cache[1]).reshape(-1, Hkv * D).copy()
    refs = [_expected(q, k, v, sp, ref_kc, ref_vc, slots.numpy()) for sp in specs]
    cd = cache.to(dev)
    got, _, _ = _run_jobs(dev, q.to(dev), k.to(dev), v.to(dev), specs, cd[0], cd[1], slots.to(dev))
    for j, (sp, ref) in enumerate(zip(specs, refs)):
        _check(got[j], ref, sp, f"job {j}")
    assert np.array_equal(bits(cd[0]).reshape(-1, Hkv * D), ref_kc)
    assert np.array_equal(bits(cd[1]).reshape(-1, Hkv * D), ref_vc)


def test_select_wide_score_workgroups_ragged(dev):
    """Four jobs of 32 KV heads with 1216 / 1100 / 1000 / 1210 candidates:
    256 candidates per score workgroup would need 5 x 32 x 4 = 640 workgroups
    (more than the 512 that fit at once), so the launch takes 304 per
    workgroup (threads 0..47 score a second candidate) -- with partly filled
    last workgroups here, head and token selection mixed."""
    print("select wide score workgroups, ragged", flush=True)
    Hq = Hkv = 32
    lens = [(1280, 1024, 64, 0.5, 1, 3), (1164, 900, 64, 0.5, 0, 3), (1064, 1000, 64, 0.25, 1, 5),
            (1274, 0, 64, 0.5, 1, 1)]
    n = sum(x[0] for x in lens)
    q, k, v = _inputs(n, Hq, Hkv, seed=304)
    specs, row0, soff = [], 0, 0
    for n_tok, bs, bl, r, hs, pk in lens:
        nk = keep_count(n_tok - bl, r)
        specs.append((row0, n_tok, bs, bl, nk, soff, hs, pk))
        row0 += n_tok
        soff += nk
    assert max(s[1] - s[3] for s in specs) == 1216
    pages = -(-soff // 256) + 1
    slots = torch.randperm(pages * 256, generator=torch.Generator().manual_seed(5))[:soff].to(torch.int32)
    cache = torch.zeros(2, pages * 256, Hkv, D, dtype=torch.bfloat16)
    ref_kc, ref_vc = bits(cache[0]).reshape(-1, Hkv * D).copy(), bits(cache[1]).reshape(-1, Hkv * D).copy()
    refs = [_expected(q, k, v, sp, ref_kc, ref_vc, slots.numpy()) for sp in specs]
    cd = cache.to(dev)
    got, _, _ = _run_jobs(dev, q.to(dev), k.to(dev), v.to(dev), specs, cd[0], cd[1], slots.to(dev))
    for j, (sp, ref) in enumerate(zip(specs, refs)):
        _check(got[j], ref, sp, f"job {j}")
    assert np.array_equal(bits(cd[0]).reshape(-1, Hkv * D), ref_kc)
    assert np.array_equal(bits(cd[1]).reshape(-1, Hkv * D), ref_vc)


def test_select_wide_score_workgroups_gqa(dev):
    """28 query / 4 KV heads, 32 jobs of up to 1216 candidates: 5 x 4 x 32 =
    640 score workgroups of 256 would need a second generation, so the launch
    takes 304 candidates per workgroup with qbar padded from 7 to 8 heads
    (the dot products run four heads at a time); ragged jobs, head and token
    selection."""
    print("select wide score workgroups, GQA 28/4, 32 jobs", flush=True)
    Hq, Hkv = 28, 4
    rng = np.random.default_rng(28)
    lens = []
    for j in range(32):
        n_tok = int(rng.integers(1000, 1281)) if j else 1280
        bl = 64
        bs = int(rng.integers(0, n_tok - bl + 1))
        lens.append((n_tok, bs, bl, 0.5, j % 2, (1, 3, 5)[j % 3]))
    n = sum(x[0] for x in lens)
    q, k, v = _inputs(n, Hq, Hkv, seed=2804)
    specs, row0, soff = [], 0, 0
    for n_tok, bs, bl, r, hs, pk in lens:
        nk = keep_count(n_tok - bl, r)
        specs.append((row0, n_tok, bs, bl, nk, soff, hs, pk))
        row0 += n_tok
        soff += nk
    assert max(s[1] - s[3] for s in specs) == 1216
    pages = -(-soff // 256) + 1
    slots = torch.randperm(pages * 256, generator=torch.Generator().manual_seed(6))[:soff].to(torch.int32)
    cache = torch.zeros(2, pages * 256, Hkv, D, dtype=torch.bfloat16)
    ref_kc, ref_vc = bits(cache[0]).reshape(-1, Hkv * D).copy(), bits(cache[1]).reshape(-1, Hkv * D).copy()
    refs = [_expected(q, k, v, sp, ref_kc, ref_vc, slots.numpy()) for sp in specs]
    cd = cache.to(dev)
    got, _, _ = _run_jobs(dev, q.to(dev), k.to(dev), v.to(dev), specs, cd[0], cd[1], slots.to(dev))
    for j, (sp, ref) in enumerate(zip(specs, refs)):
        _check(got[j], ref, sp, f"job {j}")
    assert np.array_equal(bits(cd[0]).reshape(-1, Hkv * D), ref_kc)
    assert np.array_equal(bits(cd[1]).reshape(-1, Hkv * D), ref_vc)


def test_select_mixed_configs_one_launch(dev):
    """Jobs of one launch with head_select True / False and pool 1 / 3 / 5 and
    different ratios (each SparseConfig read per sequence, attention.py:211,
    329,387)."""
    print("select mixed configs", flush=True)
    Hq, Hkv = 16, 4
    lens = [(300, 200, 32, 0.5, 1, 1), (520, 256, 64, 0.3, 0, 3), (260, 0, 16, 0.75, 1, 5), (400, 384, 16, 1.0, 0, 5)]
    n = sum(x[0] for x in lens)
    q, k, v = _inputs(n, Hq, Hkv, seed=77)
    specs, row0, soff = [], 0, 0
    for n_tok, bs, bl, r, hs, pk in lens:
        nk = keep_count(n_tok - bl, r)
        specs.append((row0, n_tok, bs, bl, nk, soff, hs, pk))
        row0 += n_tok
        soff += nk
    pages = -(-soff // 256) + 1
    slots = torch.randperm(pages * 256, generator=torch.Generator().manual_seed(3))[:soff].to(torch.int32)
    cache = torch.zeros(2, pages * 256, Hkv, D, dtype=torch.bfloat16)
    ref_kc, ref_vc = bits(cache[0]).reshape(-1, Hkv * D).copy(), bits(cache[1]).reshape(-1, Hkv * D).copy()
    refs = [_expected(q, k, v, sp, ref_kc, ref_vc, slots.numpy()) for sp in specs]
    cd = cache.to(dev)
    got, _, _ = _run_jobs(dev, q.to(dev), k.to(dev), v.to(dev), specs, cd[0], cd[1], slots.to(dev))
    for j, (sp, ref) in enumerate(zip(specs, refs)):
        _check(got[j], ref, sp, f"job {j}")
    assert np.array_equal(bits(cd[0]).reshape(-1, Hkv * D), ref_kc)
    assert np.array_equal(bits(cd[1]).reshape(-1, Hkv * D), ref_vc)


def test_select_jobs_clamped_to_launch_sizes(dev):
    """Jobs that disagree with the launch sizes (more candidates than max_kc,
    more rows kept than max_keep, slots past the slot list, rows past the
    tensors) write nothing outside the workspace, the slot list or the cache:
    guard bytes after the workspace stay intact, and a job whose slots or rows
    overflow writes no cache row."""
    print("select clamped jobs with a guarded workspace", flush=True)
    Hq = Hkv = 8
    n = 900
    q, k, v = _inputs(n, Hq, Hkv, seed=5)
    cache = torch.zeros(2, 512, Hkv, D, dtype=torch.bfloat16, device=dev)
    slots = torch.arange(100, dtype=torch.int32, device=dev)
    specs = [(0, 400, 300, 32, 300, 0, 1, 3),       # Kc 368 > max_kc 200, n_keep 300 > max_keep 50
             (400, 300, 0, 32, 40, 80, 0, 3),       # slots 80..119: past the 100-entry slot list
             (700, 300, 0, 32, 10, 0, 1, 3)]        # rows 700..999: past the 900 rows
    got, ws, need = _run_jobs(dev, q.to(dev), k.to(dev), v.to(dev), specs, cache[0], cache[1], slots,
                              max_kc=200, max_keep=50, ws_extra=4096)
    assert torch.all(ws[need:] == 0xA5), "a kernel wrote past its workspace"
    written = (cache[0].view(512, -1) != 0).any(dim=1).cpu().numpy()
    assert not written[50:].any(), "rows beyond the first job's clamped 50 slots were written"
    assert (got[1] == -1).all() and (got[2] == -1).all(), "jobs outside the launch sizes must select nothing"
    # the clamped job selects its 50 best among its first 200 candidates (rows 0..199)
    ref = osel.select(to_np(q)[300:332], to_np(k)[:200], 50, True, 3, np.float32(D ** 0.5))
    assert np.array_equal(got[0][:, :50], ref), "clamped job"
