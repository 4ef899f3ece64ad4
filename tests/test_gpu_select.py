"""K5 / K6 selection + fused cache scatter on the GPU vs the oracle.

Bar: selected indices and the whole KV cache bit-exact."""
import numpy as np
import pytest
import torch

from helpers import bits, to_np

from oracle import select as osel
from oracle import kvcache as okv
from dllm_serve_amd import _capi
from dllm_serve_amd.sparse.state import keep_count

pytestmark = pytest.mark.gpu


def _job_case(n_tok, bs, bl, Hq, Hkv, seed, n_slots_pages):
    D = 128
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(n_tok, Hq, D, generator=g).to(torch.bfloat16)
    k = torch.randn(n_tok, Hkv, D, generator=g).to(torch.bfloat16)
    v = torch.randn(n_tok, Hkv, D, generator=g).to(torch.bfloat16)
    kc = torch.randn(n_slots_pages * 256, Hkv, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(n_slots_pages * 256, Hkv, D, generator=g).to(torch.bfloat16)
    return q, k, v, kc, vc


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
    D = 128
    Kc = n_tok - bl
    n_keep = keep_count(Kc, ratio)
    pages = -(-n_keep // 256) + 2
    q, k, v, kc, vc = _job_case(n_tok, bs, bl, Hq, Hkv, seed=n_tok + bs, n_slots_pages=pages)
    g = torch.Generator().manual_seed(99)
    slots = torch.randperm(pages * 256, generator=g)[:n_keep].to(torch.int32)

    # oracle
    qn, kn, vn = to_np(q), to_np(k), to_np(v)
    cand = np.concatenate([np.arange(0, bs), np.arange(bs + bl, n_tok)])
    idx_ref = osel.select(qn[bs:bs + bl], kn[cand], n_keep, head_select, pool_k, np.float32(D ** 0.5))
    kb, vb = bits(k).reshape(n_tok, Hkv, D), bits(v).reshape(n_tok, Hkv, D)
    if head_select:
        hk = np.arange(Hkv)[None, :]
        ksel, vsel = kb[cand][idx_ref.T, hk], vb[cand][idx_ref.T, hk]
    else:
        ksel, vsel = kb[cand][idx_ref], vb[cand][idx_ref]
    ref_kc, ref_vc = bits(kc).reshape(-1, Hkv * D).copy(), bits(vc).reshape(-1, Hkv * D).copy()
    okv.store(ksel.reshape(n_keep, -1), vsel.reshape(n_keep, -1), ref_kc, ref_vc, slots.numpy())

    # GPU
    jobs = torch.tensor([[0, n_tok, bs, bl, n_keep, 0]], dtype=torch.int32, device=dev)
    kcd, vcd = kc.to(dev), vc.to(dev)
    n_sel = Hkv if head_select else 1
    idx = torch.full((1, n_sel, n_keep), -1, dtype=torch.int64, device=dev)
    ws = torch.empty(_capi.select_workspace_size(1, Kc, Hq, Hkv, D, head_select), dtype=torch.uint8, device=dev)
    _capi.select_kv_store(q.to(dev), k.to(dev), v.to(dev), jobs, 1, Kc, n_keep, bl, head_select, pool_k,
                          np.float32(D ** 0.5), kcd, vcd, slots.to(dev), idx, ws)
    torch.cuda.synchronize()
    got = idx.cpu().numpy()[0]
    ref = idx_ref if head_select else idx_ref[None, :]
    mism = int((got != ref).sum())
    assert mism == 0, f"{mism} of {got.size} selected indices differ"
    assert np.array_equal(bits(kcd).reshape(-1, Hkv * D), ref_kc)
    assert np.array_equal(bits(vcd).reshape(-1, Hkv * D), ref_vc)


def test_select_two_jobs_batched(dev):
    """Two sequences in one launch, slots concatenated, different n_keep."""
    print("select two jobs", flush=True)
    D, Hq, Hkv = 128, 16, 16
    specs = [(300, 256, 32, 0.5), (520, 256, 64, 0.3)]  # n_tok, bs, bl, ratio
    g = torch.Generator().manual_seed(1234)
    qs, ks, vs, jobs, slot_list = [], [], [], [], []
    row0, soff = 0, 0
    total_keep = sum(keep_count(n - bl, r) for n, _, bl, r in specs)
    pages = -(-total_keep // 256) + 1
    perm = torch.randperm(pages * 256, generator=g)
    for n, bs, bl, r in specs:
        qs.append(torch.randn(n, Hq, D, generator=g).to(torch.bfloat16))
        ks.append(torch.randn(n, Hkv, D, generator=g).to(torch.bfloat16))
        vs.append(torch.randn(n, Hkv, D, generator=g).to(torch.bfloat16))
        nk = keep_count(n - bl, r)
        jobs.append([row0, n, bs, bl, nk, soff])
        slot_list.append(perm[soff:soff + nk])
        row0 += n
        soff += nk
    q, k, v = torch.cat(qs), torch.cat(ks), torch.cat(vs)
    slots = torch.cat(slot_list).to(torch.int32)
    kc = torch.zeros(pages * 256, Hkv, D, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    ref_kc, ref_vc = bits(kc).reshape(-1, Hkv * D).copy(), bits(vc).reshape(-1, Hkv * D).copy()
    kb, vb = bits(k).reshape(-1, Hkv, D), bits(v).reshape(-1, Hkv, D)
    refs = []
    for (n, bs, bl, r), jb, sl in zip(specs, jobs, slot_list):
        r0 = jb[0]
        cand = np.concatenate([np.arange(0, bs), np.arange(bs + bl, n)]) + r0
        idx_ref = osel.select(to_np(q)[r0 + bs:r0 + bs + bl], to_np(k)[cand], jb[4], True, 3, np.float32(D ** 0.5))
        refs.append(idx_ref)
        hk = np.arange(Hkv)[None, :]
        okv.store(kb[cand][idx_ref.T, hk].reshape(jb[4], -1), vb[cand][idx_ref.T, hk].reshape(jb[4], -1),
                  ref_kc, ref_vc, sl.numpy())
    max_kc = max(n - bl for n, _, bl, _ in specs)
    max_keep = max(j[4] for j in jobs)
    kcd, vcd = kc.to(dev), vc.to(dev)
    idx = torch.full((2, Hkv, max_keep), -1, dtype=torch.int64, device=dev)
    ws = torch.empty(_capi.select_workspace_size(2, max_kc, Hq, Hkv, D, True), dtype=torch.uint8, device=dev)
    _capi.select_kv_store(q.to(dev), k.to(dev), v.to(dev), torch.tensor(jobs, dtype=torch.int32, device=dev), 2,
                          max_kc, max_keep, 64, True, 3, np.float32(D ** 0.5), kcd, vcd, slots.to(dev), idx, ws)
    torch.cuda.synchronize()
    got = idx.cpu().numpy()
    for j, ref in enumerate(refs):
        assert np.array_equal(got[j][:, :ref.shape[1]], ref)
    assert np.array_equal(bits(kcd).reshape(-1, Hkv * D), ref_kc)
    assert np.array_equal(bits(vcd).reshape(-1, Hkv * D), ref_vc)
