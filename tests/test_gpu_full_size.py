"""The benchmark workloads at full size, checked through properties that do not
need the CPU oracle at that size.

- C2 dense step (8 x 384 tokens, 32 heads x 128): every output row depends
  only on its own segment, so running a subset of the segments (through
  seg_ids) or one segment alone gives bit-identical rows; permuting a
  segment's keys (and values) changes only the accumulation order.
- Dream-7B GQA shape (28 / 4 heads): grouped K/V give the same rows as the
  K/V heads repeated to 28 (bit-identical: a row's arithmetic does not depend
  on which other rows share its wavefront).
- C5 (32 blocks of 32 tokens against 2048..4096 cached rows in shuffled
  pages): store -> load round trip bit-exact at 100k rows; block-cached
  attention over the pages equals dense attention over the gathered rows
  followed by the block rows.
- Softmax-max over 1024 rows of the 126464-word vocabulary: x0 is the first
  index of the row maximum (no logit is within 2^-6 of a maximum above 2),
  x0_p is bf16(1 / sum exp(l - max)) with the sum taken in f64 by torch.
Tolerances: attention max-abs 2e-2 and mean-abs 2e-3 between two bf16
computations of the same rows; x0_p within one bf16 unit."""
import numpy as np
import pytest
import torch

from helpers import MAX_ABS, MEAN_ABS
from dllm_serve_amd import _capi

pytestmark = pytest.mark.gpu

D = 128


def _varlen(q, k, v, cu_q, cu_k, n_seg, max_q, max_k, seg_ids=None, o=None):
    o = torch.zeros_like(q) if o is None else o
    _capi.attn_varlen_fwd(q, k, v, o, cu_q, cu_k, seg_ids, n_seg, max_q, D ** -0.5, max_seqlen_k=max_k)
    torch.cuda.synchronize()
    return o


def _close(a, b, what):
    d = (a.float() - b.float()).abs()
    mx, mean = d.max().item(), d.mean().item()
    assert torch.isfinite(a.float()).all() and torch.isfinite(b.float()).all(), f"{what}: non-finite"
    assert mx <= MAX_ABS and mean <= MEAN_ABS, f"{what}: max-abs {mx:.3e} mean-abs {mean:.3e}"


def test_c2_step_segments_are_independent(dev):
    print("full size: C2 dense step 8 x 384, 32 heads, subsets and one segment alone", flush=True)
    lens, H = [384] * 8, 32
    g = torch.Generator(device=dev).manual_seed(11)
    q, k, v = (torch.randn(sum(lens), H, D, generator=g, device=dev, dtype=torch.bfloat16) for _ in range(3))
    cu = torch.arange(0, 9 * 384, 384, dtype=torch.int32, device=dev)
    full = _varlen(q, k, v, cu, cu, 8, 384, 384)
    for subset in ([0, 2, 5, 7, 1], [3]):   # 160 (segment, head) pairs: 12-wavefront launch; 32: 4-wavefront
        ids = torch.tensor(subset, dtype=torch.int32, device=dev)
        part = _varlen(q, k, v, cu, cu, len(subset), 384, 384, seg_ids=ids, o=torch.full_like(q, 7.0))
        for sgm in range(8):
            rows = slice(384 * sgm, 384 * (sgm + 1))
            if sgm in subset:
                assert torch.equal(part[rows], full[rows]), f"segment {sgm} of subset {subset} differs"
            else:
                assert torch.all(part[rows] == 7.0), f"segment {sgm} outside subset {subset} was written"


def test_c2_step_key_permutation(dev):
    print("full size: C2 dense step 8 x 384, keys of segment 4 permuted", flush=True)
    lens, H = [384] * 8, 32
    g = torch.Generator(device=dev).manual_seed(12)
    q, k, v = (torch.randn(sum(lens), H, D, generator=g, device=dev, dtype=torch.bfloat16) for _ in range(3))
    cu = torch.arange(0, 9 * 384, 384, dtype=torch.int32, device=dev)
    base = _varlen(q, k, v, cu, cu, 8, 384, 384)
    perm = torch.arange(sum(lens), device=dev)
    perm[4 * 384:5 * 384] = 4 * 384 + torch.randperm(384, generator=torch.Generator().manual_seed(3)).to(dev)
    out = _varlen(q, k[perm].contiguous(), v[perm].contiguous(), cu, cu, 8, 384, 384)
    _close(out, base, "permuted keys of segment 4")
    other = torch.cat([base[:4 * 384], base[5 * 384:]]), torch.cat([out[:4 * 384], out[5 * 384:]])
    assert torch.equal(other[0], other[1]), "segments whose keys did not move changed"


def test_dream_gqa_equals_repeated_kv(dev):
    print("full size: Dream GQA 28/4, 16 ragged segments, vs K/V repeated to 28 heads", flush=True)
    lens = [725, 1101, 710, 1245, 604, 570, 751, 682, 544, 609, 890, 1175, 933, 600, 979, 410]
    Hq, Hkv = 28, 4
    g = torch.Generator(device=dev).manual_seed(13)
    n = sum(lens)
    q = torch.randn(n, Hq, D, generator=g, device=dev, dtype=torch.bfloat16)
    k = torch.randn(n, Hkv, D, generator=g, device=dev, dtype=torch.bfloat16)
    v = torch.randn(n, Hkv, D, generator=g, device=dev, dtype=torch.bfloat16)
    cu = torch.tensor([0] + np.cumsum(lens).tolist(), dtype=torch.int32, device=dev)
    gqa = _varlen(q, k, v, cu, cu, len(lens), max(lens), max(lens))
    k_rep = k.repeat_interleave(Hq // Hkv, dim=1).contiguous()
    v_rep = v.repeat_interleave(Hq // Hkv, dim=1).contiguous()
    rep = _varlen(q, k_rep, v_rep, cu, cu, len(lens), max(lens), max(lens))
    assert torch.equal(gqa, rep), "GQA rows differ from the repeated-K/V rows"


def test_c5_round_trip_and_block_cached_equals_gathered_dense(dev):
    print("full size: C5 32 x 32-token blocks vs 2048..4096 cached rows", flush=True)
    Hq = Hkv = 32
    page, blk, B = 256, 32, 32
    rng = np.random.default_rng(5)
    prefix = rng.integers(2048, 4097, B).tolist()
    pages_per = [-(-p // page) for p in prefix]
    free = rng.permutation(sum(pages_per)).tolist()
    slots, at = [], 0
    for p, npg in zip(prefix, pages_per):
        s = []
        for j, pid in enumerate(free[at:at + npg]):
            fill = page if j < npg - 1 else p - page * (npg - 1)
            s.extend(range(pid * page, pid * page + fill))
        at += npg
        slots.append(s)
    n_pre, row = sum(prefix), Hkv * D
    g = torch.Generator(device=dev).manual_seed(14)
    k_pre = torch.randn(n_pre, Hkv, D, generator=g, device=dev, dtype=torch.bfloat16)
    v_pre = torch.randn(n_pre, Hkv, D, generator=g, device=dev, dtype=torch.bfloat16)
    q = torch.randn(B * blk, Hq, D, generator=g, device=dev, dtype=torch.bfloat16)
    k = torch.randn(B * blk, Hkv, D, generator=g, device=dev, dtype=torch.bfloat16)
    v = torch.randn(B * blk, Hkv, D, generator=g, device=dev, dtype=torch.bfloat16)
    flat = torch.tensor([x for s in slots for x in s], dtype=torch.int32, device=dev)
    kc = torch.zeros(sum(pages_per) * page, Hkv, D, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    _capi.store_kvcache(k_pre, v_pre, kc, vc, flat, n_pre, row)
    k_back, v_back = torch.empty_like(k_pre), torch.empty_like(v_pre)
    _capi.load_kvcache(k_back, v_back, kc, vc, flat, n_pre, row)
    torch.cuda.synchronize()
    assert torch.equal(k_back, k_pre) and torch.equal(v_back, v_pre), "store -> load round trip"

    off = torch.tensor([0] + np.cumsum(prefix).tolist(), dtype=torch.int32, device=dev)
    cu_q = torch.arange(0, (B + 1) * blk, blk, dtype=torch.int32, device=dev)
    max_keys = max(prefix) + blk
    ws_b = _capi.block_cached_workspace_size(B, blk, max_keys, Hq, Hkv, D)
    ws = torch.empty(max(ws_b, 16), dtype=torch.uint8, device=dev) if ws_b else None
    o_cached = torch.zeros_like(q)
    _capi.attn_block_cached_fwd(q, k, v, o_cached, cu_q, None, B, blk, max_keys, kc, vc, flat, off, D ** -0.5, ws)
    # dense attention over [gathered prefix rows ; block rows] of every segment
    ks, vs, lk = [], [], []
    for b in range(B):
        a0, a1 = int(off[b]), int(off[b + 1])
        ks += [k_back[a0:a1], k[b * blk:(b + 1) * blk]]
        vs += [v_back[a0:a1], v[b * blk:(b + 1) * blk]]
        lk.append(a1 - a0 + blk)
    k_cat, v_cat = torch.cat(ks).contiguous(), torch.cat(vs).contiguous()
    cu_k = torch.tensor([0] + np.cumsum(lk).tolist(), dtype=torch.int32, device=dev)
    o_dense = _varlen(q, k_cat, v_cat, cu_q, cu_k, B, blk, max(lk))
    _close(o_cached, o_dense, "C5 block-cached vs gathered dense")


def test_softmax_max_llada_vocab_rows(dev):
    print("full size: softmax-max of 1024 x 126464 bf16 logits", flush=True)
    M, V = 1024, 126464
    g = torch.Generator(device=dev).manual_seed(15)
    logits = (torch.randn(M, V, generator=g, device=dev) * 1.3 + 3.0).to(torch.bfloat16)
    x0 = torch.empty(M, dtype=torch.int64, device=dev)
    x0_p = torch.empty(M, dtype=torch.bfloat16, device=dev)
    _capi.softmax_max(logits, x0, x0_p)
    torch.cuda.synchronize()
    lf = logits.double()
    mx = lf.max(dim=1, keepdim=True).values
    assert bool((mx.squeeze(1) > 2.0).all()), "every row maximum must exceed 2 for the closed form"
    idx = torch.arange(V, device=dev).expand(M, V)
    first = torch.where(lf == mx, idx, torch.full_like(idx, V)).min(dim=1).values
    assert torch.equal(x0, first), "x0 is not the first index of the row maximum"
    want = (1.0 / torch.exp(lf - mx).sum(dim=1)).float().to(torch.bfloat16)
    got_b = x0_p.view(torch.int16).int()
    want_b = want.view(torch.int16).int()
    assert int((got_b - want_b).abs().max()) <= 1, "x0_p more than one bf16 unit from bf16(1 / sum exp)"
