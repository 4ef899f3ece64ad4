"""Seeded random shapes for every kernel entry point, against the oracle.

Each case prints its parameters before it runs.  Attention outputs are held
to the bf16 tolerance (max-abs 2e-2, mean-abs 2e-3 against fp32 on the same
bf16 inputs); RoPE, selection and cache contents are bit-exact."""
import numpy as np
import pytest
import torch

from helpers import assert_attn_close, bits, to_np

from oracle import attention as oatt
from oracle import configs
from oracle import rope as orope
from oracle import select as osel
from oracle.bf16 import bf16_bits_to_f32
from dllm_serve_amd import _capi

pytestmark = pytest.mark.gpu

HEADS = [(8, 8), (8, 2), (16, 4), (28, 4), (32, 32), (14, 2), (16, 16), (4, 1)]


def _dense_cases(n=24, seed=2024):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        Hq, Hkv = HEADS[rng.integers(len(HEADS))]
        g = Hq // Hkv
        mode = rng.integers(3)
        if mode == 0:      # short segments, any length
            lens = rng.integers(1, 200, rng.integers(1, 6)).tolist()
        elif mode == 1:    # around the one-workgroup-per-pair sizes (257..384 M rows)
            lens = [int(max(1, x)) for x in rng.integers(257 // g, 384 // g + 1, rng.integers(1, 5))]
        else:              # longer
            lens = rng.integers(100, 700, rng.integers(1, 4)).tolist()
        subset = None
        if len(lens) > 2 and rng.random() < 0.4:
            subset = sorted(rng.choice(len(lens), size=len(lens) - 1, replace=False).tolist())
        out.append((i, lens, Hq, Hkv, subset))
    return out


@pytest.mark.parametrize("case", _dense_cases(), ids=lambda c: f"d{c[0]}")
def test_fuzz_varlen(dev, case):
    i, lens, Hq, Hkv, subset = case
    print(f"fuzz varlen {i}: lens={lens} Hq={Hq} Hkv={Hkv} subset={subset}", flush=True)
    q, k, v, cu = configs.packed_qkv(lens, Hq, Hkv, 128, seed=1000 + i)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    o = torch.full_like(qd, 3.0)
    ids = None if subset is None else torch.tensor(subset, dtype=torch.int32, device=dev)
    segs = list(range(len(lens))) if subset is None else subset
    _capi.attn_varlen_fwd(qd, kd, vd, o, cu.to(dev), cu.to(dev), ids, len(segs),
                          max(lens[s] for s in segs), 128 ** -0.5)
    torch.cuda.synchronize()
    cul = cu.tolist()
    qn, kn, vn = to_np(q), to_np(k), to_np(v)
    for s in range(len(lens)):
        r0, r1 = cul[s], cul[s + 1]
        if s in segs:
            ref = oatt.segment(qn[r0:r1], kn[r0:r1], vn[r0:r1], 128 ** -0.5, dtype=np.float32)
            assert_attn_close(o[r0:r1], ref, f"case {i} seg {s}")
        else:
            assert torch.all(o[r0:r1] == 3.0), f"case {i}: segment {s} outside the subset was written"


def _cached_cases(n=12, seed=77):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        Hq, Hkv = HEADS[rng.integers(len(HEADS))]
        nseg = int(rng.integers(1, 5))
        prefix = rng.integers(0, 1500, nseg).tolist()
        blk = rng.integers(1, 65, nseg).tolist()
        bad = bool(rng.random() < 0.3)
        out.append((i, prefix, blk, Hq, Hkv, bad))
    return out


@pytest.mark.parametrize("case", _cached_cases(), ids=lambda c: f"c{c[0]}")
def test_fuzz_block_cached(dev, case):
    i, prefix, blk, Hq, Hkv, bad = case
    print(f"fuzz cached {i}: prefix={prefix} blk={blk} Hq={Hq} Hkv={Hkv} bad_slots={bad}", flush=True)
    g = torch.Generator().manual_seed(500 + i)
    D, page = 128, 256
    pages_per = [-(-p // page) for p in prefix]
    n_pages = sum(pages_per) + 2
    perm = torch.randperm(n_pages, generator=g).tolist()
    kc = torch.randn(n_pages * page, Hkv, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(n_pages * page, Hkv, D, generator=g).to(torch.bfloat16)
    slots, at = [], 0
    for p, npg in zip(prefix, pages_per):
        s = []
        for j in range(npg):
            fill = page if j < npg - 1 else p - page * (npg - 1)
            s.extend(range(perm[at + j] * page, perm[at + j] * page + fill))
        at += npg
        if bad and s:
            s[len(s) // 2] = -1
        slots.append(s)
    q, k, v, cu = configs.packed_qkv(blk, Hq, Hkv, D, seed=600 + i)
    off = [0]
    for s in slots:
        off.append(off[-1] + len(s))
    flat = torch.tensor([x for s in slots for x in s] or [0], dtype=torch.int32)
    max_keys = max(p + b for p, b in zip(prefix, blk))
    ws_b = _capi.block_cached_workspace_size(len(blk), max(blk), max_keys, Hq, Hkv, D)
    ws = torch.empty(max(ws_b, 1), dtype=torch.uint8, device=dev) if ws_b else None
    o = torch.zeros(q.shape, dtype=torch.bfloat16, device=dev)
    _capi.attn_block_cached_fwd(q.to(dev), k.to(dev), v.to(dev), o, cu.to(dev), None, len(blk), max(blk), max_keys,
                                kc.to(dev), vc.to(dev), flat.to(dev), torch.tensor(off, dtype=torch.int32, device=dev),
                                D ** -0.5, ws)
    torch.cuda.synchronize()
    cul = cu.tolist()
    for s in range(len(blk)):
        r0, r1 = cul[s], cul[s + 1]
        ref = oatt.block_cached(to_np(q)[r0:r1], to_np(k)[r0:r1], to_np(v)[r0:r1], to_np(kc), to_np(vc), slots[s],
                                D ** -0.5, dtype=np.float32)
        assert_attn_close(o[r0:r1], ref, f"case {i} seg {s}")


def _rope_cases(n=10, seed=31):
    rng = np.random.default_rng(seed)
    return [(i, int(rng.integers(1, 400)), int(rng.integers(1, 40)), int(rng.integers(0, 9)),
             int(rng.choice([16, 64, 128, 256])), int(rng.integers(0, 3)) * 8) for i in range(n)]


@pytest.mark.parametrize("case", _rope_cases(), ids=lambda c: f"r{c[0]}")
def test_fuzz_rope(dev, case):
    i, n, Hq, Hkv, D, pad = case
    print(f"fuzz rope {i}: n={n} Hq={Hq} Hkv={Hkv} D={D} pad={pad}", flush=True)
    g = torch.Generator().manual_seed(900 + i)
    base = torch.randn(n, (Hq + Hkv) * D + pad, generator=g).to(torch.bfloat16).to(dev)
    q, k = base[:, :Hq * D], base[:, Hq * D:(Hq + Hkv) * D]
    maxp = 2048
    inv = 1.0 / (10000.0 ** (torch.arange(0, D, 2, dtype=torch.float) / D))
    freqs = torch.einsum("i,j -> ij", torch.arange(maxp, dtype=torch.float), inv)
    table = torch.cat((freqs.cos(), freqs.sin()), dim=-1)
    pos = torch.randint(0, maxp, (n,), generator=g)
    qo = torch.empty(n, Hq * D, dtype=torch.bfloat16, device=dev)
    ko = torch.empty(n, Hkv * D, dtype=torch.bfloat16, device=dev)
    _capi.rope_neox(q, qo, k, ko, pos.to(dev), table.to(dev), n, Hq, Hkv, D)
    torch.cuda.synchronize()
    tn = table.numpy()
    assert np.array_equal(bits(qo).reshape(n, Hq, D), orope.rotate_table(to_np(q).reshape(n, Hq, D), pos.numpy(), tn))
    if Hkv:
        assert np.array_equal(bits(ko).reshape(n, Hkv, D),
                              orope.rotate_table(to_np(k).reshape(n, Hkv, D), pos.numpy(), tn))


def _select_cases(n=8, seed=55):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        Hq, Hkv = HEADS[rng.integers(len(HEADS))]
        Lb = int(rng.integers(1, 48))
        Kc = int(rng.integers(0, 900))
        ratio = float(rng.choice([0.1, 0.3, 0.5, 0.75, 1.0]))
        out.append((i, Lb, Kc, Hq, Hkv, ratio, bool(rng.random() < 0.6), int(rng.integers(1, 6))))
    return out


# A raw score whose f64 sum (8.65625000006) rounds to f32 exactly onto a bf16
# midpoint: the two-step rule gives 8.625, a single f64 -> bf16 rounding 8.6875
# (candidate 340 of KV head 3 then moved ahead of two higher-ranked ones).
SELECT_REGRESSIONS = [(3, 4, 643, 16, 4, 0.75, True, 1)]


@pytest.mark.parametrize("case", _select_cases() + SELECT_REGRESSIONS, ids=lambda c: f"s{c[0]}-{c[2]}")
def test_fuzz_select_store(dev, case):
    i, Lb, Kc, Hq, Hkv, ratio, hs, pk = case
    n_keep = min(max(1, int(Kc * ratio)), Kc)
    print(f"fuzz select {i}: Lb={Lb} Kc={Kc} Hq={Hq} Hkv={Hkv} n_keep={n_keep} head_select={hs} pool={pk}",
          flush=True)
    if n_keep == 0:
        pytest.skip("no candidates")
    rng = np.random.default_rng(700 + i)
    D = 128
    blk_start = int(rng.integers(0, Kc + 1))
    n_tok = Lb + Kc
    q = torch.randn(n_tok, Hq, D, generator=torch.Generator().manual_seed(i)).to(torch.bfloat16)
    k = torch.randn(n_tok, Hkv, D, generator=torch.Generator().manual_seed(i + 1)).to(torch.bfloat16)
    v = torch.randn(n_tok, Hkv, D, generator=torch.Generator().manual_seed(i + 2)).to(torch.bfloat16)
    cand = np.r_[0:blk_start, blk_start + Lb:n_tok]
    qb = bf16_bits_to_f32(bits(q[blk_start:blk_start + Lb]))
    kcand = bf16_bits_to_f32(bits(k))[cand]
    want = osel.select(qb, kcand, n_keep, hs, pk, np.float32(D ** 0.5))
    pages = -(-n_keep // 256) + 1
    cache = torch.zeros(2, pages * 256, Hkv, D, dtype=torch.bfloat16, device=dev)
    slots = torch.randperm(pages * 256, generator=torch.Generator().manual_seed(i))[:n_keep].to(torch.int32)
    jobs = torch.tensor([[0, n_tok, blk_start, Lb, n_keep, 0, int(hs), pk]], dtype=torch.int32, device=dev)
    idx = torch.full((1, Hkv, n_keep), -1, dtype=torch.int64, device=dev)
    ws = torch.empty(max(16, _capi.select_workspace_size(1, Kc, Hq, Hkv, D)), dtype=torch.uint8, device=dev)
    _capi.select_kv_store(q.to(dev), k.to(dev), v.to(dev), jobs, 1, Kc, n_keep, np.float32(D ** 0.5),
                          cache[0], cache[1], slots.to(dev), idx, ws)
    torch.cuda.synchronize()
    got = idx.cpu().numpy()[0] if hs else idx.cpu().numpy()[0][:1]
    assert np.array_equal(got, want if hs else want[None, :]), f"case {i}: indices"
    kc, vc = cache[0].cpu(), cache[1].cpu()
    sl = slots.long()
    for h in range(Hkv):
        sel = cand[(want[h] if hs else want)]
        assert torch.equal(kc[sl, h], k[sel, h]) and torch.equal(vc[sl, h], v[sel, h]), f"case {i}: cache head {h}"
