"""K3a (dense varlen bidirectional) and K3b (block vs cached KV) on the GPU vs
the fp32 oracle.  Tolerance (bf16 output vs fp32 reference on the same bf16
inputs): max-abs <= 2e-2 and mean-abs <= 2e-3 (helpers.MAX_ABS / MEAN_ABS)."""
import numpy as np
import pytest
import torch

from helpers import assert_attn_close, to_np

from oracle import attention as oatt
from oracle import configs
from dllm_serve_amd import _capi

pytestmark = pytest.mark.gpu


def _run_varlen(q, k, v, cu, dev, seg_ids=None, o_init=None):
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    o = torch.zeros_like(qd) if o_init is None else o_init.to(dev)
    cud = cu.to(dev)
    lens = (cu[1:] - cu[:-1]).tolist()
    ids = None
    n_seg = len(lens)
    if seg_ids is not None:
        ids = torch.tensor(seg_ids, dtype=torch.int32, device=dev)
        n_seg = len(seg_ids)
        lens = [lens[i] for i in seg_ids]
    _capi.attn_varlen_fwd(qd, kd, vd, o, cud, cud, ids, n_seg, max(lens), q.shape[-1] ** -0.5)
    torch.cuda.synchronize()
    return o


def test_c1_single_layer(dev):
    """C1 shape (1 x 512 tokens, 32 heads x 128, RoPE'd), bf16 on the GPU."""
    print("varlen C1 512x32x128", flush=True)
    q, k, v, cu, scale = configs.c1_single_layer()
    qb, kb, vb = q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16)
    o = _run_varlen(qb, kb, vb, cu, dev)
    ref = oatt.varlen(to_np(qb), to_np(kb), to_np(vb), cu.numpy(), cu.numpy(), scale, dtype=np.float32)
    assert_attn_close(o, ref, "C1")


@pytest.mark.parametrize("lens,Hq,Hkv", [
    ([1, 7, 33, 64, 127, 128, 129, 300], 32, 32),     # ragged MHA, tails everywhere
    ([384] * 4, 32, 32),                               # C2 dense step shape (4 of the 8 sequences)
    ([200, 517, 1], 28, 4),                            # Dream GQA, g = 7
    ([96, 160], 8, 2),                                 # g = 4
    ([1000], 4, 4),
    ([300, 384, 1, 257, 383], 32, 32),               # 257..384 M rows, 160 pairs: one 12-wavefront workgroup each
    ([64, 96, 7, 90] * 10, 16, 4),                     # the same launch with GQA (96 x 4 = 384 M rows, 160 pairs)
    ([300, 384, 1, 257, 383], 16, 16),               # the same rows, 80 pairs: three 4-wavefront workgroups each
    ([500, 33, 1], 32, 1),                             # MQA, g = 32: one KV row serves 32 M rows
    ([260, 7], 64, 1),                                 # g = 64
])
def test_varlen_ragged(dev, lens, Hq, Hkv):
    print(f"varlen lens={lens} Hq={Hq} Hkv={Hkv}", flush=True)
    q, k, v, cu = configs.packed_qkv(lens, Hq, Hkv, 128, seed=sum(lens))
    o = _run_varlen(q, k, v, cu, dev)
    ref = oatt.varlen(to_np(q), to_np(k), to_np(v), cu.numpy(), cu.numpy(), 128 ** -0.5, dtype=np.float32)
    assert_attn_close(o, ref, f"lens={lens}")


@pytest.mark.parametrize("lens,Hq,Hkv", [
    ([2100, 300, 2048], 16, 16),      # >= 2048 keys: 8-wavefront launch, ragged last tile
    ([2500, 37], 28, 4),              # Dream GQA on the 8-wavefront launch
])
def test_varlen_long_key_streams(dev, lens, Hq, Hkv):
    print(f"varlen long lens={lens} Hq={Hq} Hkv={Hkv}", flush=True)
    q, k, v, cu = configs.packed_qkv(lens, Hq, Hkv, 128, seed=sum(lens) + Hq)
    o = _run_varlen(q, k, v, cu, dev)
    ref = oatt.varlen(to_np(q), to_np(k), to_np(v), cu.numpy(), cu.numpy(), 128 ** -0.5, dtype=np.float32)
    assert_attn_close(o, ref, f"lens={lens}")


@pytest.mark.parametrize("lens,Hq,Hkv", [
    ([150, 129, 191, 5] * 5, 16, 8),   # g = 2; 382 M rows, 160 (segment, KV head) pairs: 12-wavefront launch
    ([100, 128, 86, 1] * 5, 24, 8),    # g = 3, 384 M rows
    ([52, 76, 60, 3] * 5, 40, 8),      # g = 5, 380 M rows
    ([43, 64, 50, 2] * 5, 48, 8),      # g = 6, 384 M rows
    ([33, 48, 40, 1] * 5, 64, 8),      # g = 8, 384 M rows
    ([2100, 37], 3, 1),                # g = 3, keys >= 2048: 8-wavefront launch
    ([2050, 300], 5, 1),               # g = 5, the same
])
def test_varlen_gqa_ratios_on_the_cu_owning_launches(dev, lens, Hq, Hkv):
    """The 12- and 8-wavefront launches stage Q through LDS: M row m is token
    m / g, head hkv * g + m % g for every group size, rows past a segment read
    zero."""
    print(f"varlen gqa lens={lens} Hq={Hq} Hkv={Hkv}", flush=True)
    q, k, v, cu = configs.packed_qkv(lens, Hq, Hkv, 128, seed=7 * sum(lens) + Hq)
    o = _run_varlen(q, k, v, cu, dev)
    ref = oatt.varlen(to_np(q), to_np(k), to_np(v), cu.numpy(), cu.numpy(), 128 ** -0.5, dtype=np.float32)
    assert_attn_close(o, ref, f"lens={lens} Hq={Hq} Hkv={Hkv}")


@pytest.mark.parametrize("lq,lk", [([40, 7, 300], [100, 2200, 5]), ([128, 64], [64, 128]),
                                   ([5, 40, 9], [0, 70, 0])])   # segments without keys give zero rows
def test_varlen_different_q_and_k_lengths(dev, lq, lk):
    """cu_seqlens_q != cu_seqlens_k, as flash_attn_varlen_func allows."""
    print(f"varlen lq={lq} lk={lk}", flush=True)
    H, D = 8, 128
    g = torch.Generator().manual_seed(sum(lq) + sum(lk))
    q = torch.randn(sum(lq), H, D, generator=g).to(torch.bfloat16)
    k = torch.randn(sum(lk), H, D, generator=g).to(torch.bfloat16)
    v = torch.randn(sum(lk), H, D, generator=g).to(torch.bfloat16)
    cu_q = torch.tensor([0] + list(np.cumsum(lq)), dtype=torch.int32)
    cu_k = torch.tensor([0] + list(np.cumsum(lk)), dtype=torch.int32)
    o = torch.zeros(sum(lq), H, D, dtype=torch.bfloat16, device=dev)
    _capi.attn_varlen_fwd(q.to(dev), k.to(dev), v.to(dev), o, cu_q.to(dev), cu_k.to(dev), None, len(lq), max(lq),
                          D ** -0.5, max_seqlen_k=max(lk))
    torch.cuda.synchronize()
    ref = oatt.varlen(to_np(q), to_np(k), to_np(v), cu_q.numpy(), cu_k.numpy(), D ** -0.5, dtype=np.float32)
    assert_attn_close(o, ref, f"lq={lq} lk={lk}")


def test_varlen_subset_leaves_other_rows(dev):
    """seg_ids runs only some segments in place; other rows keep their contents."""
    print("varlen seg_ids subset", flush=True)
    lens = [50, 70, 90, 30]
    q, k, v, cu = configs.packed_qkv(lens, 16, 16, 128, seed=5)
    sentinel = torch.full_like(q, 3.0)
    o = _run_varlen(q, k, v, cu, dev, seg_ids=[1, 3], o_init=sentinel)
    ref = oatt.varlen(to_np(q), to_np(k), to_np(v), cu.numpy(), cu.numpy(), 128 ** -0.5, dtype=np.float32,
                      seg_ids=[1, 3])
    cu_l = cu.tolist()
    for s in (1, 3):
        assert_attn_close(o[cu_l[s]:cu_l[s + 1]], ref[cu_l[s]:cu_l[s + 1]], f"seg {s}")
    for s in (0, 2):
        assert torch.all(o[cu_l[s]:cu_l[s + 1]].cpu() == 3.0)


def test_varlen_strided_views(dev):
    """q/k/v as column slices of one merged qkv projection (token stride > row)."""
    print("varlen strided views", flush=True)
    Hq, Hkv, D = 28, 4, 128
    lens = [150, 260]
    n = sum(lens)
    g = torch.Generator().manual_seed(11)
    qkv = torch.randn(n, (Hq + 2 * Hkv) * D, generator=g).to(torch.bfloat16).to(dev)
    q = qkv[:, :Hq * D].view(n, Hq, D)
    k = qkv[:, Hq * D:(Hq + Hkv) * D].view(n, Hkv, D)
    v = qkv[:, (Hq + Hkv) * D:].view(n, Hkv, D)
    cu = torch.tensor([0, lens[0], n], dtype=torch.int32)
    o = torch.zeros(n, Hq, D, dtype=torch.bfloat16, device=dev)
    _capi.attn_varlen_fwd(q, k, v, o, cu.to(dev), cu.to(dev), None, 2, max(lens), D ** -0.5)
    torch.cuda.synchronize()
    ref = oatt.varlen(to_np(q), to_np(k), to_np(v), cu.numpy(), cu.numpy(), D ** -0.5, dtype=np.float32)
    assert_attn_close(o, ref, "strided")


@pytest.mark.parametrize("lens,Hq,Hkv,pad", [
    ([150, 260, 1], 8, 2, 8),               # 4-wavefront launch
    ([300, 384, 1, 257, 383] * 2, 16, 16, 24),  # 160 pairs of 257..384 M rows: 12-wavefront launch
    ([2100, 40], 4, 4, 8),                  # key streams >= 2048: 8-wavefront launch
])
def test_varlen_token_strides_not_multiple_of_256_bytes(dev, lens, Hq, Hkv, pad):
    """Rows padded by a multiple of 8 elements that is not a multiple of 128,
    so a token's K row does not start on a 256-byte boundary: the K tile's
    chunk swizzle must act on the chunk alone (an XOR over row offset + chunk
    reads the wrong 16 bytes, or the next token's)."""
    print(f"varlen token strides +{pad} lens={lens} Hq={Hq} Hkv={Hkv}", flush=True)
    D = 128
    q, k, v, cu = configs.packed_qkv(lens, Hq, Hkv, D, seed=len(lens) + pad)
    n = q.shape[0]

    def padded(t, H):
        buf = torch.full((n, H * D + pad), float("nan"), dtype=torch.bfloat16)
        buf[:, :H * D] = t.reshape(n, H * D)
        return buf.to(dev)[:, :H * D].view(n, H, D)

    qd, kd, vd = padded(q, Hq), padded(k, Hkv), padded(v, Hkv)
    assert kd.stride(0) == Hkv * D + pad and (kd.stride(0) * 2) % 256 != 0
    obuf = torch.full((n, Hq * D + pad), 7.0, dtype=torch.bfloat16, device=dev)
    o = obuf[:, :Hq * D].view(n, Hq, D)
    _capi.attn_varlen_fwd(qd, kd, vd, o, cu.to(dev), cu.to(dev), None, len(lens), max(lens), D ** -0.5)
    torch.cuda.synchronize()
    ref = oatt.varlen(to_np(q), to_np(k), to_np(v), cu.numpy(), cu.numpy(), D ** -0.5, dtype=np.float32)
    assert_attn_close(o, ref, f"stride +{pad}")
    assert torch.all(obuf[:, Hq * D:].float() == 7.0), "padding between output rows was written"


def test_varlen_bad_head_dim_raises(dev):
    q = torch.zeros(8, 4, 64, dtype=torch.bfloat16, device=dev)
    cu = torch.tensor([0, 8], dtype=torch.int32, device=dev)
    with pytest.raises(RuntimeError, match="head_dim"):
        _capi.attn_varlen_fwd(q, q, q, torch.empty_like(q), cu, cu, None, 1, 8, 0.125)


def _cached_case(prefix, blk, Hq, Hkv, seed, page=256, extra_pages=3):
    """Cache with shuffled pages; per sequence `prefix[i]` cached rows and a
    block of `blk[i]` rows."""
    g = torch.Generator().manual_seed(seed)
    D = 128
    pages_per = [-(-p // page) for p in prefix]
    n_pages = sum(pages_per) + extra_pages
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


@pytest.mark.parametrize("prefix,blk,Hq,Hkv", [
    ([608, 608, 608, 608], [64, 64, 64, 64], 32, 32),     # C4 reuse step (n_keep 608, block 64)
    ([2100, 3000, 4096], [32, 32, 32], 32, 32),            # C5-like long prefixes
    ([5, 300], [32, 17], 28, 4),                           # Dream GQA, short block tail
    ([0, 1], [8, 3], 8, 8),                                # empty / single cached row
    ([2100 + 13 * i for i in range(32)], [32] * 32, 8, 8),  # 256 pairs: one workgroup per pair, no split
    ([700] * 16, [32] * 16, 28, 4),                        # Dream denoise step: 448 M tiles, paired row blocks
    ([300, 1000, 0], [32, 16, 5], 32, 1),                  # MQA, g = 32: 32 M tiles per segment, paired row blocks
    ([257, 40], [3, 9], 64, 1),                            # g = 64, blocks of a few rows
])
def test_block_cached(dev, prefix, blk, Hq, Hkv):
    print(f"block_cached prefix={prefix} blk={blk} Hq={Hq} Hkv={Hkv}", flush=True)
    q, k, v, cu, kc, vc, slots = _cached_case(prefix, blk, Hq, Hkv, seed=sum(prefix) + 1)
    D = 128
    slot_off = [0]
    for s in slots:
        slot_off.append(slot_off[-1] + len(s))
    flat_slots = torch.tensor([x for s in slots for x in s] or [0], dtype=torch.int32)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    o = torch.zeros_like(qd)
    max_keys = max(p + b for p, b in zip(prefix, blk))
    ws_bytes = _capi.block_cached_workspace_size(len(blk), max(blk), max_keys, Hq, Hkv, D)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev) if ws_bytes else None
    _capi.attn_block_cached_fwd(qd, kd, vd, o, cu.to(dev), None, len(blk), max(blk), max_keys,
                                kc.to(dev), vc.to(dev), flat_slots.to(dev),
                                torch.tensor(slot_off, dtype=torch.int32, device=dev), D ** -0.5, ws)
    torch.cuda.synchronize()
    kcn, vcn = to_np(kc), to_np(vc)
    cul = cu.tolist()
    qn, kn, vn = to_np(q), to_np(k), to_np(v)
    for i in range(len(blk)):
        r0, r1 = cul[i], cul[i + 1]
        ref = oatt.block_cached(qn[r0:r1], kn[r0:r1], vn[r0:r1], kcn, vcn, slots[i], D ** -0.5, dtype=np.float32)
        assert_attn_close(o[r0:r1], ref, f"seq {i}")


def test_block_cached_paired_row_blocks_ragged(dev):
    """Two 32-row blocks per workgroup (more than one generation of
    single-block workgroups): ragged blocks of 1..32 tokens with 7 query
    heads per KV head (2..7 M tiles, odd counts leave a workgroup's second
    block empty), empty and short prefixes, and slots outside the cache."""
    blk = [32, 17, 5, 1, 32, 31, 9, 32, 24, 32, 2, 32, 32, 13, 32, 28, 32, 7, 32, 32]
    prefix = [700, 0, 1, 255, 256, 257, 900, 33, 512, 640, 3, 700, 128, 380, 777, 64, 1000, 90, 300, 450]
    Hq, Hkv = 28, 4
    mt = [-(-b * 7 // 32) for b in blk]
    assert len(blk) * Hkv * max(mt) > 512, "meant for the paired launch"
    print(f"block_cached paired row blocks: {len(blk)} segments, ragged", flush=True)
    q, k, v, cu, kc, vc, slots = _cached_case(prefix, blk, Hq, Hkv, seed=5)
    slots[0][3] = -1
    slots[8][511] = kc.shape[0]
    slots[16][500] = 2 ** 31 - 1
    D = 128
    slot_off = [0]
    for s_ in slots:
        slot_off.append(slot_off[-1] + len(s_))
    flat = torch.tensor([x for s_ in slots for x in s_], dtype=torch.int32)
    o = torch.full(q.shape, float("nan"), dtype=torch.bfloat16, device=dev)
    max_keys = max(p + b for p, b in zip(prefix, blk))
    ws_bytes = _capi.block_cached_workspace_size(len(blk), max(blk), max_keys, Hq, Hkv, D)
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=dev) if ws_bytes else None
    _capi.attn_block_cached_fwd(q.to(dev), k.to(dev), v.to(dev), o, cu.to(dev), None, len(blk), max(blk), max_keys,
                                kc.to(dev), vc.to(dev), flat.to(dev),
                                torch.tensor(slot_off, dtype=torch.int32, device=dev), D ** -0.5, ws)
    torch.cuda.synchronize()
    assert not torch.isnan(o).any(), "rows left unwritten"
    kcn, vcn = to_np(kc), to_np(vc)
    cul = cu.tolist()
    qn, kn, vn = to_np(q), to_np(k), to_np(v)
    for i in range(len(blk)):
        r0, r1 = cul[i], cul[i + 1]
        ref = oatt.block_cached(qn[r0:r1], kn[r0:r1], vn[r0:r1], kcn, vcn, slots[i], D ** -0.5, dtype=np.float32)
        assert_attn_close(o[r0:r1], ref, f"seq {i}")


@pytest.mark.parametrize("prefix,Hq,Hkv", [([300, 700], 8, 8), ([2100 + 7 * i for i in range(32)], 8, 8)])
def test_block_cached_without_a_cache(dev, prefix, Hq, Hkv):
    """cache_slots = 0 (no cache tensor, no slots): every cached row is
    outside the cache, so the blocks attend to themselves only."""
    print(f"block_cached without a cache: {len(prefix)} segments", flush=True)
    D = 128
    blk = [32] * len(prefix)
    q, k, v, cu = configs.packed_qkv(blk, Hq, Hkv, D, seed=len(prefix))
    off = torch.tensor([0] + np.cumsum(prefix).tolist(), dtype=torch.int32, device=dev)
    max_keys = max(prefix) + 32
    ws_b = _capi.block_cached_workspace_size(len(blk), 32, max_keys, Hq, Hkv, D)
    ws = torch.empty(max(ws_b, 16), dtype=torch.uint8, device=dev) if ws_b else None
    o = torch.zeros(q.shape, dtype=torch.bfloat16, device=dev)
    _capi.attn_block_cached_fwd(q.to(dev), k.to(dev), v.to(dev), o, cu.to(dev), None, len(blk), 32, max_keys,
                                None, None, None, off, D ** -0.5, ws)
    torch.cuda.synchronize()
    ref = oatt.varlen(to_np(q), to_np(k), to_np(v), cu.numpy(), cu.numpy(), D ** -0.5, dtype=np.float32)
    assert_attn_close(o, ref, "blocks only")


@pytest.mark.parametrize("lens,Hq,Hkv", [
    ([333, 20, 517], 28, 4),     # 4-wavefront launch: 29 m-tiles, chunks of 16, 348 blocks in a grid of 384
    ([300] * 5, 32, 32),         # 12-wavefront launch: 160 pairs, chunks of 1, grid 160
    ([2500, 100], 8, 2),         # 8-wavefront launch: 40 m-tiles, chunks of 16, 160 blocks in a grid of 256
    ([129, 5, 131], 8, 8),       # 4-wavefront launch: 2 m-tiles, chunks of 2, 48 blocks in a grid of 48
])
def test_varlen_xcd_interleave_covers_every_block(dev, lens, Hq, Hkv):
    """Logical blocks are dealt to the XCDs in chunks and the grid is padded
    to a multiple of 8 chunks: every output row is written (none left at the
    NaN fill) and matches the oracle."""
    print(f"varlen xcd interleave lens={lens} Hq={Hq} Hkv={Hkv}", flush=True)
    q, k, v, cu = configs.packed_qkv(lens, Hq, Hkv, 128, seed=7 + sum(lens))
    o = _run_varlen(q, k, v, cu, dev, o_init=torch.full(q.shape, float("nan"), dtype=torch.bfloat16))
    assert not torch.isnan(o).any(), "rows left unwritten"
    ref = oatt.varlen(to_np(q), to_np(k), to_np(v), cu.numpy(), cu.numpy(), 128 ** -0.5, dtype=np.float32)
    assert_attn_close(o, ref, f"lens={lens}")


def test_block_cached_xcd_interleave_covers_every_block(dev):
    """Key-split launch (chunks of n_split x m-tiles, padded grid): every row
    written and equal to the oracle."""
    prefix, blk, Hq, Hkv = [1000, 37, 650], [20, 20, 9], 28, 4
    print(f"block_cached xcd interleave prefix={prefix}", flush=True)
    q, k, v, cu, kc, vc, slots = _cached_case(prefix, blk, Hq, Hkv, seed=11)
    D = 128
    slot_off = [0]
    for s_ in slots:
        slot_off.append(slot_off[-1] + len(s_))
    flat_slots = torch.tensor([x for s_ in slots for x in s_], dtype=torch.int32)
    o = torch.full(q.shape, float("nan"), dtype=torch.bfloat16, device=dev)
    max_keys = max(p + b for p, b in zip(prefix, blk))
    ws_bytes = _capi.block_cached_workspace_size(len(blk), max(blk), max_keys, Hq, Hkv, D)
    assert ws_bytes > 0, "this shape is meant to split the keys"
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    _capi.attn_block_cached_fwd(q.to(dev), k.to(dev), v.to(dev), o, cu.to(dev), None, len(blk), max(blk), max_keys,
                                kc.to(dev), vc.to(dev), flat_slots.to(dev),
                                torch.tensor(slot_off, dtype=torch.int32, device=dev), D ** -0.5, ws)
    torch.cuda.synchronize()
    assert not torch.isnan(o).any(), "rows left unwritten"
    kcn, vcn = to_np(kc), to_np(vc)
    cul = cu.tolist()
    qn, kn, vn = to_np(q), to_np(k), to_np(v)
    for i in range(len(blk)):
        r0, r1 = cul[i], cul[i + 1]
        ref = oatt.block_cached(qn[r0:r1], kn[r0:r1], vn[r0:r1], kcn, vcn, slots[i], D ** -0.5, dtype=np.float32)
        assert_attn_close(o[r0:r1], ref, f"seq {i}")


@pytest.mark.parametrize("Hq,Hkv", [(8, 8), (16, 4)])
def test_block_cached_invalid_slots_are_excluded(dev, Hq, Hkv):
    """Slots outside the cache are left out of the softmax (one 32-row block
    per (segment, KV head), and four, two per workgroup)."""
    print(f"block_cached invalid slots Hq={Hq} Hkv={Hkv}", flush=True)
    q, k, v, cu, kc, vc, slots = _cached_case([300, 700], [32, 32], Hq, Hkv, seed=77)
    slots[0][5] = -3
    slots[0][100] = kc.shape[0]
    slots[1][699] = 10 ** 8
    D = 128
    off = [0, len(slots[0]), len(slots[0]) + len(slots[1])]
    flat = torch.tensor(slots[0] + slots[1], dtype=torch.int32)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    o = torch.zeros_like(qd)
    ws_b = _capi.block_cached_workspace_size(2, 32, 732, Hq, Hkv, D)
    ws = torch.empty(max(ws_b, 1), dtype=torch.uint8, device=dev) if ws_b else None
    _capi.attn_block_cached_fwd(qd, kd, vd, o, cu.to(dev), None, 2, 32, 732, kc.to(dev), vc.to(dev), flat.to(dev),
                                torch.tensor(off, dtype=torch.int32, device=dev), D ** -0.5, ws)
    torch.cuda.synchronize()
    cul = cu.tolist()
    for i in range(2):
        r0, r1 = cul[i], cul[i + 1]
        ref = oatt.block_cached(to_np(q)[r0:r1], to_np(k)[r0:r1], to_np(v)[r0:r1], to_np(kc), to_np(vc), slots[i],
                                D ** -0.5, dtype=np.float32)
        assert_attn_close(o[r0:r1], ref, f"seq {i}")
