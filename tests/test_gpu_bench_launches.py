"""The exact launches the benchmark times, at full size, against the fp32
oracle (bf16 output vs fp32 reference on the same bf16 inputs: max-abs
<= 2e-2, mean-abs <= 2e-3).

- C2 headline: one LLaDA-8B dense denoise step's attention call, 8 x 384
  tokens, 32 / 32 heads -- the 12-wavefront launch (one workgroup per
  (sequence, head)); the launch shape is asserted through the C ABI's query.
- C3: the 16 Dream-7B prompt lengths + 256 generated tokens, 28 / 4 heads, in
  the step plan's order (longest first, through a segment-id table), as the
  layer calls run it -- the 4-wavefront launch.
- C5: the 32 blocks of 32 tokens against 2048..4096 cached rows in shuffled
  pages (the benchmark's seeded inputs), the prefixes written by K1; every
  segment against oracle.block_cached, the cached rows bit-exact in the cache.
These reference the flash_attn_varlen_func call of
dllmserve/layers/attention.py:289-299 and its mode-2 inputs (:235-265)."""
import numpy as np
import pytest
import torch

from helpers import assert_attn_close, bits, to_np
from oracle import attention as oatt
from oracle import configs
from dllm_serve_amd import _capi
from dllm_serve_amd.layers.attention import store_kvcache

pytestmark = pytest.mark.gpu

D = 128


def _varlen(q, k, v, cu, seg_ids, dev):
    lens = (cu[1:] - cu[:-1]).tolist()
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    o = torch.full_like(qd, float("nan"))
    ids = None if seg_ids is None else torch.tensor(seg_ids, dtype=torch.int32, device=dev)
    _capi.attn_varlen_fwd(qd, kd, vd, o, cu.to(dev), cu.to(dev), ids, len(lens), max(lens), D ** -0.5)
    torch.cuda.synchronize()
    return o


def test_c2_headline_launch(dev):
    lens = configs.c2_dense_lens()
    assert lens == [384] * 8
    shape = _capi.varlen_launch_shape(8, 384, 384, 32, 32, D)
    print(f"C2 headline launch 8 x 384, 32/32 heads: {shape}", flush=True)
    assert shape["wavefronts"] == 12 and shape["grid"] == 256
    q, k, v, cu = configs.packed_qkv(lens, 32, 32, D, seed=202)
    o = _varlen(q, k, v, cu, None, dev)
    ref = oatt.varlen(to_np(q), to_np(k), to_np(v), cu.numpy(), cu.numpy(), D ** -0.5, dtype=np.float32)
    assert_attn_close(o, ref, "C2 8 x 384")


def test_c3_dream_launch(dev):
    lens = configs.c3_lens()
    order = sorted(range(len(lens)), key=lambda i: (-lens[i], i))   # the step plan's order
    shape = _capi.varlen_launch_shape(len(lens), max(lens), max(lens), 28, 4, D)
    print(f"C3 Dream launch, 16 segments of {min(lens)}..{max(lens)} tokens, 28/4 heads: {shape}", flush=True)
    assert shape["wavefronts"] == 4
    q, k, v, cu = configs.packed_qkv(lens, 28, 4, D, seed=303)
    o = _varlen(q, k, v, cu, order, dev)
    ref = oatt.varlen(to_np(q), to_np(k), to_np(v), cu.numpy(), cu.numpy(), D ** -0.5, dtype=np.float32)
    assert_attn_close(o, ref, "C3 Dream 16 segments")


def test_c5_all_segments(dev):
    c = configs.c5_cached()
    Hq = Hkv = 32
    page, blk, B = c["page"], c["blk"], len(c["prefix"])
    max_keys = max(c["prefix"]) + blk
    shape = _capi.block_cached_launch_shape(B, blk, max_keys, Hq, Hkv, D)
    print(f"C5 block-cached launch, {B} x {blk} tokens vs {min(c['prefix'])}..{max(c['prefix'])} cached: {shape}",
          flush=True)
    assert shape["n_split"] == 1
    kc = torch.zeros(c["num_pages"] * page, Hkv, D, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    flat = [x for s in c["slots"] for x in s]
    slots = torch.tensor(flat, dtype=torch.int32, device=dev)
    store_kvcache(c["k_pre"].to(dev), c["v_pre"].to(dev), kc.view(-1, page, Hkv, D), vc.view(-1, page, Hkv, D), slots)
    off = np.concatenate([[0], np.cumsum(c["prefix"])]).astype(np.int64)
    q, k, v = c["q"].to(dev), c["k"].to(dev), c["v"].to(dev)
    cu = torch.arange(0, (B + 1) * blk, blk, dtype=torch.int32, device=dev)
    slot_off = torch.tensor(off, dtype=torch.int32, device=dev)
    o = torch.full_like(q, float("nan"))
    _capi.attn_block_cached_fwd(q, k, v, o, cu, None, B, blk, max_keys, kc, vc, slots, slot_off, D ** -0.5, None)
    torch.cuda.synchronize()
    # the cached rows the kernel read: K1 put every prefix row at its slot, bit-exact
    idx = torch.tensor(flat, dtype=torch.int64, device=dev)
    assert np.array_equal(bits(kc[idx]), bits(c["k_pre"])) and np.array_equal(bits(vc[idx]), bits(c["v_pre"]))
    # every segment against the oracle's mode-2 attention over the same rows
    kp, vp = to_np(c["k_pre"]), to_np(c["v_pre"])
    qn, kn, vn = to_np(c["q"]), to_np(c["k"]), to_np(c["v"])
    ref = np.zeros(qn.shape, dtype=np.float32)
    for s in range(B):
        r = slice(s * blk, (s + 1) * blk)
        ref[r] = oatt.block_cached(qn[r], kn[r], vn[r], kp, vp, np.arange(off[s], off[s + 1]), D ** -0.5,
                                   dtype=np.float32)
    assert_attn_close(o, ref, "C5 32 segments")
