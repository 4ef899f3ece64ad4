"""The full-model denoise driver the bench times (bench.LLaDA8B + bench.denoise:
LLaDA-8B shapes -- hidden 4096, 32 heads x 128, SwiGLU 12288, vocab 126464 --
random N(0, 0.02) weights, here 2 of its 32 layers) checked against the oracle
inside its own loop: every Attention call of every step is shadowed by
oracle.attention.mixed_step on the same q / k / v (the bf16 values the model
produced), and the model goes on with the kernels' output.  The sparse run
(head_select, retention 0.5, pool 3, delay 1, block 32) passes through cache
states 0, 1 and 2 in both blocks; outputs within the bf16 tolerance (max-abs
2e-2, mean-abs 2e-3) of the fp32 oracle, and after every call the shadow
cache -- written by the oracle's selection and store -- equals the model's
cache bit for bit.  The dense run's steps are checked the same way."""
import os
import sys

import numpy as np
import pytest
import torch

from helpers import assert_attn_close, bits, to_np
from oracle import attention as oatt
from oracle.bf16 import f32_to_bf16_bits
from dllm_serve_amd.engine.sequence import slot_mapping_for
from dllm_serve_amd.layers.attention import StepLayout
from dllm_serve_amd.utils.context import get_context

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


class ShadowAttention:
    """Calls the layer's Attention and checks its output (and, after a
    selection, the cache) against the oracle run on the same inputs."""

    def __init__(self, attn, layer, log):
        self.attn, self.layer, self.log = attn, layer, log
        self.rk = self.rv = None

    def bind(self):
        kc = self.attn.k_cache
        rows = kc.numel() // (self.attn.num_kv_heads * self.attn.head_dim)
        self.rk = np.zeros((rows, self.attn.num_kv_heads, self.attn.head_dim), dtype=np.float32)
        self.rv = np.zeros_like(self.rk)

    def __call__(self, q, k, v):
        out = self.attn(q, k, v)
        ctx = get_context()
        lay = StepLayout(ctx.seqs)
        desc, slot_lists = [], []
        for i, seq in enumerate(ctx.seqs):
            mode, rows = lay.modes[i], lay.rows[i]
            d = dict(mode=mode, rows=rows)
            if mode in (1, 2):
                bs, bl = lay.spans[i]
                hs, pool = lay.cfgs[i]
                d.update(blk_start=bs, blk_len=bl, n_keep=lay.keeps[i], head_select=hs, pool_k=pool)
                slot_lists.append(slot_mapping_for(seq))
            else:
                slot_lists.append([])
            desc.append(d)
        torch.cuda.synchronize()
        ref, _ = oatt.mixed_step(to_np(q), to_np(k), to_np(v), desc, self.rk, self.rv, slot_lists,
                                 self.attn.scale, dtype=np.float32)
        n, H, D = q.shape[0], q.shape[1], q.shape[2]
        what = f"layer {self.layer}, modes {[d['mode'] for d in desc]}"
        assert_attn_close(out.view(n, H, D), ref, what)
        if self.rk is not None and any(d["mode"] == 1 for d in desc):
            kc = bits(self.attn.k_cache).reshape(self.rk.shape[0], -1)
            vc = bits(self.attn.v_cache).reshape(self.rv.shape[0], -1)
            assert np.array_equal(kc, f32_to_bf16_bits(self.rk.reshape(self.rk.shape[0], -1))), what + ": K cache"
            assert np.array_equal(vc, f32_to_bf16_bits(self.rv.reshape(self.rv.shape[0], -1))), what + ": V cache"
        self.log.append(tuple(d["mode"] for d in desc))
        return out


@pytest.fixture(scope="module")
def model(dev):
    import bench

    m = bench.LLaDA8B(dev, cfg=dict(bench.LLADA_8B, layers=2))
    yield m
    del m
    torch.cuda.empty_cache()


def _shadow(model, log):
    """Swap the model's attention layers for shadows; the cache binding still
    binds the real layers (then sizes the shadow caches)."""
    real_attn = model.attn
    shadows = [ShadowAttention(a, i, log) for i, a in enumerate(real_attn)]
    real_bind = model.bind_cache

    def bind_cache(num_pages):
        model.attn = real_attn
        try:
            real_bind(num_pages)
        finally:
            model.attn = shadows
        for s in shadows:
            s.bind()

    model.bind_cache = bind_cache
    return shadows, real_bind


def test_full_model_sparse_denoise_against_oracle(dev, model):
    """2 sequences x (96 prompt + 64 generated) tokens, block 32, 8 steps (4 per
    block): full, select-and-store, then reuse, in both blocks."""
    import bench

    print("full model (2 LLaDA-8B layers): sparse denoise, 8 steps, shadowed by the oracle", flush=True)
    log = []
    shadows, _ = _shadow(model, log)
    attn = model.attn
    model.attn = shadows
    try:
        _, steps, tok = bench.denoise(model, 2, 96, 64, 8, 32, True, dev, seed=3, ratio=0.5, head_select=True)
    finally:
        model.attn = attn
        del model.bind_cache  # the class's own method again
    assert steps == 8 and len(log) == 2 * 8
    seen = {m for modes in log for m in modes}
    assert {0, 1, 2} <= seen, f"cache states seen: {sorted(seen)}"
    # the sampler unmasked at least one position of each sequence per step
    unmasked = (tok[:, 96:] != bench.LLADA_8B["mask_id"]).sum(dim=1)
    assert bool((unmasked >= steps).all()), f"unmasked positions per sequence: {unmasked.tolist()}"


def test_full_model_dense_denoise_against_oracle(dev, model):
    """The dense run (no SparseConfig): 4 steps of full attention over 2 x 160 tokens."""
    import bench

    print("full model (2 LLaDA-8B layers): dense denoise, 4 steps, shadowed by the oracle", flush=True)
    log = []
    shadows, _ = _shadow(model, log)
    attn = model.attn
    model.attn = shadows
    try:
        bench.denoise(model, 2, 96, 64, 4, 32, False, dev, seed=4)
    finally:
        model.attn = attn
        del model.bind_cache  # the class's own method again
    assert len(log) == 2 * 4 and all(m == (0, 0) for m in log)
