"""Benchmark of the diffusion attention path on one MI355X.

Headline workload (LLaDA-8B, B=8, prompt 256 + gen 128, bf16): one dense
denoising step's attention = 32 layer calls of Attention.forward over 8
packed sequences of 384 tokens (32 heads x 128), each layer with its own
q/k/v resident in HBM.  `value` = attention TFLOP/s over the timed steps
(FLOPs = 4 * sum Lq*Lk*Hq*D).  Extra fields report the other shapes of the
path (Dream GQA varlen, head-sparse C4 full/reuse, long-prefix block-cached
attention with the KV scatter) and the CPU oracle baseline.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "dllm-serve_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np  # noqa: E402
import torch  # noqa: E402

METRIC = "bidirectional attn TFLOP/s (% MFMA peak); denoise-step tokens/s, LLaDA-8B, 1 GPU"
PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


class Timer:
    """HIP events on torch's current stream (the stream every kernel of the
    path is launched on)."""

    def __init__(self):
        self.a = torch.cuda.Event(enable_timing=True)
        self.b = torch.cuda.Event(enable_timing=True)

    def start(self):
        self.a.record()

    def stop_ms(self) -> float:
        self.b.record()
        self.b.synchronize()
        return self.a.elapsed_time(self.b)


def make_layers(lens, Hq, Hkv, D, n_layers, dev, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    n = int(sum(lens))
    out = []
    for _ in range(n_layers):
        q = torch.randn(n, Hq, D, generator=g, device=dev, dtype=torch.bfloat16)
        k = torch.randn(n, Hkv, D, generator=g, device=dev, dtype=torch.bfloat16)
        v = torch.randn(n, Hkv, D, generator=g, device=dev, dtype=torch.bfloat16)
        out.append((q, k, v))
    return out


def dense_context(lens, dev):
    """Context of a dense diffusion step (no SparseConfig) as the runner sets it."""
    from dllm_serve_amd.engine.sequence import Sequence, prepare_step

    seqs = [Sequence([0] * (n - 0), 0, 126336, None, device=dev) for n in lens]
    prepare_step(seqs, dev)


# The GPU's clocks ramp up over the first ~40 ms of sustained work (a step of
# the headline workload goes from 1.15 ms cold to 0.93 ms after that, then
# drifts to ~0.95 ms as the part warms): every timed region is preceded by
# this much untimed work of the same kind, so it measures the steady state.
SETTLE_S = 0.25


def settle(fn, seconds=SETTLE_S):
    """Run fn (GPU work) repeatedly for `seconds` of wall time, synchronised."""
    t0 = time.perf_counter()
    while True:
        for _ in range(8):
            fn()
        torch.cuda.synchronize()
        if time.perf_counter() - t0 >= seconds:
            return


def time_layer_calls(attn, layers, steps, warmup):
    """Run `steps` timed steps, each = one Attention.forward per layer."""

    def step():
        for q, k, v in layers:
            attn(q, k, v)

    settle(step)
    for _ in range(warmup):
        for q, k, v in layers:
            attn(q, k, v)
    torch.cuda.synchronize()
    t = Timer()
    t.start()
    for _ in range(steps):
        for q, k, v in layers:
            attn(q, k, v)
    ms = t.stop_ms()
    torch.cuda.synchronize()
    return ms / steps


def time_kernel(fn, iters=50, warmup=5, settle_s=0.1):
    if settle_s:
        settle(fn, settle_s)
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t = Timer()
    t.start()
    for _ in range(iters):
        fn()
    return t.stop_ms() / iters


def bench_dense(lens, Hq, Hkv, D, n_layers, steps, warmup, dev, seed=0):
    from oracle.configs import attention_bytes, attention_flops
    from dllm_serve_amd import _capi
    from dllm_serve_amd.layers.attention import Attention
    from dllm_serve_amd.utils.context import get_context, reset_context

    attn = Attention(Hq, D, D ** -0.5, Hkv, causal=False)
    layers = make_layers(lens, Hq, Hkv, D, n_layers, dev, seed)
    dense_context(lens, dev)
    ms_step = time_layer_calls(attn, layers, steps, warmup)
    flops_call = attention_flops(lens, lens, Hq, D)
    bytes_call = attention_bytes(lens, lens, Hq, Hkv, D)
    # per-launch kernel time: the raw varlen kernel over distinct layers' buffers,
    # with the step plan's segment order (longest first), as the layer calls run it
    plan = get_context()._dllm_plan
    outs = [torch.empty_like(q) for q, _, _ in layers]
    state = {"i": 0}

    def one():
        i = state["i"] % n_layers
        state["i"] += 1
        q, k, v = layers[i]
        _capi.attn_varlen_fwd(q, k, v, outs[i], plan.cu, plan.cu, None if plan.dense_identity else plan.dense_ids,
                              plan.n_dense, plan.max_q_dense, D ** -0.5)

    ms_kernel = time_kernel(one, iters=4 * n_layers)
    # the same step's layer calls captured once in a HIP graph and replayed
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for q, k, v in layers:
            attn(q, k, v)
    ms_graph = time_kernel(graph.replay, iters=steps, warmup=warmup)
    del graph
    reset_context()
    return dict(ms_per_step=ms_step, flops_per_call=flops_call, bytes_per_call=bytes_call,
                tflops_step=flops_call * n_layers / (ms_step * 1e-3) / 1e12,
                kernel_us=ms_kernel * 1e3, tflops_kernel=flops_call / (ms_kernel * 1e-3) / 1e12,
                ms_per_step_graph=ms_graph, tflops_step_graph=flops_call * n_layers / (ms_graph * 1e-3) / 1e12)


def c5_case(dev):
    """C5 inputs resident on the device: 32 x 32-token blocks against 2-4k-token
    cached prefixes in shuffled 256-row pages (LLaDA shape).  Returns the two
    launches -- store_kvcache of the prefixes and the block-cached attention --
    and their algorithmic bytes / FLOPs."""
    from oracle import configs
    from dllm_serve_amd import _capi
    from dllm_serve_amd.layers.attention import store_kvcache

    c = configs.c5_cached()
    Hq = Hkv = 32
    D = 128
    page = c["page"]
    kc = torch.zeros(c["num_pages"] * page, Hkv, D, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    slots = torch.tensor([x for s in c["slots"] for x in s], dtype=torch.int32, device=dev)
    k_pre, v_pre = c["k_pre"].to(dev), c["v_pre"].to(dev)
    n_pre = k_pre.shape[0]
    q, k, v = c["q"].to(dev), c["k"].to(dev), c["v"].to(dev)
    B, blk = len(c["prefix"]), c["blk"]
    cu = torch.arange(0, (B + 1) * blk, blk, dtype=torch.int32, device=dev)
    off = [0]
    for p in c["prefix"]:
        off.append(off[-1] + p)
    slot_off = torch.tensor(off, dtype=torch.int32, device=dev)
    max_keys = max(c["prefix"]) + blk
    ws_b = _capi.block_cached_workspace_size(B, blk, max_keys, Hq, Hkv, D)
    ws = torch.empty(max(ws_b, 1), dtype=torch.uint8, device=dev)
    o = torch.empty_like(q)

    def store():
        store_kvcache(k_pre, v_pre, kc.view(-1, page, Hkv, D), vc.view(-1, page, Hkv, D), slots)

    def attend():
        _capi.attn_block_cached_fwd(q, k, v, o, cu, None, B, blk, max_keys, kc, vc, slots, slot_off, D ** -0.5,
                                    ws if ws_b else None)

    return dict(store=store, attend=attend, store_bytes=8.0 * n_pre * Hkv * D + 4.0 * n_pre,
                flops=sum(4.0 * blk * (p + blk) * Hq * D for p in c["prefix"]),
                bytes=sum(2.0 * (2 * blk * Hq * D + 2 * (p + blk) * Hkv * D) + 4.0 * p for p in c["prefix"]))


def bench_block_cached(dev, quick):
    """C5 timing: the KV scatter of the prefixes, then the block-cached attention."""
    c = c5_case(dev)
    ms_store = time_kernel(c["store"], iters=20)
    ms = time_kernel(c["attend"], iters=50)
    byts = c["bytes"]
    return dict(kernel_us=ms * 1e3, gbs=byts / (ms * 1e-3) / 1e9, tflops=c["flops"] / (ms * 1e-3) / 1e12,
                bytes_per_call=byts, store_us=ms_store * 1e3, store_gbs=c["store_bytes"] / (ms_store * 1e-3) / 1e9)


def bench_mfma_probe(dev, iters=20000, reps=5):
    """The library's register-only MFMA clock probe (one workgroup of eight
    wavefronts per CU, four independent MFMA chains each): median TFLOP/s of
    `reps` launches.  Its rate moves with the shader clock only, so it is
    the same-run control for the kernel timings beside it."""
    from dllm_serve_amd import _capi

    n_cu = torch.cuda.get_device_properties(dev).multi_processor_count
    sink = torch.empty(n_cu * 512, dtype=torch.float32, device=dev)
    flops = _capi.mfma_probe(sink, n_cu, iters)  # untimed first launch
    torch.cuda.synchronize()
    times = []
    for _ in range(reps):
        t = Timer()
        t.start()
        _capi.mfma_probe(sink, n_cu, iters)
        times.append(t.stop_ms())
    ms = sorted(times)[reps // 2]
    tf = flops / (ms * 1e-3) / 1e12
    return dict(mfma_probe_tflops=round(tf, 1), of_peak=round(tf / PEAK_BF16_TFLOPS, 4), cus=n_cu,
                ms=round(ms, 4))


def bench_copy(dev, nbytes=1 << 30):
    """A plain device-to-device copy of 1 GiB (torch / HIP runtime): the
    practical HBM rate the copy-like kernels (KV scatter, RoPE, block-cached
    reads) are compared with."""
    src = torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    ms = time_kernel(lambda: dst.copy_(src), iters=10, warmup=2)
    del src, dst
    return dict(bytes=2.0 * nbytes, us=ms * 1e3, gbs=2.0 * nbytes / (ms * 1e-3) / 1e9)


def _paged_slots(prefix, seed, page=256):
    """Per-sequence slot lists over shuffled 256-row pages, and the page count."""
    pages_per = [-(-p // page) for p in prefix]
    n_pages = sum(pages_per) + 1
    perm = torch.randperm(n_pages, generator=torch.Generator().manual_seed(seed)).tolist()
    slots, at = [], 0
    for p, npg in zip(prefix, pages_per):
        for j in range(npg):
            fill = page if j < npg - 1 else p - page * (npg - 1)
            slots.extend(range(perm[at + j] * page, perm[at + j] * page + fill))
        at += npg
    return slots, n_pages


# (name, segments, block rows, cached rows per segment, Hq, Hkv): the state-2
# (reuse) steps of the denoise loops.  C4 at retention 1.0 is the same block
# against all 1216 candidate rows.
DENOISE_CACHED_SHAPES = (
    ("c2_cached_8x32_vs_352", 8, 32, 352, 32, 32),
    ("c4_reuse_4x64_vs_608", 4, 64, 608, 32, 32),
    ("c4_ret1_4x64_vs_1216", 4, 64, 1216, 32, 32),
    ("dream_gqa_16x32_vs_700", 16, 32, 700, 28, 4),
)


def bench_denoise_shapes(dev, n_layers=8):
    """K3b (block-cached attention) at the denoise-loop reuse shapes, each
    launch on another layer's q/k/v and cache (n_layers of them, so the cache
    rows come from HBM, not from a previous launch's cache residue).  Bytes
    are the algorithmic ones: Q and O of the block, K/V of block and cached
    rows, the int32 slot list."""
    from oracle.configs import attention_bytes, attention_flops
    from dllm_serve_amd import _capi

    D = 128
    out = {}
    for name, B, Lq, n_c, Hq, Hkv in DENOISE_CACHED_SHAPES:
        prefix = [n_c] * B
        slots, n_pages = _paged_slots(prefix, seed=1)
        g = torch.Generator(device=dev).manual_seed(0)
        n = B * Lq
        layers = []
        for _ in range(n_layers):
            kc = torch.randn(n_pages * 256, Hkv, D, generator=g, device=dev, dtype=torch.bfloat16)
            vc = torch.randn(n_pages * 256, Hkv, D, generator=g, device=dev, dtype=torch.bfloat16)
            q = torch.randn(n, Hq, D, generator=g, device=dev, dtype=torch.bfloat16)
            k = torch.randn(n, Hkv, D, generator=g, device=dev, dtype=torch.bfloat16)
            v = torch.randn(n, Hkv, D, generator=g, device=dev, dtype=torch.bfloat16)
            layers.append((q, k, v, torch.empty_like(q), kc, vc))
        cu = torch.arange(0, n + 1, Lq, dtype=torch.int32, device=dev)
        sl = torch.tensor(slots, dtype=torch.int32, device=dev)
        so = torch.tensor([i * n_c for i in range(B + 1)], dtype=torch.int32, device=dev)
        max_keys = n_c + Lq
        ws_b = _capi.block_cached_workspace_size(B, Lq, max_keys, Hq, Hkv, D)
        ws = torch.empty(max(ws_b, 16), dtype=torch.uint8, device=dev) if ws_b else None
        state = {"i": 0}

        def one():
            q, k, v, o, kc, vc = layers[state["i"] % n_layers]
            state["i"] += 1
            _capi.attn_block_cached_fwd(q, k, v, o, cu, None, B, Lq, max_keys, kc, vc, sl, so, D ** -0.5, ws)

        reps = [time_kernel(one, iters=8 * n_layers, settle_s=0.05 if r else 0.1) for r in range(5)]
        ms = sorted(reps)[2]
        byts = attention_bytes([Lq] * B, [n_c + Lq] * B, Hq, Hkv, D) + 4.0 * B * n_c
        fl = attention_flops([Lq] * B, [n_c + Lq] * B, Hq, D)
        out[name] = dict(kernel_us=round(ms * 1e3, 2), bytes_per_call=byts, gbs=round(byts / (ms * 1e-3) / 1e9, 1),
                         frac_of_hbm=round(byts / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                         tflops=round(fl / (ms * 1e-3) / 1e12, 1))
        del layers
    out["c4_ret1_over_reuse_kernel_ratio"] = round(out["c4_ret1_4x64_vs_1216"]["kernel_us"]
                                                   / out["c4_reuse_4x64_vs_608"]["kernel_us"], 3)
    torch.cuda.empty_cache()
    return out


# (name, jobs, tokens per sequence, block start, block length, retention, head_select, Hq, Hkv): the
# state-1 (selection) steps: C4 head-sparse, C4 token-level, C2 at retention 1.0 (token level, the
# SparseConfig default), Dream GQA shape at retention 0.5
SELECT_SHAPES = (
    ("c4_head_select_4x1280", 4, 1280, 1024, 64, 0.5, True, 32, 32),
    ("c4_token_select_4x1280", 4, 1280, 1024, 64, 0.5, False, 32, 32),
    ("c2_cached_8x384_ret1", 8, 384, 256, 32, 1.0, False, 32, 32),
    ("dream_gqa_16x832", 16, 832, 576, 32, 0.5, True, 28, 4),
)


def bench_select(dev, n_layers=4):
    """K5/K6 (selection + fused scatter of the kept rows into the paged
    cache) per layer call, rotating n_layers layers' q/k/v and caches.
    Bytes (algorithmic): read the block queries and the candidate keys for
    scoring, read the kept K/V rows and write them into the cache, write the
    int64 indices."""
    from dllm_serve_amd import _capi
    from dllm_serve_amd.sparse.state import keep_count

    D = 128
    out = {}
    for name, B, n_tok, bs, bl, ratio, hs, Hq, Hkv in SELECT_SHAPES:
        Kc = n_tok - bl
        keep = keep_count(Kc, ratio)
        slots, n_pages = _paged_slots([keep] * B, seed=2)
        g = torch.Generator(device=dev).manual_seed(0)
        n = B * n_tok
        layers = []
        for _ in range(n_layers):
            q = torch.randn(n, Hq, D, generator=g, device=dev, dtype=torch.bfloat16)
            k = torch.randn(n, Hkv, D, generator=g, device=dev, dtype=torch.bfloat16)
            v = torch.randn(n, Hkv, D, generator=g, device=dev, dtype=torch.bfloat16)
            kc = torch.zeros(n_pages * 256, Hkv, D, dtype=torch.bfloat16, device=dev)
            layers.append((q, k, v, kc, torch.zeros_like(kc)))
        jobs = torch.tensor([[b * n_tok, n_tok, bs, bl, keep, b * keep, int(hs), 3] for b in range(B)],
                            dtype=torch.int32, device=dev)
        sl = torch.tensor(slots, dtype=torch.int32, device=dev)
        idx = torch.empty(B, Hkv, keep, dtype=torch.int64, device=dev)
        ws = torch.empty(_capi.select_workspace_size(B, Kc, Hq, Hkv, D), dtype=torch.uint8, device=dev)
        state = {"i": 0}

        def one():
            q, k, v, kc, vc = layers[state["i"] % n_layers]
            state["i"] += 1
            _capi.select_kv_store(q, k, v, jobs, B, Kc, keep, np.float32(D ** 0.5), kc, vc, sl, idx, ws)

        reps = [time_kernel(one, iters=8 * n_layers, settle_s=0.05 if r else 0.1) for r in range(5)]
        ms = sorted(reps)[2]
        byts = B * (2.0 * (bl * Hq * D + Kc * Hkv * D) + 8.0 * keep * Hkv * D + 8.0 * Hkv * keep)
        out[name] = dict(us=round(ms * 1e3, 2), kept_rows=keep, bytes_per_call=byts,
                         gbs=round(byts / (ms * 1e-3) / 1e9, 1),
                         frac_of_hbm=round(byts / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4))
        del layers
    torch.cuda.empty_cache()
    return out


def _block_attention_ms(dev, prompts, gen, Hq, Hkv, n_layers, cfgs, steps_block, graphed, D=128):
    """Attention time of one block of denoising steps per layer: sequences of
    the given prompt lengths (+ gen masked tokens), sequence i under
    SparseConfig cfgs[i] (None: dense), n_layers Attention layers with their
    own q/k/v and cache pages, every step through Attention.forward.

    graphed: each step's tables built on the device and the step replayed
    from a HIP graph captured once per launch shape (StepGraphs); two blocks
    run and the second, all replays enqueued back to back, is timed with HIP
    events around the block.  Eager: every layer call from the host, timed
    from before each step's host plan (StepPlan) and from after it; returns
    (ms, ms with the host plan)."""
    from dllm_serve_amd.engine.device_step import DeviceStepState, StepGraphs
    from dllm_serve_amd.engine.sequence import PageAllocator, Sequence, prepare_step
    from dllm_serve_amd.layers.attention import Attention
    from dllm_serve_amd.utils.context import get_context, reset_context

    B = len(prompts)
    attns = [Attention(Hq, D, D ** -0.5, Hkv, causal=False) for _ in range(n_layers)]
    seqs = [Sequence([1] * P, gen, 126336, cfg, device=dev, steps=gen) for P, cfg in zip(prompts, cfgs)]
    pages = max(1, sum(s.num_blocks for s in seqs))
    cache = torch.zeros(2, n_layers, pages, 256, Hkv, D, dtype=torch.bfloat16, device=dev)
    for i, a in enumerate(attns):
        a.k_cache, a.v_cache = cache[0, i], cache[1, i]
    alloc = PageAllocator(range(pages))
    for s in seqs:
        if s.sparse_state is not None:
            alloc.allocate(s)
    g = torch.Generator(device=dev).manual_seed(1)
    rows_all = sum(P + gen for P in prompts)
    full = [(torch.randn(rows_all, Hq, D, generator=g, device=dev, dtype=torch.bfloat16),
             torch.randn(rows_all, Hkv, D, generator=g, device=dev, dtype=torch.bfloat16),
             torch.randn(rows_all, Hkv, D, generator=g, device=dev, dtype=torch.bfloat16))
            for _ in range(n_layers)]
    torch.cuda.synchronize()
    total = total_plan = 0.0
    t_all, t = Timer(), Timer()
    if graphed:
        def step_fn(tables):
            n = tables.layout.total_rows
            for a, (q, k, v) in zip(attns, full):
                a(q[:n], k[:n], v[:n])

        tok = torch.zeros(B, max(prompts) + gen, dtype=torch.int64, device=dev)
        sg = StepGraphs(DeviceStepState(seqs, dev, tok.stride(0)), step_fn)
        for block in range(2):
            if block:  # the second block's replays, enqueued back to back
                torch.cuda.synchronize()
                t.start()
            for step in range(steps_block):
                sg.run(seqs)
                for s in seqs:
                    s.advance()
            if block:
                total = t.stop_ms() / n_layers
        del sg
        torch.cuda.synchronize()
        del full, cache
        return total, None
    for step in range(steps_block):
        prepare_step(seqs, dev)
        rows = sum(s.step_rows()[1] for s in seqs)
        t_all.start()  # the GPU is idle here (the previous step ended with a synchronisation)
        attns[0]._plan(get_context(), dev)  # per-step host plan, shared by all layers
        t.start()
        for a, (q, k, v) in zip(attns, full):
            a(q[:rows], k[:rows], v[:rows])
        total += t.stop_ms() / n_layers
        total_plan += t_all.a.elapsed_time(t.b) / n_layers
        reset_context()
        for s in seqs:
            s.advance()
    del full, cache
    return total, total_plan


def bench_sparse_c4(dev, steps_block=64, n_layers=32):
    """C4 attention per 64-step block and per layer (B=4, P=1024, gen 256,
    block 64, LLaDA-8B shape): sparse = head_select retention 0.5 (1 full
    step, 1 full step + selection/store, 62 reuse steps); dense = 64 full
    recompute steps.  Each step runs the model's 32 attention layers (own
    q/k/v and cache pages each), so the per-step table work is shared as in
    the model; the figure is the block's time divided by n_layers.  Primary
    figures from the device-step path (graphs), `eager` from host layer calls
    (see _block_attention_ms)."""
    from dllm_serve_amd.sparse.state import SparseConfig

    Hq = Hkv = 32
    B, P, gen, blk = 4, 1024, 256, 64
    cfgs = dict(sparse=SparseConfig(enabled=True, default_block_len=blk, retention_ratio=0.5, pool_kernel=3,
                                    delay_step=1, head_select=True),
                ret1=SparseConfig(enabled=True, default_block_len=blk, retention_ratio=1.0, pool_kernel=3,
                                  delay_step=1, head_select=True),
                dense=None)

    def run(cfg, graphed):
        return _block_attention_ms(dev, [P] * B, gen, Hq, Hkv, n_layers, [cfg] * B, steps_block, graphed)

    graphed = {k: run(c, True)[0] for k, c in cfgs.items()}
    eager = {k: run(c, False) for k, c in cfgs.items()}
    out = {f"ms_per_block_{k}": v for k, v in graphed.items()}
    out.update(speedup_vs_dense=graphed["dense"] / graphed["sparse"], speedup_vs_ret1=graphed["ret1"] / graphed["sparse"])
    ea = {f"ms_per_block_{k}": v[0] for k, v in eager.items()}
    ea.update({f"ms_per_block_{k}_with_host_plan": v[1] for k, v in eager.items()})
    ea.update(speedup_vs_dense=eager["dense"][0] / eager["sparse"][0],
              speedup_vs_ret1=eager["ret1"][0] / eager["sparse"][0],
              speedup_vs_ret1_with_host_plan=eager["ret1"][1] / eager["sparse"][1])
    out["eager"] = ea
    return out


def bench_sparse_dream(dev, n_layers=28):
    """Dream-7B attention (28 layers, 28 query / 4 KV heads) per 16-step block
    and per layer over the C3 batch: the 16 seeded prompt lengths of
    128..1024 tokens + 256 generated tokens each, block length 16.  `mixed`
    follows the reference's Dream test (tests/unit/test_dream_sparse.py:49):
    sequences cycle through [dense, SparseConfig(retention 0.5, block 16),
    dense] (token selection, the SparseConfig default); `sparse` puts every
    sequence under that config, `ret1` under retention 1.0, `dense` under
    none.  A 16-step block of a sparse sequence is one full step, one full
    step with selection and store, and 14 reuse steps.  Device-step path
    (graphs), as in bench_sparse_c4."""
    from oracle.configs import c3_lens
    from dllm_serve_amd.sparse.state import SparseConfig

    gen, blk = 256, 16
    prompts = [n - gen for n in c3_lens()]
    sp = SparseConfig(enabled=True, retention_ratio=0.5, default_block_len=blk)
    r1 = SparseConfig(enabled=True, retention_ratio=1.0, default_block_len=blk)
    B = len(prompts)
    cfgs = dict(mixed=[sp if i % 3 == 1 else None for i in range(B)], sparse=[sp] * B, ret1=[r1] * B,
                dense=[None] * B)
    ms = {k: _block_attention_ms(dev, prompts, gen, 28, 4, n_layers, c, blk, True)[0] for k, c in cfgs.items()}
    out = {f"ms_per_block_{k}": v for k, v in ms.items()}
    # tokens a block of the batch generates: gen / (gen / blk) = blk per sequence
    out.update(speedup_sparse_vs_dense=ms["dense"] / ms["sparse"], speedup_sparse_vs_ret1=ms["ret1"] / ms["sparse"],
               speedup_mixed_vs_dense=ms["dense"] / ms["mixed"],
               attention_tokens_per_s_mixed=B * blk / (ms["mixed"] * n_layers * 1e-3),
               attention_tokens_per_s_dense=B * blk / (ms["dense"] * n_layers * 1e-3),
               n_sparse_in_mixed=sum(c is not None for c in cfgs["mixed"]), block_len=blk, layers=n_layers)
    return out


# ---------------------------------------------------------------------------
# Full-model denoising driver (LLaDA-8B architecture, random N(0, 0.02)
# weights): the caller of the attention path, used to report denoise-step
# tokens/s = B * gen_length / total denoise time (the reference's formula,
# tests/unit/test_llada_sparse.py:56).  Layer structure as
# dllmserve/models/llada.py:61-97; low-confidence remasking as
# dllmserve/engine/model_runner.py:756-949 (temperature 0).
LLADA_8B = dict(layers=32, hidden=4096, heads=32, head_dim=128, mlp=12288, vocab=126464, eps=1e-5,
                theta=500000.0, mask_id=126336)


class LLaDA8B:
    def __init__(self, dev, cfg=LLADA_8B, seed=0):
        from dllm_serve_amd.layers.attention import Attention

        g = torch.Generator(device=dev).manual_seed(seed)
        H, F, V = cfg["hidden"], cfg["mlp"], cfg["vocab"]

        def w(*shape):
            return (torch.randn(*shape, generator=g, device=dev, dtype=torch.bfloat16) * 0.02)

        self.cfg = cfg
        self.dev = dev
        self.wte = w(V, H)
        self.lm_head = w(V, H)
        self.layers = []
        for _ in range(cfg["layers"]):
            self.layers.append(dict(qkv=w(3 * H, H), o=w(H, H), gate_up=w(2 * F, H), down=w(H, F),
                                    attn_norm=torch.ones(H, device=dev, dtype=torch.bfloat16),
                                    ff_norm=torch.ones(H, device=dev, dtype=torch.bfloat16)))
        self.ln_f = torch.ones(H, device=dev, dtype=torch.bfloat16)
        self.attn = [Attention(cfg["heads"], cfg["head_dim"], cfg["head_dim"] ** -0.5, cfg["heads"], causal=False)
                     for _ in range(cfg["layers"])]
        from dllm_serve_amd.layers.rotary_embedding import RotaryEmbedding

        D = cfg["head_dim"]
        # q / k are column views of the QKV projection output: rotate in place (K7)
        self.rope = RotaryEmbedding(D, D, 8192, cfg["theta"], inplace=True).to(dev)

    def bind_cache(self, num_pages):
        c = self.cfg
        self.kv = torch.zeros(2, c["layers"], num_pages, 256, c["heads"], c["head_dim"], dtype=torch.bfloat16,
                              device=self.dev)
        for i, a in enumerate(self.attn):
            a.k_cache, a.v_cache = self.kv[0, i], self.kv[1, i]

    def _rms(self, x, w):
        # torch's fused RMSNorm kernel (f32 statistics, bf16 out), in place of the
        # reference's compiled one (dllmserve/layers/layernorm.py:18-27)
        return torch.nn.functional.rms_norm(x, (x.shape[-1],), w, self.cfg["eps"])

    def forward(self, ids, pos):
        c = self.cfg
        H, nh, D = c["hidden"], c["heads"], c["head_dim"]
        n = ids.shape[0]
        h = self.wte[ids]
        for L, a in zip(self.layers, self.attn):
            x = self._rms(h, L["attn_norm"])
            qkv = x @ L["qkv"].t()
            q, k = self.rope(pos, qkv[:, :H], qkv[:, H:2 * H])
            q, k, v = q.view(n, nh, D), k.view(n, nh, D), qkv[:, 2 * H:].view(n, nh, D)
            h = torch.addmm(h, a(q, k, v), L["o"].t())  # residual add inside the GEMM (beta = 1)
            x = self._rms(h, L["ff_norm"])
            gu = x @ L["gate_up"].t()
            h = torch.addmm(h, torch.nn.functional.silu(gu[:, :c["mlp"]]) * gu[:, c["mlp"]:], L["down"].t())
        return self._rms(h, self.ln_f)


def denoise(model, batch, prompt, gen, steps, block, sparse, dev, seed=0, ratio=1.0, head_select=True,
            graphed=False):
    """Generate `gen` tokens for `batch` random prompts; returns (seconds,
    steps, final token table).

    Token ids stay on the device; each step's LM head runs on the rows that
    may be unmasked (all generated rows when dense, the current block when
    cached) and RemaskSampler unmasks ceil(masked / remaining steps) of them
    by confidence = max softmax probability (K8 + K9, no host round trip).
    graphed=True builds each step's tables on the device (dllm_step_build /
    dllm_step_advance) and replays the steps from HIP graphs captured once
    per launch shape (StepGraphs; the captures run inside the timed loop)."""
    from dllm_serve_amd.engine.device_step import DeviceStepState, StepGraphs
    from dllm_serve_amd.engine.sampler import RemaskSampler, sample_device_windows
    from dllm_serve_amd.engine.sequence import PageAllocator, Sequence, prepare_step
    from dllm_serve_amd.sparse.state import SparseConfig
    from dllm_serve_amd.utils.context import reset_context

    c = model.cfg
    g = torch.Generator().manual_seed(seed)
    cfg = SparseConfig(enabled=True, default_block_len=block, retention_ratio=ratio, pool_kernel=3, delay_step=1,
                       head_select=head_select) if sparse else None
    seqs = [Sequence(torch.randint(0, c["mask_id"], (prompt,), generator=g).tolist(), gen, c["mask_id"], cfg,
                     device=dev, steps=steps) for _ in range(batch)]
    if sparse:
        pages = sum(s.num_blocks for s in seqs)
        model.bind_cache(pages)
        alloc = PageAllocator(range(pages))
        for s in seqs:
            alloc.allocate(s)
    tok = torch.tensor([s.token_ids for s in seqs], dtype=torch.int64, device=dev)  # [B, N]
    sampler = RemaskSampler(lambda h: h @ model.lm_head.t(), c["mask_id"])
    graphs = None
    if graphed:
        def step_fn(t):
            hidden = model.forward(tok.view(-1).index_select(0, t.token_index), t.positions)
            sample_device_windows(sampler, hidden, tok, t.smp_rows, t.smp_params, t.max_win)

        graphs = StepGraphs(DeviceStepState(seqs, dev, tok.stride(0)), step_fn)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        if graphs is not None:
            graphs.run(seqs)
        else:
            rows = [s.step_rows() for s in seqs]
            ids = torch.cat([tok[i, a:a + n] for i, (a, n) in enumerate(rows)])
            pos = torch.cat([torch.arange(a, a + n, device=dev) for a, n in rows])
            prepare_step(seqs, dev, build_inputs=False)  # Context: cu_seqlens, slot lists, seqs
            hidden = model.forward(ids, pos)
            reset_context()
            sampler(hidden, seqs, tok)                   # K8 + K9: unmask in place on the device
        for s in seqs:
            s.advance()
    torch.cuda.synchronize()
    secs = time.perf_counter() - t0
    del graphs
    return secs, steps, tok


def bench_denoise(dev):
    """C2: LLaDA-8B, B=8, prompt 256, gen 128, steps 128, block 32; eager
    steps on host-built tables, and the same run replayed from HIP graphs
    over device-built tables (its tokens must equal the eager run's)."""
    model = LLaDA8B(dev)
    out = {}
    for name, sparse in (("cached_ret1", True), ("dense", False)):
        denoise(model, 8, 256, 128, 4, 32, sparse, dev, seed=1)  # warm-up (kernels, allocator)
        secs, steps, tok = denoise(model, 8, 256, 128, 128, 32, sparse, dev)
        out[name] = dict(seconds=round(secs, 3), steps=steps, tokens_per_s=round(8 * 128 / secs, 1),
                         ms_per_step=round(secs / steps * 1e3, 3))
        secs_g, _, tok_g = denoise(model, 8, 256, 128, 128, 32, sparse, dev, graphed=True)
        out[name + "_graphs"] = dict(seconds=round(secs_g, 3), steps=steps,
                                     tokens_per_s=round(8 * 128 / secs_g, 1),
                                     ms_per_step=round(secs_g / steps * 1e3, 3),
                                     tokens_equal_eager=bool(torch.equal(tok, tok_g)))
        del tok, tok_g
        torch.cuda.empty_cache()
    del model
    torch.cuda.empty_cache()
    return out


def bench_denoise_c4(dev):
    """C4: LLaDA-8B, B=4, prompt 1024, gen 256, block 64: one 64-step block,
    head-sparse (retention 0.5, head_select, pool 3) vs dense recompute."""
    model = LLaDA8B(dev)
    out = {}
    for name, sparse in (("head_sparse_r0.5", True), ("dense", False)):
        denoise(model, 4, 1024, 256, 3, 64, sparse, dev, seed=1, ratio=0.5)  # warm-up
        secs, steps, _ = denoise(model, 4, 1024, 256, 64, 64, sparse, dev, ratio=0.5)
        out[name] = dict(seconds=round(secs, 3), steps=steps, tokens_per_s=round(4 * 64 / secs, 1),
                         ms_per_step=round(secs / steps * 1e3, 3))
    out["speedup"] = round(out["dense"]["seconds"] / out["head_sparse_r0.5"]["seconds"], 2)
    del model
    torch.cuda.empty_cache()
    return out


def bench_rope(dev, n=8 * 384, Hq=32, Hkv=32, D=128, theta=500000.0):
    """K7 at the C2 step's token count: q and k of one layer rotated in place
    (positions of 8 sequences x 384), vs the reference's f32 tensor expression
    evaluated by torch (rotary_embedding.py:6-17) on the same device."""
    from dllm_serve_amd.layers.rotary_embedding import RotaryEmbedding

    rope = RotaryEmbedding(D, D, 8192, theta, inplace=True).to(dev)
    g = torch.Generator(device=dev).manual_seed(5)
    # eight layers' QKV outputs (600 MB, beyond the 256 MB last-level cache),
    # rotated in turn, so the timing reads and writes HBM
    bufs = [torch.randn(n, (Hq + 2 * Hkv) * D, generator=g, device=dev, dtype=torch.bfloat16) for _ in range(8)]
    views = [(b[:, :Hq * D], b[:, Hq * D:(Hq + Hkv) * D]) for b in bufs]
    pos = torch.arange(384, device=dev).repeat(n // 384)
    state = {"i": 0}

    def one():
        q_, k_ = views[state["i"] % len(views)]
        state["i"] += 1
        rope(pos, q_, k_)

    ms = time_kernel(one, iters=96)
    q, k = views[0]
    table = rope.cos_sin_cache

    def torch_expr():
        cs = table[pos]
        cos, sin = cs[:, None, :D // 2], cs[:, None, D // 2:]
        for x in (q.view(n, Hq, D), k.view(n, Hkv, D)):
            x1, x2 = torch.chunk(x.to(torch.float32), 2, dim=-1)
            torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), dim=-1).to(x.dtype)

    ms_torch = time_kernel(torch_expr, iters=20)
    del bufs, views
    algo = 2.0 * 2 * n * (Hq + Hkv) * D + 4.0 * n * D  # q/k read + written, one table row per token
    return dict(tokens=n, kernel_us=ms * 1e3, gbs=algo / (ms * 1e-3) / 1e9, frac_of_hbm=algo / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS,
                torch_expr_us=ms_torch * 1e3, speedup_vs_torch_expr=ms_torch / ms)


def reference_style_unmask(x0, x0_p, tok, wins, mask_id):
    """The reference's per-sequence unmasking loop (model_runner.py:895-949)
    in torch ops, for timing beside K9: mask test, .item() of the mask count,
    topk and the index write-back per sequence."""
    import math

    r = 0
    for b, (lo, n, sr) in enumerate(wins):
        t = tok[b]
        mask_index = t[lo:lo + n] == mask_id
        confidence = torch.where(mask_index, x0_p[r:r + n], -float("inf"))
        nmask = mask_index.sum().item()
        k = min(math.ceil(float(nmask) / sr), nmask)
        top = torch.topk(confidence, k=k).indices
        t[lo + top] = x0[r:r + n][top]
        r += n


def bench_sampler(dev):
    """K8 + K9 at the C2 shapes (LLaDA vocabulary 126464): the dense step's
    8 x 128 generated rows and the block step's 8 x 32, vs torch's
    softmax + max on the same logits and the reference's per-sequence loop;
    plus the whole sampling step (LM head GEMM included) at 8 x 128."""
    from dllm_serve_amd import _capi
    from dllm_serve_amd.engine.sampler import RemaskSampler
    from dllm_serve_amd.engine.sequence import Sequence

    V, mask_id = 126464, 126336
    out = {}
    for name, B, n in (("dense_8x128_rows", 8, 128), ("block_8x32_rows", 8, 32)):
        M = B * n
        g = torch.Generator(device=dev).manual_seed(M)
        # distinct logits buffers, 0.5 GB in all (beyond the 256 MB last-level cache)
        nb = max(2, (512 << 20) // (2 * M * V))
        bufs = [(torch.randn(M, V, generator=g, device=dev) * 1.3).to(torch.bfloat16) for _ in range(nb)]
        x0 = torch.empty(M, dtype=torch.int64, device=dev)
        p = torch.empty(M, dtype=torch.bfloat16, device=dev)
        ws = None  # the kernel needs no workspace
        state = {"i": 0}

        def k8():
            _capi.softmax_max(bufs[state["i"] % nb], x0, p, ws)
            state["i"] += 1

        ms8 = time_kernel(k8, iters=20 * nb)
        temp1 = torch.ones(M, dtype=torch.float64, device=dev)

        def k8_gumbel():
            _capi.softmax_max_sample(bufs[state["i"] % nb], temp1, 1234 + state["i"], 0, x0, p, ws)
            state["i"] += 1

        ms8g = time_kernel(k8_gumbel, iters=4 * nb)

        def ref_gumbel():  # add_gumbel_noise + softmax + max as the reference runs them (f64 tensors)
            lg = bufs[0].to(torch.float64)
            noise = torch.rand_like(lg)
            v = (lg.exp() / (-torch.log(noise))).to(torch.bfloat16)
            torch.max(torch.softmax(v, dim=-1), dim=-1)

        ms_tg = time_kernel(ref_gumbel, iters=3, warmup=1, settle_s=0)
        ms_t = time_kernel(lambda: torch.max(torch.softmax(bufs[0], dim=-1), dim=-1), iters=10)
        # K9 over 8 windows of n positions, most of them masked; steps_remain
        # large so that each call unmasks one position per sequence
        N = 256 + n
        tok = torch.full((B, N), mask_id, dtype=torch.int64, device=dev)
        params = torch.tensor([(b * N + 256, n, b * n, 10 ** 6, 0) for b in range(B)], dtype=torch.int32,
                              device=dev)
        ms9 = time_kernel(lambda: _capi.lowconf_unmask(tok, params, B, n, x0, p, mask_id), iters=40, settle_s=0)
        tok.fill_(mask_id)
        wins = [(256, n, 10 ** 6)] * B

        def ref_loop():
            reference_style_unmask(x0, p, tok, wins, mask_id)

        ms_loop = time_kernel(ref_loop, iters=10, warmup=2, settle_s=0)
        algo = 2.0 * M * V
        out[name] = dict(rows=M, k8_us=ms8 * 1e3, k8_gbs=algo / (ms8 * 1e-3) / 1e9,
                         k8_frac_of_hbm=algo / (ms8 * 1e-3) / 1e9 / PEAK_HBM_GBS,
                         torch_softmax_max_us=ms_t * 1e3, k8_speedup_vs_torch=ms_t / ms8,
                         k8_temperature1_us=ms8g * 1e3, torch_gumbel_softmax_max_us=ms_tg * 1e3,
                         k8_temperature1_speedup_vs_torch=ms_tg / ms8g,
                         k9_us=ms9 * 1e3, reference_loop_us=ms_loop * 1e3, k9_speedup_vs_loop=ms_loop / ms9)
        del bufs
    # whole sampling step of the C2 dense batch: hidden [8 x 384, 4096], LM head [126464, 4096]
    g = torch.Generator(device=dev).manual_seed(7)
    H = 4096
    w = (torch.randn(V, H, generator=g, device=dev, dtype=torch.bfloat16) * 0.02)
    hidden = torch.randn(8 * 384, H, generator=g, device=dev, dtype=torch.bfloat16)
    seqs = [Sequence([1] * 256, 128, mask_id, None, device=dev, steps=128) for _ in range(8)]
    tok = torch.tensor([s.token_ids for s in seqs], dtype=torch.int64, device=dev)
    sampler = RemaskSampler(lambda h: h @ w.t(), mask_id)
    tok0 = tok.clone()

    def our_step():
        tok.copy_(tok0)          # every timed call starts from the same masked tokens
        sampler(hidden, seqs, tok)

    ms_step = time_kernel(our_step, iters=10, warmup=2)

    def ref_step():
        tok.copy_(tok0)
        sel = torch.cat([hidden[b * 384 + 256:(b + 1) * 384] for b in range(8)])
        pr, xx = torch.max(torch.softmax(sel @ w.t(), dim=-1), dim=-1)
        reference_style_unmask(xx, pr, tok, [(256, 128, 128)] * 8, mask_id)

    ms_ref = time_kernel(ref_step, iters=10, warmup=2, settle_s=0)
    ms_gemm = time_kernel(lambda: hidden[:1024] @ w.t(), iters=10)
    out["c2_dense_sampling_step"] = dict(ms=ms_step, reference_style_ms=ms_ref, lm_head_gemm_ms=ms_gemm,
                                         speedup=ms_ref / ms_step)
    del w, hidden
    torch.cuda.empty_cache()
    return out


def cpu_setup():
    """Host threads for the CPU oracle runs: every core in this process's
    affinity set, capped by OMP_NUM_THREADS when the environment sets one (a
    shared host's per-GPU share of cores); torch and the BLAS pool numpy uses
    both get that count.  Returns (threads, affinity cores, CPU model)."""
    cores = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS", "")
    threads = min(cores, int(env)) if env.isdigit() and int(env) > 0 else cores
    torch.set_num_threads(threads)
    try:
        from threadpoolctl import threadpool_limits
        threadpool_limits(limits=threads)
    except ImportError:
        pass
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return threads, cores, model


def cpu_timed(fn, reps=5):
    """One untimed warm-up, then the median of `reps` perf_counter runs (s)."""
    fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return sorted(ts)[len(ts) // 2]


def cpu_baseline(lens, Hq, Hkv, D):
    """Oracle (numpy fp32) attention of one headline layer call (8 x 384
    tokens, 32 heads x 128) on the host cores: one warm-up, median of 5."""
    from oracle import attention as oatt
    from oracle.configs import attention_flops, packed_qkv

    threads, cores, model = cpu_setup()
    q, k, v, cu = packed_qkv(lens, Hq, Hkv, D, seed=0, dtype=torch.float32)
    qn, kn, vn, cun = q.numpy(), k.numpy(), v.numpy(), cu.numpy()
    t = cpu_timed(lambda: oatt.varlen(qn, kn, vn, cun, cun, D ** -0.5, dtype=np.float32))
    flops = attention_flops(lens, lens, Hq, D)
    return dict(value=flops / t / 1e12, unit="TFLOP/s", cores=threads, kind="port",
                sample=f"one layer call of the headline step (8 x 384 tokens, 32 heads x 128), numpy fp32 oracle: "
                       f"1 warm-up + median of 5 = {t:.3f} s; {threads} threads ({cores} cores in the affinity "
                       f"set), {model}", cpu_model=model, seconds=t)


def cpu_other_configs():
    """The oracle (numpy fp32) on the other configurations' single layer calls,
    on the host cores (one warm-up, median of 5 each): C1 whole attention
    (1 x 512 tokens), C4 full step (4 x 1280), C4 selection + scatter (4 jobs
    of 1280 tokens, head_select, 608 kept) and reuse step (4 x 64 rows
    against 608 cached + 64 block rows), C5 (32 x 32 rows against 2048-4096
    cached rows)."""
    from oracle import attention as oatt
    from oracle import configs
    from oracle import select as osel

    threads, cores, model = cpu_setup()
    out = {}
    q, k, v, cu, scale = configs.c1_single_layer()
    qn, kn, vn, cun = q.numpy(), k.numpy(), v.numpy(), cu.numpy()
    t = cpu_timed(lambda: oatt.varlen(qn, kn, vn, cun, cun, scale, dtype=np.float32))
    fl = configs.attention_flops([512], [512], 32, 128)
    out["c1_512_tokens"] = dict(seconds=round(t, 4), gflops=round(fl / t / 1e9, 1))
    q, k, v, cu = configs.packed_qkv([1280] * 4, 32, 32, 128, seed=4, dtype=torch.float32)
    qn, kn, vn, cun = q.numpy(), k.numpy(), v.numpy(), cu.numpy()
    t = cpu_timed(lambda: oatt.varlen(qn, kn, vn, cun, cun, 128 ** -0.5, dtype=np.float32))
    fl = configs.attention_flops([1280] * 4, [1280] * 4, 32, 128)
    out["c4_full_step_layer"] = dict(seconds=round(t, 3), gflops=round(fl / t / 1e9, 1))
    # C4 selection + scatter (state 1) of one layer: the oracle's head_select
    # rule on bf16 inputs, then the kept rows written into a paged cache
    qb, kb, vb, _ = configs.packed_qkv([1280] * 4, 32, 32, 128, seed=5)
    qs, ks, vs = (x.float().numpy() for x in (qb, kb, vb))
    n_keep, Kc = 608, 1216
    kcache = np.zeros((4 * n_keep, 32, 128), dtype=np.float32)
    vcache = np.zeros_like(kcache)

    cand = np.concatenate([np.arange(1024), np.arange(1088, 1280)])  # prefix and suffix rows around the block

    def select_store():
        for i in range(4):
            qi, ki, vi = qs[i * 1280:(i + 1) * 1280], ks[i * 1280:(i + 1) * 1280], vs[i * 1280:(i + 1) * 1280]
            idx = osel.select(qi[1024:1088], ki[cand], n_keep, True, 3, np.float32(128 ** 0.5))
            rows = cand[idx]  # [Hkv, n_keep] token rows per KV head
            for h in range(32):
                kcache[i * n_keep:(i + 1) * n_keep, h] = ki[rows[h], h]
                vcache[i * n_keep:(i + 1) * n_keep, h] = vi[rows[h], h]

    t = cpu_timed(select_store)
    by = 4 * (2.0 * (64 * 32 * 128 + Kc * 32 * 128) + 8.0 * n_keep * 32 * 128 + 8.0 * 32 * n_keep)
    out["c4_select_store_layer"] = dict(seconds=round(t, 3), gbs_bf16_equivalent=round(by / t / 1e9, 2))
    rng = np.random.default_rng(0)
    n_c, blk = 608, 64
    kc = rng.standard_normal((4 * n_c, 32, 128)).astype(np.float32)
    vc = rng.standard_normal((4 * n_c, 32, 128)).astype(np.float32)
    qr = rng.standard_normal((4 * blk, 32, 128)).astype(np.float32)
    slots = [list(range(i * n_c, (i + 1) * n_c)) for i in range(4)]

    def reuse():
        for i in range(4):
            r = slice(i * blk, (i + 1) * blk)
            oatt.block_cached(qr[r], qr[r], qr[r], kc, vc, slots[i], 128 ** -0.5, dtype=np.float32)

    t = cpu_timed(reuse)
    fl = configs.attention_flops([blk] * 4, [n_c + blk] * 4, 32, 128)
    by = configs.attention_bytes([blk] * 4, [n_c + blk] * 4, 32, 32, 128)
    out["c4_reuse_step_layer"] = dict(seconds=round(t, 4), gflops=round(fl / t / 1e9, 1),
                                      gbs_bf16_equivalent=round(by / t / 1e9, 2))
    c = configs.c5_cached()
    kp, vp = c["k_pre"].float().numpy(), c["v_pre"].float().numpy()
    qc, kb5, vb5 = c["q"].float().numpy(), c["k"].float().numpy(), c["v"].float().numpy()
    off = np.cumsum([0] + c["prefix"])
    slots5 = [list(range(off[i], off[i + 1])) for i in range(len(c["prefix"]))]  # prefixes packed in order

    def c5():
        for i in range(len(c["prefix"])):
            r = slice(i * c["blk"], (i + 1) * c["blk"])
            oatt.block_cached(qc[r], kb5[r], vb5[r], kp, vp, slots5[i], 128 ** -0.5, dtype=np.float32)

    t = cpu_timed(c5)
    blks = [c["blk"]] * len(c["prefix"])
    fl = configs.attention_flops(blks, [p + c["blk"] for p in c["prefix"]], 32, 128)
    by = configs.attention_bytes(blks, [p + c["blk"] for p in c["prefix"]], 32, 32, 128)
    out["c5_layer"] = dict(seconds=round(t, 3), gflops=round(fl / t / 1e9, 1),
                           gbs_bf16_equivalent=round(by / t / 1e9, 2))
    out["threads"] = threads
    out["cores_in_affinity_set"] = cores
    out["cpu_model"] = model
    out["timing"] = "1 warm-up + median of 5 perf_counter runs each"
    out["kind"] = "port"
    return out


def profile_run(lens, Hq, Hkv, D, n_layers, dev):
    """Fixed dispatch sequence for hardware-counter runs."""
    from dllm_serve_amd import _capi

    src = torch.empty(256 << 20, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)  # reads and writes exactly 256 MiB
    layers = make_layers(lens, Hq, Hkv, D, n_layers, dev, seed=0)
    cu = torch.zeros(len(lens) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(lens, dtype=torch.int32), 0)
    cu = cu.to(dev)
    for q, k, v in layers:
        o = torch.empty_like(q)
        _capi.attn_varlen_fwd(q, k, v, o, cu, cu, None, len(lens), max(lens), D ** -0.5)
    torch.cuda.synchronize()
    # RoPE of one layer's q and k at the same token count, in place
    from dllm_serve_amd.layers.rotary_embedding import RotaryEmbedding
    rope = RotaryEmbedding(D, D, 8192, 500000.0, inplace=True).to(dev)
    n = int(sum(lens))
    pos = torch.cat([torch.arange(x, device=dev) for x in lens])
    for q, k, _ in layers:
        rope(pos, q, k)
    # C5: the prefix scatter once, then four block-cached attention launches
    c5 = c5_case(dev)
    c5["store"]()
    for _ in range(4):
        c5["attend"]()
    del c5
    # K8 softmax-max over LLaDA logits, two buffers alternating: the C2 dense step's 8 x 128 rows
    # (256-thread workgroups), then its block step's 8 x 32 rows (1024-thread workgroups)
    V = 126464
    for M in (1024, 256):
        g = torch.Generator(device=dev).manual_seed(M)
        bufs = [(torch.randn(M, V, generator=g, device=dev) * 1.3).to(torch.bfloat16) for _ in range(2)]
        x0 = torch.empty(M, dtype=torch.int64, device=dev)
        p = torch.empty(M, dtype=torch.bfloat16, device=dev)
        for i in range(8):
            _capi.softmax_max(bufs[i % 2], x0, p)
        torch.cuda.synchronize()
        del bufs
    log(f"profile run done: 3 x 256 MiB copies, {n_layers} attention launches, {n_layers} RoPE launches "
        f"({n} tokens), 1 C5 store + 4 C5 block-cached launches, 8 + 8 K8 launches (1024 and 256 x {V} logits)")


def profile_denoise_run(dev):
    """Fixed dispatch sequence for counter runs of the denoise-loop kernels:
    three 256 MiB device copies (counter calibration); K3b at each
    DENOISE_CACHED_SHAPES case, 16 launches rotating 8 layers' caches; the
    selection chain at each SELECT_SHAPES case, 8 launches rotating 4
    layers; the dense kernel at C3 (16 ragged Dream GQA segments) and at the
    C4 full step (4 x 1280), 4 launches each over distinct layers."""
    from oracle.configs import c3_lens
    from dllm_serve_amd import _capi
    from dllm_serve_amd.sparse.state import keep_count

    D = 128
    src = torch.empty(256 << 20, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    for name, B, Lq, n_c, Hq, Hkv in DENOISE_CACHED_SHAPES:
        slots, n_pages = _paged_slots([n_c] * B, seed=1)
        g = torch.Generator(device=dev).manual_seed(0)
        n = B * Lq
        layers = [tuple(torch.randn(r, H, D, generator=g, device=dev, dtype=torch.bfloat16)
                        for r, H in ((n, Hq), (n, Hkv), (n, Hkv), (n_pages * 256, Hkv), (n_pages * 256, Hkv)))
                  for _ in range(8)]
        o = torch.empty(n, Hq, D, dtype=torch.bfloat16, device=dev)
        cu = torch.arange(0, n + 1, Lq, dtype=torch.int32, device=dev)
        sl = torch.tensor(slots, dtype=torch.int32, device=dev)
        so = torch.tensor([i * n_c for i in range(B + 1)], dtype=torch.int32, device=dev)
        ws_b = _capi.block_cached_workspace_size(B, Lq, n_c + Lq, Hq, Hkv, D)
        ws = torch.empty(max(ws_b, 16), dtype=torch.uint8, device=dev) if ws_b else None
        for i in range(16):
            q, k, v, kc, vc = layers[i % 8]
            _capi.attn_block_cached_fwd(q, k, v, o, cu, None, B, Lq, n_c + Lq, kc, vc, sl, so, D ** -0.5, ws)
        torch.cuda.synchronize()
        del layers
        log(f"profile: K3b {name}, 16 launches")
    for name, B, n_tok, bs, bl, ratio, hs, Hq, Hkv in SELECT_SHAPES:
        Kc = n_tok - bl
        keep = keep_count(Kc, ratio)
        slots, n_pages = _paged_slots([keep] * B, seed=2)
        g = torch.Generator(device=dev).manual_seed(0)
        n = B * n_tok
        layers = [tuple(torch.randn(r, H, D, generator=g, device=dev, dtype=torch.bfloat16)
                        for r, H in ((n, Hq), (n, Hkv), (n, Hkv))) for _ in range(4)]
        kc = torch.zeros(n_pages * 256, Hkv, D, dtype=torch.bfloat16, device=dev)
        vc = torch.zeros_like(kc)
        jobs = torch.tensor([[b * n_tok, n_tok, bs, bl, keep, b * keep, int(hs), 3] for b in range(B)],
                            dtype=torch.int32, device=dev)
        sl = torch.tensor(slots, dtype=torch.int32, device=dev)
        idx = torch.empty(B, Hkv, keep, dtype=torch.int64, device=dev)
        ws = torch.empty(_capi.select_workspace_size(B, Kc, Hq, Hkv, D), dtype=torch.uint8, device=dev)
        for i in range(8):
            q, k, v = layers[i % 4]
            _capi.select_kv_store(q, k, v, jobs, B, Kc, keep, np.float32(D ** 0.5), kc, vc, sl, idx, ws)
        torch.cuda.synchronize()
        del layers
        log(f"profile: selection {name}, 8 launches")
    for name, lens, Hq, Hkv in (("c3", c3_lens(), 28, 4), ("c4_full", [1280] * 4, 32, 32)):
        layers = make_layers(lens, Hq, Hkv, D, 4, dev, seed=3)
        order = sorted(range(len(lens)), key=lambda i: (-lens[i], i))  # the step plan's segment order
        ids = torch.tensor(order, dtype=torch.int32, device=dev)
        cu = torch.zeros(len(lens) + 1, dtype=torch.int32)
        cu[1:] = torch.cumsum(torch.tensor(lens, dtype=torch.int32), 0)
        cu = cu.to(dev)
        for q, k, v in layers:
            o = torch.empty_like(q)
            _capi.attn_varlen_fwd(q, k, v, o, cu, cu, None if order == list(range(len(lens))) else ids,
                                  len(lens), max(lens), D ** -0.5)
        torch.cuda.synchronize()
        del layers
        log(f"profile: dense {name}, 4 launches")


TRAFFIC_SUMMARY = os.path.join(ROOT, "profiles", "attn_dense_kernel_llada_c2_8x384_counters.md")
KERNEL_SOURCE = os.path.join(ROOT, "dllm-serve_amd", "csrc", "attn.hip")


def kernel_source_sha256() -> str:
    """First 16 hex digits of the SHA-256 of the attention kernels' source file."""
    import hashlib
    with open(KERNEL_SOURCE, "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()[:16]


def measured_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE summary (counters scaled by a plain 256 MiB copy), and where that
    figure was recorded: the summary's `recorded_on:` line names the commit and
    the SHA-256 of `attn.hip` of the build the counters ran on, which is compared
    with the source this run loads.  Returns (bytes or None, provenance dict)."""
    prov = {"summary": os.path.relpath(TRAFFIC_SUMMARY, ROOT), "commit": None,
            "kernel_source_sha256": None, "current_kernel_source_sha256": kernel_source_sha256()}
    try:
        text = open(TRAFFIC_SUMMARY).read()
    except OSError:
        return None, prov
    lines = text.splitlines()
    if kernel not in lines[0]:
        return None, prov
    traffic = None
    for line in lines:
        if line.startswith("traffic_bytes_per_launch:"):
            traffic = int(line.split(":")[1].strip())
        elif line.startswith("recorded_on:"):
            for part in line.split(":", 1)[1].split(";"):
                key, _, val = part.strip().partition(" ")
                if key == "commit":
                    prov["commit"] = val.strip()
                elif key == "attn.hip_sha256":
                    prov["kernel_source_sha256"] = val.strip()
    prov["source_matches"] = prov["kernel_source_sha256"] == prov["current_kernel_source_sha256"]
    return traffic, prov


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--quick", action="store_true", help="headline only (no extra shapes, no CPU baseline)")
    ap.add_argument("--profile", nargs="?", const="headline", choices=("headline", "denoise"),
                    help="counter run, prints no JSON.  headline: a 256 MiB device copy (x3, calibrates "
                         "FETCH_SIZE / WRITE_SIZE), 32 launches of the headline attention kernel, 32 RoPE "
                         "launches, the C5 store, 4 C5 block-cached launches and 8 softmax-max launches over "
                         "1024 x 126464 logits.  denoise: the copies, then block-cached attention at the "
                         "denoise reuse shapes, the selection chain at the state-1 shapes and the dense kernel "
                         "at C3 and the C4 full step")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); the library has no multi-GPU path",
              file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    from dllm_serve_amd import _capi

    _capi.load()
    dev = torch.device("cuda:0")
    Hq = Hkv = 32
    D = 128
    lens = [256 + 128] * 8
    n_layers = 32
    if args.profile == "headline":
        profile_run(lens, Hq, Hkv, D, n_layers, dev)
        return
    if args.profile == "denoise":
        profile_denoise_run(dev)
        return
    log("headline: C2 dense step attention, 32 layers x 8 x 384 tokens")
    r = bench_dense(lens, Hq, Hkv, D, n_layers, args.steps, args.warmup, dev)
    log("clock control: register-only MFMA probe")
    clock = bench_mfma_probe(dev)
    extra = {}
    if not args.quick:
        log("C3: Dream-7B GQA 28/4 varlen")
        from oracle.configs import c3_lens
        c3 = c3_lens()
        r3 = bench_dense(c3, 28, 4, D, 4, 3, 1, dev, seed=3)
        extra["c3_dream_gqa_varlen"] = dict(lens=c3, kernel_us=round(r3["kernel_us"], 2),
                                            tflops=round(r3["tflops_kernel"], 1),
                                            mfma_frac=round(r3["tflops_kernel"] / PEAK_BF16_TFLOPS, 4))
        log("C4 full-step shape: 4 x 1280 tokens")
        r4 = bench_dense([1280] * 4, Hq, Hkv, D, 4, 3, 1, dev, seed=4)
        extra["c4_full_step_attention"] = dict(kernel_us=round(r4["kernel_us"], 2),
                                               tflops=round(r4["tflops_kernel"], 1),
                                               mfma_frac=round(r4["tflops_kernel"] / PEAK_BF16_TFLOPS, 4))
        log("C5: block-cached attention + KV scatter")
        r5 = bench_block_cached(dev, args.quick)
        extra["c5_block_cached"] = {k: round(v, 3) for k, v in r5.items()}
        log("HBM: plain 1 GiB device copy")
        extra["hbm_copy_1gib"] = {k: round(v, 1) for k, v in bench_copy(dev).items()}
        log("K7: RoPE of q and k at the C2 step's token count")
        extra["rope_c2_tokens"] = {k: round(v, 3) for k, v in bench_rope(dev).items()}
        log("K8 / K9: remask sampler at the C2 shapes")
        extra["sampler_c2"] = {k: ({kk: round(vv, 3) for kk, vv in v.items()} if isinstance(v, dict) else v)
                               for k, v in bench_sampler(dev).items()}
        log("C4: sparse vs dense attention per 64-step block")
        r4s = bench_sparse_c4(dev)
        log("C3 Dream: mixed / sparse / dense attention per 16-step block")
        extra["c3_dream_sparse_per_block"] = {k: round(v, 3) if isinstance(v, float) else v
                                              for k, v in bench_sparse_dream(dev).items()}
        extra["c4_head_sparse_per_block"] = {k: (round(v, 3) if not isinstance(v, dict) else
                                                 {kk: round(vv, 3) for kk, vv in v.items()}) for k, v in r4s.items()}
        log("K3b at the denoise-loop reuse shapes (8 layers' caches rotated)")
        extra["block_cached_denoise_shapes"] = bench_denoise_shapes(dev)
        log("K5/K6 selection + scatter at the state-1 shapes")
        extra["select_store"] = bench_select(dev)
    if not args.quick:
        log("C2 full model: LLaDA-8B denoise, B=8, prompt 256, gen 128, 128 steps (cached and dense)")
        extra["c2_denoise_llada8b"] = bench_denoise(dev)
        log("C4 full model: LLaDA-8B, B=4, prompt 1024, gen 256, one 64-step block, head-sparse vs dense")
        extra["c4_denoise_llada8b_one_block"] = bench_denoise_c4(dev)
    cpu = None
    if not args.quick:
        log("CPU baseline (oracle)")
        cpu = cpu_baseline(lens, Hq, Hkv, D)
        cpu["value"] = round(cpu["value"], 4)
        cpu["seconds"] = round(cpu["seconds"], 4)
        log("CPU oracle on the other configurations' layer calls")
        extra["cpu_oracle_other_configs"] = cpu_other_configs()
    # The binding ceiling of the headline kernel: HBM when its arithmetic
    # intensity (algorithmic FLOPs / algorithmic bytes) is below the machine
    # balance peak_flops / peak_bw, else MFMA.
    kernel_name = "attn_dense_kernel<12, 1, 2, 32, 3>"
    intensity = r["flops_per_call"] / r["bytes_per_call"]
    balance = PEAK_BF16_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9)
    mfma_frac = r["tflops_kernel"] / PEAK_BF16_TFLOPS
    if intensity < balance:
        achieved = r["bytes_per_call"] / (r["kernel_us"] * 1e-6) / 1e9
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(achieved / PEAK_HBM_GBS, 4)}
    else:
        roof = {"bound": "mfma", "achieved": round(r["tflops_kernel"], 2), "peak": PEAK_BF16_TFLOPS,
                "unit": "TFLOP/s", "frac": round(mfma_frac, 4)}
    traffic, traffic_prov = measured_traffic(kernel_name)
    line = {
        "metric": METRIC,
        "value": round(r["tflops_step"], 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "LLaDA-8B dense denoise-step attention: 32 layers x 8 sequences x 384 tokens "
                               "(prompt 256 + gen 128), 32 heads x 128, non-causal varlen",
                   "global_batch": 8, "seq_len": 384, "layers": n_layers},
        "roofline": dict(roof, traffic=traffic, traffic_recorded_on=traffic_prov, kernel=kernel_name,
                         kernel_us=round(r["kernel_us"], 3), flops_per_launch=r["flops_per_call"],
                         algorithmic_bytes_per_launch=r["bytes_per_call"],
                         arithmetic_intensity=round(intensity, 1), machine_balance=round(balance, 1),
                         kernel_tflops=round(r["tflops_kernel"], 2), mfma_frac=round(mfma_frac, 4)),
        "clock_control": clock,
        "cpu_baseline": cpu,
        "gpu_settle_s": SETTLE_S,
    }
    line["headline_step_as_hip_graph"] = dict(ms_per_step=round(r["ms_per_step_graph"], 4),
                                              tflops=round(r["tflops_step_graph"], 2))
    line.update(extra)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
