"""Attention.forward inside a captured HIP graph.

After one eager call per step (which builds the step's launch tables and
workspaces), the layer's launches record into a graph: nothing in the path
synchronises, copies from the host or sets memory.  Each graph is replayed
several times with new q/k/v copied into its static inputs between replays
(eager work and synchronisation in between), and every replay must equal
the eager calls on the same inputs bit for bit -- outputs and, for the
select-and-store step, the KV cache."""
import pytest
import torch

from dllm_serve_amd.engine.sequence import PageAllocator, Sequence, prepare_step
from dllm_serve_amd.layers.attention import Attention
from dllm_serve_amd.sparse.state import SparseConfig
from dllm_serve_amd.utils.context import reset_context

pytestmark = pytest.mark.gpu

MASK = 126336


@pytest.mark.parametrize("Hq,Hkv", [(32, 32), (28, 4)])
def test_layer_calls_replay_in_a_graph(dev, Hq, Hkv):
    D = 128
    layers = 3
    attn = Attention(Hq, D, D ** -0.5, Hkv, causal=False)
    cache = torch.zeros(2, 8, 256, Hkv, D, dtype=torch.bfloat16, device=dev)
    attn.k_cache, attn.v_cache = cache[0], cache[1]
    cfg = SparseConfig(enabled=True, default_block_len=32, retention_ratio=0.5, pool_kernel=3, delay_step=1,
                       head_select=True)
    seqs = [Sequence([1] * 100, 64, MASK, None, device=dev), Sequence([2] * 200, 64, MASK, cfg, device=dev),
            Sequence([3] * 150, 64, MASK, cfg, device=dev)]
    alloc = PageAllocator(range(8))
    for s in seqs[1:]:
        alloc.allocate(s)
    g = torch.Generator().manual_seed(11)

    def fresh(n, h):
        return torch.randn(n, h * D, generator=g).to(torch.bfloat16)

    # step 0: full attention everywhere (eager only)
    prepare_step(seqs, dev)
    n0 = 164 + 264 + 214
    attn(fresh(n0, Hq).to(dev), fresh(n0, Hkv).to(dev), fresh(n0, Hkv).to(dev))
    reset_context()
    for s in seqs:
        s.advance()

    # step 1: select + store (state 1), step 2: block vs cache (state 2); one graph each
    for step, n in ((1, n0), (2, 164 + 32 + 32)):
        print(f"graph step {step} Hq={Hq} Hkv={Hkv}", flush=True)
        prepare_step(seqs, dev)
        qs = [fresh(n, Hq).to(dev) for _ in range(layers)]
        ks = [fresh(n, Hkv).to(dev) for _ in range(layers)]
        vs = [fresh(n, Hkv).to(dev) for _ in range(layers)]
        for i in range(layers):  # warm-up: launch tables, workspaces, kernel attributes
            attn(qs[i], ks[i], vs[i])
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            outs = [attn(qs[i], ks[i], vs[i]) for i in range(layers)]
        for rep in range(3):
            for i in range(layers):
                qs[i].copy_(fresh(n, Hq))
                ks[i].copy_(fresh(n, Hkv))
                vs[i].copy_(fresh(n, Hkv))
            graph.replay()
            torch.cuda.synchronize()
            got = [o.clone() for o in outs]
            got_cache = cache.clone()
            want = [attn(qs[i], ks[i], vs[i]) for i in range(layers)]
            torch.cuda.synchronize()
            for i in range(layers):
                assert torch.equal(got[i], want[i]), f"step {step} replay {rep} layer {i}"
            assert torch.equal(got_cache, cache), f"step {step} replay {rep}: cache"
        del graph
        reset_context()
        for s in seqs:
            s.advance()
