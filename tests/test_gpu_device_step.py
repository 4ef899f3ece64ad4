"""Device-side step metadata (dllm_step_build / dllm_step_advance) and whole
denoising steps replayed from captured HIP graphs.

* Over many steps of a mixed batch (no SparseConfig, and sparse sequences
  with delay_step 0 / 1 / 3, block lengths 4 / 8 / 16, several retention
  ratios and prompt lengths), the tables the device builds equal the ones the
  host path builds (StepPlan from prepare_step's Context, prepare_step's
  positions, step_windows) and the device state advanced by the kernel
  equals the host Sequence objects' state, entry for entry.  The same tables
  are also checked against oracle.step (rows, positions, cu_seqlens_k, slot
  lists, selection jobs, cached segments).
* A tiny model (2 layers, 2 heads x 128, vocabulary 1024) denoises a mixed
  batch eagerly on the host path and again with StepGraphs (device tables,
  steps captured once per launch shape and replayed); the generated tokens
  are identical."""
import numpy as np
import pytest
import torch

from oracle import step as ostep

from dllm_serve_amd import _capi
from dllm_serve_amd.engine.device_step import DeviceStepState, StepGraphs, state_row
from dllm_serve_amd.engine.sampler import RemaskSampler, sample_device_windows, step_windows
from dllm_serve_amd.engine.sequence import PageAllocator, Sequence, prepare_step
from dllm_serve_amd.layers.attention import Attention, StepPlan
from dllm_serve_amd.layers.rotary_embedding import RotaryEmbedding
from dllm_serve_amd.sparse.state import SparseConfig
from dllm_serve_amd.utils.context import get_context, reset_context

pytestmark = pytest.mark.gpu

MASK = 1000


def _batch(dev, specs, steps=None):
    seqs = []
    for P, gen, cfg in specs:
        seqs.append(Sequence(list(range(1, P + 1)), gen, MASK, cfg, device=dev, steps=steps or gen))
    pages = sum(s.num_blocks for s in seqs) + 2
    alloc = PageAllocator(reversed(range(pages)))          # shuffled-looking page ids
    for s in seqs:
        alloc.allocate(s)
    return seqs, pages


def _np(t):
    return t.cpu().numpy()


def _mirror(s):
    st = s.sparse_state
    cfg = None if st is None else ostep.Cfg(st.config.default_block_len, st.config.retention_ratio,
                                            st.config.delay_step)
    return ostep.SparseSeq(s.num_prompt_tokens, s.num_tokens, s.block_table if st is not None else (), cfg)


def _check_tables_against_oracle(t, mirrors, step):
    """Device-built tables of one step against oracle.step."""
    per, cu = ostep.step_inputs(mirrors)
    p = t.plan
    assert list(_np(p.cu)) == list(cu), f"step {step}: cu"
    assert np.array_equal(_np(t.positions), np.concatenate([q for _, q, _ in per])), f"step {step}: positions"
    jobs = _np(p.jobs)[:8 * p.n_job].reshape(-1, 8)
    slots = _np(p.slots)
    cached = list(_np(p.cached_ids)[:p.n_cached])
    slot_off = _np(p.slot_off)
    dense = set(_np(p.dense_ids)[:p.n_dense].tolist())
    for i, (mode, q, sl) in enumerate(per):
        assert (i in dense) == (mode in (0, 1)), (step, i)
        if mode == 1:
            row = [r for r in jobs if r[0] == cu[i]]
            assert len(row) == 1, (step, i)
            bs, bl = mirrors[i].span()
            assert list(row[0][1:5]) == [len(q), bs, bl, len(sl)], (step, i)
            assert list(slots[row[0][5]:row[0][5] + len(sl)]) == sl, (step, i)
        elif mode == 2:
            r = cached.index(i)
            assert list(slots[slot_off[r]:slot_off[r + 1]]) == sl, (step, i)


def test_device_tables_equal_host_tables(dev):
    cfgs = [None,
            SparseConfig(default_block_len=8, retention_ratio=0.5, delay_step=1, head_select=True),
            SparseConfig(default_block_len=4, retention_ratio=0.3, delay_step=0, pool_kernel=1),
            SparseConfig(default_block_len=16, retention_ratio=0.75, delay_step=3, head_select=True),
            SparseConfig(default_block_len=8, retention_ratio=1.0, delay_step=1, head_select=True)]
    specs = [(37, 24, cfgs[0]), (50, 32, cfgs[1]), (29, 16, cfgs[2]), (300, 64, cfgs[3]), (5, 40, cfgs[4]),
             (64, 32, cfgs[1])]
    seqs, _ = _batch(dev, specs, steps=16)
    N = max(s.num_tokens for s in seqs) + 3
    ds = DeviceStepState(seqs, dev, N)
    mirrors = [_mirror(s) for s in seqs]
    checked = 0
    for step in range(16):
        print(f"device tables step {step}", flush=True)
        try:
            t = ds.build(seqs)  # steps may mix head_select / pool_kernel across sequences
        except (ZeroDivisionError, RuntimeError, ValueError):
            t = None
        if t is not None:
            ids, pos = prepare_step(seqs, dev)
            host = StepPlan(get_context(), torch.device(dev))
            reset_context()
            torch.cuda.synchronize()
            p = t.plan
            assert _np(t.counts)[6] == 0 and _np(t.counts)[7] == 0
            assert np.array_equal(_np(p.cu), _np(host.cu))
            assert np.array_equal(_np(p.dense_ids)[:host.n_dense], _np(host.dense_ids)[:host.n_dense])
            assert np.array_equal(_np(p.cached_ids)[:host.n_cached], _np(host.cached_ids)[:host.n_cached])
            assert np.array_equal(_np(p.slot_off), _np(host.slot_off))
            nj = _capi.JOB_COLS * host.n_job
            assert np.array_equal(_np(p.jobs)[:nj], _np(host.jobs)[:nj])
            n_sl = t.layout.total_slots
            assert np.array_equal(_np(p.slots)[:n_sl], _np(host.slots)[:n_sl])
            assert np.array_equal(_np(t.positions), _np(pos))
            starts = [s.step_rows()[0] for s in seqs]
            want_ti = np.concatenate([b * N + starts[b] + np.arange(n) for b, n in enumerate(t.layout.rows)])
            assert np.array_equal(_np(t.token_index), want_ti)
            tok_flat = np.concatenate([np.array(s.token_ids + [0] * (N - s.num_tokens)) for s in seqs])
            assert np.array_equal(tok_flat[_np(t.token_index)], _np(ids))
            wins = step_windows(seqs)
            r = 0
            want_p, want_rows = [], []
            for b, (h0, lo, n, sr, first) in enumerate(wins):
                want_p.append((b * N + lo, n, r, sr, first))
                want_rows.extend(range(h0, h0 + n))
                r += n
            assert np.array_equal(_np(t.smp_params), np.array(want_p, np.int32))
            assert np.array_equal(_np(t.smp_rows), np.array(want_rows, np.int64))
            _check_tables_against_oracle(t, mirrors, step)
            checked += 1
        ds.advance()
        for s, m in zip(seqs, mirrors):
            s.advance()
            if m.cfg is not None:
                m.advance()
        torch.cuda.synchronize()
        assert np.array_equal(_np(ds.state), np.array([state_row(s) for s in seqs], np.int32)), f"step {step}"
    assert checked >= 8


class TinyDLM:
    """2-layer bidirectional transformer with our attention, RoPE and sampler
    (random weights): a caller of the path for the capture test."""

    def __init__(self, dev, H=256, heads=2, D=128, F=512, V=1024, layers=2, seed=0):
        g = torch.Generator(device=dev).manual_seed(seed)

        def w(*shape):
            return torch.randn(*shape, generator=g, device=dev, dtype=torch.bfloat16) * 0.05

        self.wte, self.lm_head = w(V, H), w(V, H)
        self.layers = [dict(qkv=w(3 * H, H), o=w(H, H), up=w(2 * F, H), down=w(H, F)) for _ in range(layers)]
        self.attn = [Attention(heads, D, D ** -0.5, heads, causal=False) for _ in range(layers)]
        self.rope = RotaryEmbedding(D, D, 4096, 10000.0, inplace=True).to(dev)
        self.H, self.heads, self.D, self.F = H, heads, D, F
        bias = torch.zeros(V, device=dev, dtype=torch.bfloat16)
        bias[MASK] = -1e4                     # never predict the mask token itself
        self.sampler = RemaskSampler(lambda h: h @ self.lm_head.t() + bias, MASK)

    def bind_cache(self, pages, dev):
        self.kv = torch.zeros(2, len(self.layers), pages, 256, self.heads, self.D, dtype=torch.bfloat16, device=dev)
        for i, a in enumerate(self.attn):
            a.k_cache, a.v_cache = self.kv[0, i], self.kv[1, i]

    def forward(self, ids, pos):
        H, n = self.H, ids.shape[0]
        h = self.wte[ids]
        for L, a in zip(self.layers, self.attn):
            qkv = h @ L["qkv"].t()
            q, k = self.rope(pos, qkv[:, :H], qkv[:, H:2 * H])
            h = h + a(q, k, qkv[:, 2 * H:]) @ L["o"].t()
            u = h @ L["up"].t()
            h = h + (torch.nn.functional.silu(u[:, :self.F]) * u[:, self.F:]) @ L["down"].t()
        return h


def _specs():
    c1 = SparseConfig(default_block_len=8, retention_ratio=0.5, delay_step=1, head_select=True)
    c2 = SparseConfig(default_block_len=8, retention_ratio=1.0, delay_step=1, head_select=True)
    return [(40, 32, c1), (70, 32, c1), (33, 32, c2), (50, 32, None)]


def test_graph_replayed_denoise_matches_eager(dev):
    steps = 32
    outs = []
    for mode in ("eager", "graph"):
        print(f"tiny denoise {mode}", flush=True)
        seqs, pages = _batch(dev, _specs(), steps=steps)
        model = TinyDLM(dev)
        model.bind_cache(pages, dev)
        N = max(s.num_tokens for s in seqs)
        tok = torch.zeros(len(seqs), N, dtype=torch.int64)
        for b, s in enumerate(seqs):
            tok[b, :s.num_tokens] = torch.tensor(s.token_ids)
        tok = tok.to(dev)
        if mode == "eager":
            for _ in range(steps):
                rows = [s.step_rows() for s in seqs]
                ids = torch.cat([tok[i, a:a + n] for i, (a, n) in enumerate(rows)])
                pos = torch.cat([torch.arange(a, a + n, device=dev) for a, n in rows])
                prepare_step(seqs, dev, build_inputs=False)
                hidden = model.forward(ids, pos)
                reset_context()
                model.sampler(hidden, seqs, tok)
                for s in seqs:
                    s.advance()
        else:
            ds = DeviceStepState(seqs, dev, tok.stride(0))

            def step_fn(t):
                hidden = model.forward(tok.view(-1).index_select(0, t.token_index), t.positions)
                sample_device_windows(model.sampler, hidden, tok, t.smp_rows, t.smp_params, t.max_win)

            graphs = StepGraphs(ds, step_fn)
            for _ in range(steps):
                graphs.run(seqs)
                for s in seqs:
                    s.advance()
            assert graphs.replays >= steps // 2 and len(graphs.graphs) >= 2
        torch.cuda.synchronize()
        outs.append(tok.cpu().numpy())
    assert not np.any(outs[0] == MASK), "eager run left masked positions"
    assert np.array_equal(outs[0], outs[1])
