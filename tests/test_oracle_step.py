"""oracle.step (the per-step inputs of a batch) pinned to hand-derived values
from the reference's rules (sparse/state.py:42-104,123-144,
engine/sequence.py:87-152, engine/model_runner.py:240-302), then the host
planner (prepare_step, StepPlan) checked against it over a mixed batch."""
import numpy as np
import pytest
import torch

from oracle import step as ostep
from dllm_serve_amd.engine.sequence import PageAllocator, Sequence, prepare_step
from dllm_serve_amd.layers.attention import StepPlan
from dllm_serve_amd.sparse.state import SparseConfig
from dllm_serve_amd.utils.context import get_context, reset_context

MASK = 126336


def _states(delay, block_len, steps):
    s = ostep.SparseSeq(10, 10 + 4 * block_len, cfg=ostep.Cfg(block_len, 0.5, delay))
    out = []
    for _ in range(steps):
        out.append((s.state, s.blk))
        s.advance()
    return out


def test_oracle_state_sequences():
    # delay 1: 0 at a block's first step, 1 at its second, 2 after
    assert [x for x, _ in _states(1, 4, 9)] == [0, 1, 2, 2, 0, 1, 2, 2, 0]
    assert [b for _, b in _states(1, 4, 9)] == [0, 0, 0, 0, 1, 1, 1, 1, 2]
    # delay 0: 1 at a block's first step, 2 after -- the very first step is the initial 0
    assert [x for x, _ in _states(0, 4, 9)] == [0, 2, 2, 2, 1, 2, 2, 2, 1]
    # delay d >= 2: 0 below d, 1 at d, 2 above
    assert [x for x, _ in _states(2, 4, 9)] == [0, 0, 1, 2, 0, 0, 1, 2, 0]
    assert [x for x, _ in _states(5, 4, 9)] == [0] * 9


def test_oracle_spans_and_keep():
    s = ostep.SparseSeq(10, 30, cfg=ostep.Cfg(8, 0.5, 1))
    got = []
    for b in range(4):
        s.blk = b
        got.append((s.span(), s.unused()))
    assert got == [((10, 8), 22), ((18, 8), 22), ((26, 4), 26), ((34, -4), 34)]  # past the end: over-count
    assert ostep.SparseSeq(10, 10, cfg=ostep.Cfg(8, 0.5, 1)).span() == (10, 0)
    c4 = ostep.SparseSeq(1024, 1280, cfg=ostep.Cfg(64, 0.5, 1))
    assert c4.unused() == 1216 and c4.n_keep() == 608
    assert ostep.SparseSeq(100, 233, cfg=ostep.Cfg(100, 0.3, 1)).n_keep() == 39   # int(133 * 0.3) = int(39.9)
    assert ostep.SparseSeq(30, 33, cfg=ostep.Cfg(33, 0.0, 1)).n_keep() == 1      # at least one row


def test_oracle_slot_lists_and_inputs():
    c4 = ostep.SparseSeq(1024, 1280, pages=[7, 3, 9], cfg=ostep.Cfg(64, 0.5, 1))
    want = list(range(7 * 256, 8 * 256)) + list(range(3 * 256, 4 * 256)) + list(range(9 * 256, 9 * 256 + 96))
    assert c4.slot_list() == want                     # 608 = 256 + 256 + 96
    full = ostep.SparseSeq(100, 612, pages=[2, 5], cfg=ostep.Cfg(100, 1.0, 1))   # n_keep 512: two whole pages
    assert full.slot_list() == list(range(512, 768)) + list(range(1280, 1536))
    dense = ostep.SparseSeq(5, 9)
    c4.state = 2
    per, cu = ostep.step_inputs([dense, c4])
    assert per[0][0] == 0 and per[0][2] is None and list(per[0][1]) == list(range(9))
    assert per[1][0] == 2 and list(per[1][1]) == list(range(1024, 1088)) and per[1][2] == want
    assert list(cu) == [0, 9, 73]
    c4.state = 1
    per, cu = ostep.step_inputs([c4, dense])
    assert per[0][0] == 1 and len(per[0][1]) == 1280 and per[0][2] == want and list(cu) == [0, 1280, 1289]
    c4.blk = 5                                        # 1024 + 5 * 64 > 1280: past the end
    c4.state = 2
    with pytest.raises(ValueError):
        ostep.step_inputs([c4])


def _mirror(s):
    st = s.sparse_state
    cfg = None if st is None else ostep.Cfg(st.config.default_block_len, st.config.retention_ratio,
                                            st.config.delay_step)
    return ostep.SparseSeq(s.num_prompt_tokens, s.num_tokens, s.block_table if st is not None else (), cfg)


def test_host_planner_matches_oracle():
    """prepare_step + StepPlan against oracle.step over 40 steps of a mixed
    batch: rows, positions, slot lists, selection jobs and cached segments."""
    cfgs = [None, SparseConfig(default_block_len=8, retention_ratio=0.5, delay_step=1, head_select=True),
            SparseConfig(default_block_len=4, retention_ratio=0.3, delay_step=0, pool_kernel=1),
            SparseConfig(default_block_len=16, retention_ratio=0.75, delay_step=3),
            SparseConfig(default_block_len=8, retention_ratio=1.0, delay_step=1)]
    # generation lengths past 40 tokens: every one of the 40 steps has a block inside each sequence
    specs = [(37, 48, cfgs[0]), (50, 44, cfgs[1]), (29, 41, cfgs[2]), (300, 64, cfgs[3]), (5, 60, cfgs[4]),
             (600, 48, cfgs[1])]
    seqs = [Sequence(list(range(1, P + 1)), gen, MASK, c, device="cpu", steps=gen) for P, gen, c in specs]
    alloc = PageAllocator(reversed(range(sum(s.num_blocks for s in seqs) + 2)))
    for s in seqs:
        alloc.allocate(s)
    mirrors = [_mirror(s) for s in seqs]
    checked = 0
    for step in range(40):
        try:
            per, cu = ostep.step_inputs(mirrors)
        except ValueError:   # a block past the end, or state 1 with an empty block
            per = None
        if per is None:      # the planner refuses the same steps
            with pytest.raises((ValueError, RuntimeError)):
                prepare_step(seqs, "cpu")
                StepPlan(get_context(), torch.device("cpu"))
            reset_context()
        else:
            _, pos = prepare_step(seqs, "cpu")
            plan = StepPlan(get_context(), torch.device("cpu"))
            reset_context()
            assert list(plan.cu.numpy()) == list(cu), f"step {step}"
            assert np.array_equal(pos.numpy(), np.concatenate([p for _, p, _ in per]))
            jobs = plan.jobs.numpy().reshape(-1, 8)[:plan.n_job]
            slots = plan.slots.numpy()
            cached = list(plan.cached_ids.numpy()[:plan.n_cached])
            slot_off = plan.slot_off.numpy()
            dense = set(plan.dense_ids.numpy()[:plan.n_dense].tolist())
            for i, (mode, p, sl) in enumerate(per):
                assert (i in dense) == (mode in (0, 1)), (step, i)
                if mode == 1:
                    row = [r for r in jobs if r[0] == cu[i]]
                    assert len(row) == 1, (step, i)
                    j = row[0]
                    bs, bl = mirrors[i].span()
                    assert list(j[1:5]) == [len(p), bs, bl, len(sl)], (step, i)
                    assert list(slots[j[5]:j[5] + len(sl)]) == sl, (step, i)
                elif mode == 2:
                    r = cached.index(i)
                    assert list(slots[slot_off[r]:slot_off[r + 1]]) == sl, (step, i)
            checked += 1
        for s, m in zip(seqs, mirrors):
            s.advance()
            if m.cfg is not None:
                m.advance()
    assert checked == 40
