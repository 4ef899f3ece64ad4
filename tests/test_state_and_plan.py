"""Host logic on the CPU: the sparse state machine, request sizing, slot
maps, the per-step launch plan and the no-CPU-fallback rule.  Expected
values are hand-derived from the reference's rules (sparse/state.py:44-104,
engine/sequence.py:87-152, engine/model_runner.py:257-302)."""
import pytest
import torch

from dllm_serve_amd.engine.sequence import PageAllocator, Sequence, prepare_step, slot_mapping_for
from dllm_serve_amd.layers.attention import Attention, StepLayout, StepPlan, store_kvcache
from dllm_serve_amd.sparse.state import PerRequestSparseState, SparseConfig, keep_count
from dllm_serve_amd.utils.context import get_context, reset_context, set_context

MASK = 126336


def _states(delay, block_len, steps):
    st = PerRequestSparseState(0, SparseConfig(default_block_len=block_len, delay_step=delay), "cpu")
    out = []
    for _ in range(steps):
        out.append((st.cache_state, st.current_block_idx))
        st.advance_step()
    return out


def test_state_tables():
    assert [s for s, _ in _states(1, 4, 9)] == [0, 1, 2, 2, 0, 1, 2, 2, 0]
    assert [b for _, b in _states(1, 4, 9)] == [0, 0, 0, 0, 1, 1, 1, 1, 2]
    # delay 0: the first block starts in state 0 and never computes (reference behaviour)
    assert [s for s, _ in _states(0, 4, 9)] == [0, 2, 2, 2, 1, 2, 2, 2, 1]
    assert [s for s, _ in _states(2, 4, 9)] == [0, 0, 1, 2, 0, 0, 1, 2, 0]
    assert [s for s, _ in _states(5, 4, 9)] == [0] * 9
    assert [s for s, _ in _states(1, 16, 34)][15:19] == [2, 0, 1, 2]


def test_block_boundaries_and_unused_counts():
    st = PerRequestSparseState(0, SparseConfig(default_block_len=8), "cpu")
    spans = []
    for b in range(4):
        st.current_block_idx = b
        spans.append((st.compute_block_boundaries(10, 30), st.block_span(10, 30), st.num_unused_tokens(10, 30)))
    assert spans[0] == ((10, 8), (10, 8), 22)
    assert spans[2] == ((26, 4), (26, 4), 26)
    assert spans[3] == ((34, -4), (34, 0), 34)   # past the end: the reference's own over-count
    for b in range(4):
        st.current_block_idx = b
        assert st.num_unused_tokens(10, 30) == len(st.get_unuse_block_indices(10, 30))
        if b < 3:
            assert st.block_span(10, 30)[1] == len(st.get_block_indices(10, 30))
        else:  # torch.arange(34, 30) raises, as the reference's block indices do past the end
            with pytest.raises(RuntimeError):
                st.get_block_indices(10, 30)
    assert st.compute_block_boundaries(10, 10) == (10, 0)


def test_keep_count():
    assert keep_count(1216, 0.5) == 608
    assert keep_count(133, 0.3) == 39          # int(39.9)
    assert keep_count(33, 0.0) == 1
    assert keep_count(0, 0.5) == 0
    assert keep_count(10, 1.0) == 10


def test_sequence_sizing_c4_and_slots():
    cfg = SparseConfig(enabled=True, default_block_len=64, retention_ratio=0.5, head_select=True)
    s = Sequence([1] * 1024, 256, MASK, cfg, device="cpu")
    assert s.num_tokens == 1280 and s.max_sparse_token == 640 and s.num_blocks == 3
    s.sparse_state.cache_state = 1
    assert s.current_sparse_token == 608
    assert s.num_should_cached_blocks == 3 and s.last_block_num_tokens_cached_sparse == 96
    s.block_table = [7, 3, 9]
    slots = slot_mapping_for(s)
    assert slots == list(range(7 * 256, 8 * 256)) + list(range(3 * 256, 4 * 256)) + list(range(9 * 256, 9 * 256 + 96))
    s.sparse_state.cache_state = 0
    with pytest.raises(NotImplementedError):
        s.num_should_cached_blocks
    assert Sequence([1] * 10, 5, MASK, None, device="cpu").max_sparse_token == 0


def test_page_allocator_order():
    cfg = SparseConfig(retention_ratio=0.5)
    alloc = PageAllocator([4, 1, 3, 0, 2])
    a = Sequence([1] * 600, 100, MASK, cfg, device="cpu")   # ceil(700*0.5)=350 -> 2 pages
    b = Sequence([1] * 100, 50, MASK, cfg, device="cpu")    # 75 -> 1 page
    alloc.allocate(a)
    alloc.allocate(b)
    assert a.block_table == [4, 1] and b.block_table == [3]
    with pytest.raises(RuntimeError):
        alloc.allocate(Sequence([1] * 2000, 0, MASK, cfg, device="cpu"))
    alloc.release(a)
    assert list(alloc.free)[:2] == [4, 1]


def _mixed_seqs():
    hs = SparseConfig(enabled=True, default_block_len=32, retention_ratio=0.5, head_select=True)
    A = Sequence([1] * 100, 64, MASK, None, device="cpu")   # dense, 164 rows
    B = Sequence([2] * 200, 64, MASK, hs, device="cpu")     # 264 rows
    C = Sequence([3] * 150, 64, MASK, hs, device="cpu")     # 214 rows
    alloc = PageAllocator([5, 2, 7, 0])
    alloc.allocate(B)
    alloc.allocate(C)
    return A, B, C


def test_step_plan_tables():
    A, B, C = _mixed_seqs()
    B.sparse_state.cache_state = 2   # reuse: feeds its block only
    C.sparse_state.cache_state = 1   # compute + store
    prepare_step([A, B, C], "cpu")
    ctx = get_context()
    plan = StepPlan(ctx, torch.device("cpu"), 32, 128, 32)
    assert plan.total_rows == 164 + 32 + 214
    assert plan.cu.tolist() == [0, 164, 196, 410]
    # dense segments longest first: C (214 rows) before A (164)
    assert plan.n_dense == 2 and plan.dense_ids.tolist() == [2, 0] and plan.max_q_dense == 214
    assert plan.n_cached == 1 and plan.cached_ids.tolist() == [1]
    n_b = keep_count(264 - 32, 0.5)   # 116
    n_c = keep_count(214 - 32, 0.5)   # 91
    assert plan.slot_off.tolist() == [0, n_b]
    assert plan.slots.tolist() == list(range(5 * 256, 5 * 256 + n_b)) + list(range(2 * 256, 2 * 256 + n_c))
    # row0, n_tok, blk_start, blk_len, n_keep, slot_off, head_select, pool_k
    assert plan.n_job == 1 and plan.jobs.tolist() == [196, 214, 150, 32, n_c, n_b, 1, 3]
    assert plan.max_kc == 182 and plan.max_keep == n_c
    assert plan.max_q_cached == 32 and plan.max_keys_cached == 32 + n_b
    reset_context()


def test_step_plan_mixes_sparse_configs():
    """Sequences of one step with different head_select / pool_kernel: each
    selection job carries its own (the reference reads both per sequence,
    attention.py:211,329,387)."""
    cfgs = [SparseConfig(enabled=True, default_block_len=32, retention_ratio=0.5, head_select=True, pool_kernel=1),
            SparseConfig(enabled=True, default_block_len=16, retention_ratio=0.25, head_select=False, pool_kernel=5),
            SparseConfig(enabled=True, default_block_len=32, retention_ratio=1.0, head_select=True, pool_kernel=3)]
    seqs = [Sequence([i + 1] * (100 + 40 * i), 64, MASK, c, device="cpu") for i, c in enumerate(cfgs)]
    seqs.append(Sequence([9] * 50, 32, MASK, None, device="cpu"))
    alloc = PageAllocator(range(8))
    for s_ in seqs[:3]:
        alloc.allocate(s_)
        s_.sparse_state.cache_state = 1
    prepare_step(seqs, "cpu")
    plan = StepPlan(get_context(), torch.device("cpu"), 32, 128, 32)
    jobs = plan.jobs.view(-1, 8).tolist()
    assert plan.n_job == 3 and [j[6:] for j in jobs] == [[1, 1], [0, 5], [1, 3]]
    assert [j[4] for j in jobs] == [keep_count(164 - 32, 0.5), keep_count(204 - 16, 0.25), 244 - 32]
    lay = StepLayout(seqs)
    assert lay.signature()[-1] == ((True, 1), (False, 5), (True, 3))
    reset_context()


def test_step_plan_errors():
    A, B, C = _mixed_seqs()
    B.sparse_state.cache_state = 1
    prepare_step([A, B, C], "cpu")
    ctx = get_context()
    ctx.slot_mapping[1] = ctx.slot_mapping[1][:-1]   # one slot short
    with pytest.raises(AssertionError):
        StepPlan(ctx, torch.device("cpu"), 32, 128, 32)
    # cache state 1 with the block past the end of the sequence
    B.sparse_state.current_block_idx = 5
    prepare_step([A, B], "cpu")
    with pytest.raises(ValueError):
        StepPlan(get_context(), torch.device("cpu"), 32, 128, 32)
    reset_context()


def test_no_cpu_fallback():
    attn = Attention(4, 128, 128 ** -0.5, 4, causal=False)
    A = Sequence([1] * 8, 8, MASK, None, device="cpu")
    prepare_step([A], "cpu")
    x = torch.zeros(16, 4 * 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU"):
        attn(x, x, x)
    reset_context()
    set_context(True, is_diffusion=False)
    with pytest.raises(NotImplementedError):
        attn(x, x, x)
    reset_context()
    k = torch.zeros(4, 2, 128, dtype=torch.bfloat16)
    cache = torch.zeros(1, 256, 2, 128, dtype=torch.bfloat16)
    with pytest.raises(AssertionError):   # slot count mismatch, as the reference asserts
        store_kvcache(k, k, cache, cache, torch.zeros(3, dtype=torch.int32))
    with pytest.raises(RuntimeError, match="GPU"):
        store_kvcache(k, k, cache, cache, torch.zeros(4, dtype=torch.int32))
