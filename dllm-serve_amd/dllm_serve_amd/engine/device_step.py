"""Device-side step metadata and captured denoising steps.

The reference rebuilds every step's inputs on the host: per-sequence row and
position lists, slot lists uploaded one sequence at a time, the mode tables
of _mixed_sparse_dense_attention, and the sampler's windows with ``.item()``
reads (dllmserve/engine/model_runner.py:231-321,756-949,
dllmserve/layers/attention.py:168-265).  Here a device table holds each
sequence's state (prompt and total length, block length and index, step in
block, cache state, delay, steps, current step), and two kernels replace that
host work:

* ``dllm_step_build`` writes the step's attention launch tables (the same
  tables ``StepPlan`` uploads from the host), the positions and token-table
  indices of the fed rows, and the sampler's windows;
* ``dllm_step_advance`` advances every sequence's state after the step
  (scheduler.py:117-120, state.py:77-104).

The host keeps its own ``Sequence`` objects in step (their state machine is
deterministic) only for launch sizes and validation; it reads nothing back.
A whole step -- tables, embedding gather, forward, sampler, advance -- then
depends on no host data and can be captured once per distinct launch shape
(``StepLayout.signature``) and replayed: ``StepGraphs``.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Callable

import torch

from .. import _capi
from ..layers.attention import StepLayout, StepPlan
from ..utils.context import get_context, reset_context, set_context
from .sampler import MAX_WINDOW, step_windows

STATE_COLS = 12


def state_row(seq) -> list[int]:
    """The device state of one sequence (column order of dllm_step_build)."""
    st = seq.sparse_state
    steps = seq.sampling_params.steps if getattr(seq, "sampling_params", None) is not None else seq.steps
    if st is None:
        return [seq.num_prompt_tokens, seq.num_tokens, 0, 1, 0, 0, 0, 0, steps, seq.current_step, 0, 1]
    return [seq.num_prompt_tokens, seq.num_tokens, 1, st.block_len, st.current_block_idx, st.step_in_block,
            st.cache_state, st.config.delay_step, steps, seq.current_step, int(bool(st.config.head_select)),
            int(st.config.pool_kernel)]


@dataclass
class StepTables:
    layout: StepLayout
    plan: StepPlan
    positions: torch.Tensor     # int64 [rows]
    token_index: torch.Tensor   # int64 [rows]
    smp_params: torch.Tensor    # int32 [n_seq, 5]
    smp_rows: torch.Tensor      # int64 [window positions]
    max_win: int
    counts: torch.Tensor        # int32 [8]


class DeviceStepState:
    """Device state and table buffers of one batch of sequences.

    ``tok_stride`` is the row stride of the caller's [B, N_max] int64 token
    table.  Buffers are sized once from the sequences (all their tokens) and
    reused every step, so their addresses stay fixed for graph replay."""

    def __init__(self, seqs, device, tok_stride: int):
        if not seqs:
            raise ValueError("no sequences")
        self.device = torch.device(device)
        if self.device.type == "cuda" and self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.n = n = len(seqs)
        for s in seqs:
            if s.sparse_state is not None and s.sparse_state.block_len < 1:
                raise ValueError("block_len must be >= 1")
        host = torch.tensor([state_row(s) for s in seqs], dtype=torch.int32)
        self.state = host.to(self.device)
        self.ratio = torch.tensor([s.sparse_state.retention_ratio if s.sparse_state is not None else 0.0
                                   for s in seqs], dtype=torch.float64, device=self.device)
        pages, off = [], [0]
        for s in seqs:
            pages.extend(s.block_table if s.sparse_state is not None else [])
            off.append(len(pages))
        self.pages = torch.tensor(pages or [0], dtype=torch.int32, device=self.device)
        self.page_off = torch.tensor(off, dtype=torch.int32, device=self.device)
        self.tok_stride = int(tok_stride)
        rows_cap = sum(s.num_tokens for s in seqs)
        slots_cap = max(1, sum(s.num_tokens for s in seqs if s.sparse_state is not None))
        m = max(1, n)
        jc = _capi.JOB_COLS
        i32 = torch.zeros((n + 1) + m + m + (n + 1) + jc * m + 5 * n + 8, dtype=torch.int32, device=self.device)
        o = 0

        def take(k):
            nonlocal o
            v = i32[o:o + k]
            o += k
            return v

        self.cu, self.dense_ids, self.cached_ids = take(n + 1), take(m), take(m)
        self.slot_off, self.jobs = take(n + 1), take(jc * m)
        self.smp_params, self.counts = take(5 * n).view(n, 5), take(8)
        self.slots = torch.zeros(slots_cap, dtype=torch.int32, device=self.device)
        self.positions = torch.zeros(rows_cap, dtype=torch.int64, device=self.device)
        self.token_index = torch.zeros(rows_cap, dtype=torch.int64, device=self.device)
        self.smp_rows = torch.zeros(rows_cap, dtype=torch.int64, device=self.device)

    def build(self, seqs) -> StepTables:
        """Enqueue the table builder for the step the sequences are at (the
        host objects give launch sizes and are validated as the host path
        would; the device reads its own state table)."""
        if len(seqs) != self.n:
            raise ValueError("batch changed; build a new DeviceStepState")
        lay = StepLayout(seqs)
        if lay.any_skipped:
            raise ValueError("a sequence is in an unrecognised cache state")
        wins = step_windows(seqs)
        if any(w[2] > MAX_WINDOW for w in wins):
            raise ValueError(f"window exceeds {MAX_WINDOW} positions")
        n_win = sum(w[2] for w in wins)
        _capi.step_build(self.state, self.ratio, self.pages, self.page_off, self.n, self.tok_stride, self.cu,
                         self.dense_ids, self.cached_ids, self.slot_off, self.jobs, self.slots, self.positions,
                         self.token_index, self.smp_params, self.smp_rows, self.counts)
        plan = StepPlan.from_device(lay, self.device, self.cu, self.dense_ids[:max(1, lay.n_dense)],
                                    self.cached_ids[:max(1, lay.n_cached)], self.slot_off[:lay.n_cached + 1],
                                    self.jobs[:_capi.JOB_COLS * max(1, lay.n_job)], self.slots)
        return StepTables(lay, plan, self.positions[:lay.total_rows], self.token_index[:lay.total_rows],
                          self.smp_params, self.smp_rows[:n_win], max((w[2] for w in wins), default=0),
                          self.counts)

    def advance(self) -> None:
        _capi.step_advance(self.state, self.n)


def install_context(seqs, tables: StepTables) -> None:
    """The Context the layers read, with the device-built plan attached."""
    set_context(True, cu_seqlens_q=None, cu_seqlens_k=tables.plan.cu, max_seqlen_q=0,
                max_seqlen_k=tables.layout.total_rows, slot_mapping=[], is_diffusion=True, seqs=seqs)
    get_context()._dllm_plan = tables.plan


class StepGraphs:
    """Denoising steps replayed from captured HIP graphs.

    ``step_fn(tables)`` must enqueue one step's device work (forward and
    sampler) from the tables only.  ``run(seqs)`` builds the tables, runs
    ``step_fn`` and advances the device state; the first time a launch shape
    is seen the step runs eagerly (warming up libraries and workspaces), the
    second time it is captured, and afterwards it is replayed.  The caller
    advances its host ``Sequence`` objects after each call, as the
    scheduler does."""

    def __init__(self, dstate: DeviceStepState, step_fn: Callable[[StepTables], None]):
        self.dstate = dstate
        self.step_fn = step_fn
        self.seen: set = set()
        self.graphs: dict = {}
        self.replays = 0

    def _body(self, seqs) -> StepTables:
        t = self.dstate.build(seqs)
        install_context(seqs, t)
        self.step_fn(t)
        reset_context()
        self.dstate.advance()
        return t

    def run(self, seqs) -> None:
        key = StepLayout(seqs).signature()
        g = self.graphs.get(key)
        if g is not None:
            g.replay()
            self.replays += 1
            return
        if key not in self.seen:
            self.seen.add(key)
            self._body(seqs)
            return
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self._body(seqs)
        self.graphs[key] = g
        g.replay()
        self.replays += 1
