"""Request sizing and per-step inputs of the diffusion attention path.

``Sequence`` keeps the attribute names and the sparse sizing properties of
dllmserve/engine/sequence.py:19-152 (``num_tokens``, ``num_prompt_tokens``,
``sparse_state``, ``block_table``, ``max_sparse_token``,
``current_sparse_token``, ``num_blocks``, ``num_should_cached_blocks``,
``last_block_num_tokens_cached_sparse``); the scheduling/status fields the
path does not read are omitted.

``slot_mapping_for`` restates the slot lists of
dllmserve/engine/model_runner.py:257-273,287-302 and ``prepare_step`` the
packed inputs and Context of model_runner.py:231-321, so tests and benchmarks
drive ``Attention`` exactly as the reference runner does.  ``PageAllocator``
hands out 256-row cache pages from a free list in order, like
BlockManager.allocate_sparse (block_manager.py:64-68).
"""
from __future__ import annotations

import math
from collections import deque
from itertools import count
from typing import Iterable, Optional

import torch

from ..sparse.state import PerRequestSparseState, SparseConfig, keep_count
from ..utils.context import set_context


class Sequence:
    block_size = 256
    counter = count()

    def __init__(self, token_ids: list[int], gen_length: int, mask_token_id: int,
                 sparse_config: Optional[SparseConfig] = None, device="cuda", steps: Optional[int] = None):
        self.seq_id = next(Sequence.counter)
        self.num_prompt_tokens = len(token_ids)
        self.token_ids = list(token_ids) + [mask_token_id] * gen_length
        self.num_tokens = len(self.token_ids)
        self.gen_length = gen_length
        self.steps = gen_length if steps is None else steps
        self.current_step = 0
        self.sparse_state = (
            PerRequestSparseState(self.seq_id, sparse_config, device) if sparse_config is not None else None
        )
        self.block_table: list[int] = []

    def __len__(self) -> int:
        return self.num_tokens

    # ---- sparse sizing (sequence.py:87-152) -------------------------------
    @property
    def max_sparse_token(self) -> int:
        if self.sparse_state is None:
            return 0
        return max(1, math.ceil(self.num_tokens * self.sparse_state.retention_ratio))

    @property
    def current_sparse_token(self) -> int:
        if self.sparse_state is None:
            return 0
        unused = self.sparse_state.num_unused_tokens(self.num_prompt_tokens, self.num_tokens)
        return keep_count(unused, self.sparse_state.retention_ratio)

    @property
    def num_blocks(self) -> int:
        if self.sparse_state is None:
            return 0
        return (self.max_sparse_token + self.block_size - 1) // self.block_size

    @property
    def num_should_cached_blocks(self) -> int:
        st = self.sparse_state
        if st is not None and (st.should_compute_cache or st.should_reuse_cache):
            return (self.current_sparse_token + self.block_size - 1) // self.block_size
        raise NotImplementedError

    @property
    def last_block_num_tokens_cached_sparse(self) -> int:
        st = self.sparse_state
        if st is not None and (st.should_compute_cache or st.should_reuse_cache):
            return ((self.current_sparse_token - 1) % self.block_size) + 1
        raise NotImplementedError

    # ---- rows fed to the model this step ----------------------------------
    def step_rows(self) -> tuple[int, int]:
        """(first position, row count) the runner feeds for this sequence."""
        st = self.sparse_state
        if st is None or st.is_full_attention or st.should_compute_cache:
            return 0, self.num_tokens
        if st.should_reuse_cache:
            return st.block_span(self.num_prompt_tokens, self.num_tokens)
        raise ValueError(f"unrecognized sparse cache_state {st.cache_state}")

    def advance(self) -> None:
        """Scheduler.postprocess bookkeeping (scheduler.py:117-120)."""
        self.current_step += 1
        if self.sparse_state is not None:
            self.sparse_state.advance_step()


def slot_mapping_for(seq: Sequence, block_size: int = 256) -> list[int]:
    """Cache slots of the retained rows: whole pages of the block table, the
    last one filled to last_block_num_tokens_cached_sparse."""
    slots: list[int] = []
    n = seq.num_should_cached_blocks
    for j in range(n):
        start = seq.block_table[j] * block_size
        end = start + (block_size if j != n - 1 else seq.last_block_num_tokens_cached_sparse)
        slots.extend(range(start, end))
    return slots


class PageAllocator:
    """Free list of cache pages; pages are handed out in list order."""

    def __init__(self, page_ids: Iterable[int]):
        self.free = deque(page_ids)

    def allocate(self, seq: Sequence) -> None:
        if len(self.free) < seq.num_blocks:
            raise RuntimeError(f"out of KV pages: need {seq.num_blocks}, have {len(self.free)}")
        for _ in range(seq.num_blocks):
            seq.block_table.append(self.free.popleft())

    def release(self, seq: Sequence) -> None:
        for p in reversed(seq.block_table):
            self.free.appendleft(p)
        seq.block_table.clear()


def prepare_step(seqs: list[Sequence], device, block_size: int = 256, build_inputs: bool = True):
    """Install the Context of one forward and (optionally) build its
    (input_ids, positions) from the sequences' host token lists.

    Rows of a sequence are all its tokens for cache states 0/1 and only the
    current block for state 2; slot lists are given for states 1/2.
    """
    dev = torch.device(device)
    pinned = dev.type == "cuda"

    def upload(t: torch.Tensor) -> torch.Tensor:
        # asynchronous copies from pinned memory: building a step never waits for the GPU
        return t.pin_memory().to(dev, non_blocking=True) if pinned else t.to(dev)

    ids, pos, lens, slot_mapping = [], [], [], []
    for seq in seqs:
        st = seq.sparse_state
        start, n = seq.step_rows()
        if build_inputs:
            ids.extend(seq.token_ids[start:start + n])
            pos.extend(range(start, start + n))
        lens.append(n)
        if st is None or st.is_full_attention:
            slot_mapping.append([])
        else:
            slot_mapping.append(upload(torch.tensor(slot_mapping_for(seq, block_size), dtype=torch.int32)))
    cu = torch.zeros(len(seqs) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(lens, dtype=torch.int32), 0)
    cu = upload(cu)
    set_context(True, cu_seqlens_q=None, cu_seqlens_k=cu, max_seqlen_q=0,
                max_seqlen_k=int(sum(lens)), slot_mapping=slot_mapping, is_diffusion=True, seqs=seqs)
    if not build_inputs:
        return None
    return (torch.tensor(ids, dtype=torch.int64, device=device),
            torch.tensor(pos, dtype=torch.int64, device=device))
