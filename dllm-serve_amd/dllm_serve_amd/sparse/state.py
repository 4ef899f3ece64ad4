"""Sparse-attention configuration and the per-request block / cache state
machine.

Interface follows dllmserve/sparse/state.py:6-163 (``SparseConfig`` field
names and defaults, ``PerRequestSparseState`` methods and properties), since
callers construct and inspect these objects directly.  Behaviour kept from
the reference on purpose:

* ``SparseConfig.enabled`` is stored but not consulted by the attention path:
  any non-None config engages the state machine (state.py:64-75 is never
  called by the reference either).
* ``advance_step`` moves to the next block every ``default_block_len`` steps
  and sets ``cache_state`` from ``delay_step`` (state.py:77-104):
    delay_step == 1: step 0 -> 0, step 1 -> 1, later -> 2
    delay_step == 0: step 0 -> 1, later -> 2
    delay_step >= 2: step < d -> 0, step == d -> 1, later -> 2
* The block of a request is [prompt_len + idx*block_len, +min(block_len,
  total - start)) (state.py:44-62); its length can be <= 0 once the block
  index runs past the generation, in which case it holds no rows.

``block_span`` / ``num_unused_tokens`` are host-integer forms used by the
attention layer to plan a step without creating device tensors.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch


@dataclass
class SparseConfig:
    enabled: bool = False
    default_block_len: int = 32
    retention_ratio: float = 0.5
    pool_kernel: int = 3
    delay_step: int = 1
    head_select: bool = False


@dataclass
class SparseContext:
    """Per-request view used by callers that pass sparse metadata explicitly
    (kept for interface parity with state.py:18-29; the path does not read it)."""

    cache_state: int
    block_indices: torch.Tensor
    block_spans: torch.Tensor
    retention_ratio: float
    pool_kernel: int
    seq_sparse_state: Optional["PerRequestSparseState"] = None


class PerRequestSparseState:
    def __init__(self, seq_id: int, config: SparseConfig, device) -> None:
        self.seq_id = seq_id
        self.config = config
        self.device = device
        self.current_block_idx = 0
        self.step_in_block = 0
        self.cache_state = 0

    # ---- block geometry -------------------------------------------------
    def compute_block_boundaries(self, prompt_len: int, total_len: int) -> tuple[int, int]:
        """(block_start, block_length) of the current block; length may be <= 0."""
        if total_len - prompt_len <= 0:
            return prompt_len, 0
        start = prompt_len + self.current_block_idx * self.block_len
        return start, min(self.block_len, total_len - start)

    def block_span(self, prompt_len: int, total_len: int) -> tuple[int, int]:
        """(block_start, number of block rows), the row count clamped at 0."""
        start, length = self.compute_block_boundaries(prompt_len, total_len)
        return start, max(0, length)

    def num_unused_tokens(self, prompt_len: int, total_len: int) -> int:
        """len(get_unuse_block_indices(...)) without building the tensors."""
        start, length = self.compute_block_boundaries(prompt_len, total_len)
        return max(0, start) + max(0, total_len - (start + length))

    def get_cache_state(self) -> int:
        return self.cache_state if self.config.enabled else 0

    def advance_step(self) -> None:
        self.step_in_block += 1
        if self.step_in_block % self.block_len == 0:
            self.step_in_block = 0
            self.current_block_idx += 1
        d = self.config.delay_step
        s = self.step_in_block
        if d == 1:
            self.cache_state = 0 if s == 0 else (1 if s == 1 else 2)
        elif d == 0:
            self.cache_state = 1 if s == 0 else 2
        else:
            self.cache_state = 0 if s < d else (1 if s == d else 2)

    def get_block_indices(self, prompt_len: int, total_len: int) -> torch.Tensor:
        start, length = self.compute_block_boundaries(prompt_len, total_len)
        self.block_indices = torch.arange(start, start + length, dtype=torch.int64, device=self.device)
        return self.block_indices

    def get_unuse_block_indices(self, prompt_len: int, total_len: int) -> torch.Tensor:
        start, length = self.compute_block_boundaries(prompt_len, total_len)
        self.block_indices_prefix = torch.arange(0, start, dtype=torch.int64, device=self.device)
        self.block_indices_suffix = torch.arange(start + length, total_len, dtype=torch.int64, device=self.device)
        self.block_indices = torch.cat([self.block_indices_prefix, self.block_indices_suffix], dim=0)
        return self.block_indices

    # ---- config views and state predicates --------------------------------
    @property
    def pool_kernel(self) -> int:
        return self.config.pool_kernel

    @property
    def retention_ratio(self) -> float:
        return self.config.retention_ratio

    @property
    def block_len(self) -> int:
        return self.config.default_block_len

    @property
    def should_compute_cache(self) -> bool:
        return self.cache_state == 1

    @property
    def should_reuse_cache(self) -> bool:
        return self.cache_state == 2

    @property
    def is_full_attention(self) -> bool:
        return self.cache_state == 0


def keep_count(num_candidates: int, ratio: float) -> int:
    """Rows kept per selection head: min(max(1, int(Kc * ratio)), Kc)
    (attention.py:338-339, 399; sequence.py:119-122)."""
    return min(max(1, int(num_candidates * ratio)), num_candidates)
