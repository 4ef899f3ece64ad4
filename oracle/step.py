"""CPU restatement of the per-step inputs the reference feeds its attention
layer for a batch of diffusion sequences: each sequence's sparse state and how
it advances, the rows it feeds (and their positions), cu_seqlens_k, and the
KV-cache slot list of a sparse sequence.

Test infrastructure: only tests/ import this module (to check the host planner
and the device-side step builder); the product path never does.

Follows:
- dllmserve/sparse/state.py:30-40 (initial state), 42-58 (block boundaries),
  75-104 (advance_step), 123-144 (block / unused indices);
- dllmserve/engine/sequence.py:87-96 (cached pages), 119-132 (n_keep),
  146-152 (tokens cached in the last page);
- dllmserve/engine/model_runner.py:240-302 (rows, positions, cu_seqlens_k,
  slot lists per mode).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

PAGE = 256  # model_runner's block_size: slots per KV-cache page


@dataclass(frozen=True)
class Cfg:
    """The SparseConfig fields the step inputs depend on."""
    block_len: int
    ratio: float
    delay: int


class SparseSeq:
    """One sequence of the batch: prompt length, total length (prompt +
    generation), its KV pages and its sparse config (None: dense)."""

    def __init__(self, prompt: int, total: int, pages=(), cfg: Cfg | None = None):
        self.prompt, self.total = int(prompt), int(total)
        self.pages = list(pages)
        self.cfg = cfg
        self.blk = 0      # current_block_idx
        self.step = 0     # step_in_block
        self.state = 0    # cache_state: 0 full, 1 compute + cache, 2 reuse

    def span(self) -> tuple[int, int]:
        """(block start, block length) of the current block (state.py:42-58);
        the length is negative past the end of the sequence."""
        if self.total - self.prompt <= 0:
            return self.prompt, 0
        bs = self.prompt + self.blk * self.cfg.block_len
        return bs, min(self.cfg.block_len, self.total - bs)

    def advance(self) -> None:
        """state.py:75-104."""
        self.step += 1
        if self.step % self.cfg.block_len == 0:
            self.step = 0
            self.blk += 1
        d = self.cfg.delay
        if d == 1:
            self.state = 0 if self.step == 0 else (1 if self.step == 1 else 2)
        elif d == 0:
            self.state = 1 if self.step == 0 else 2
        else:
            self.state = 0 if self.step < d else (1 if self.step == d else 2)

    def unused(self) -> int:
        """Length of the non-block indices [0, bs) ++ [bs + bl, total) (state.py:130-144)."""
        bs, bl = self.span()
        return len(range(0, bs)) + len(range(bs + bl, self.total))

    def n_keep(self) -> int:
        """sequence.py:119-132."""
        u = self.unused()
        return min(max(1, int(u * self.cfg.ratio)), u)

    def slot_list(self) -> list[int]:
        """Slots of the n_keep cached rows: whole pages, then the last page's
        first ((n_keep - 1) % 256) + 1 slots (model_runner.py:257-270, 280-290;
        sequence.py:87-96, 146-152)."""
        nk = self.n_keep()
        n_pages = (nk + PAGE - 1) // PAGE
        last = (nk - 1) % PAGE + 1
        out: list[int] = []
        for j in range(n_pages):
            start = self.pages[j] * PAGE
            out.extend(range(start, start + (PAGE if j != n_pages - 1 else last)))
        return out


def step_inputs(seqs):
    """Per sequence (mode, positions, slot list or None), and cu_seqlens_k
    (model_runner.py:240-302): a dense sequence, or one in state 0 or 1, feeds
    all its rows (state 1 also carries its slot list); a state-2 sequence
    feeds its current block only, with its slot list."""
    per, lengths = [], []
    for s in seqs:
        mode = 0 if s.cfg is None else s.state
        if mode == 1 and s.span()[1] <= 0:
            # the reference would average an empty block (NaN scores) and keep
            # arbitrary rows; the product refuses such a step, and so does this
            raise ValueError("state 1 with an empty block")
        if mode in (0, 1):
            pos = np.arange(s.total, dtype=np.int64)
            slots = None if mode == 0 else s.slot_list()
        else:
            bs, bl = s.span()
            if bl < 0:  # torch.arange(bs, bs + bl) raises in the reference
                raise ValueError("block past the end of the sequence")
            pos = np.arange(bs, bs + bl, dtype=np.int64)
            slots = s.slot_list()
        per.append((mode, pos, slots))
        lengths.append(len(pos))
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    return per, cu
