"""Ambient per-forward metadata read by ``Attention.forward``.

Mirrors the interface of dllmserve/utils/context.py:6-68 (same field names,
``get_context`` / ``set_context`` / ``reset_context``), so a model runner
written against the reference fills it unchanged.  Module-global and not
re-entrant, like the reference (context.py:21): one forward at a time per
process.

The diffusion path reads ``seqs``, ``cu_seqlens_k`` and ``slot_mapping`` (a
list with one int32 slot tensor per sequence, empty for dense sequences).
The attention layer caches its per-step launch plan on the Context object in
the private attribute ``_dllm_plan`` so that the host work is done once per
step, not once per layer.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch


@dataclass
class Context:
    is_prefill: bool = False
    cu_seqlens_q: Optional[torch.Tensor] = None
    cu_seqlens_k: Optional[torch.Tensor] = None
    max_seqlen_q: int = 0
    max_seqlen_k: int = 0
    slot_mapping: Optional[object] = None
    extra_slot_mapping: Optional[object] = None
    context_lens: Optional[torch.Tensor] = None
    block_tables: Optional[torch.Tensor] = None
    is_diffusion: bool = False
    seqs: Optional[list] = None


_CONTEXT = Context()


def get_context() -> Context:
    return _CONTEXT


def set_context(
    is_prefill,
    cu_seqlens_q=None,
    cu_seqlens_k=None,
    max_seqlen_q=0,
    max_seqlen_k=0,
    slot_mapping=None,
    extra_slot_mapping=None,
    context_lens=None,
    block_tables=None,
    is_diffusion=False,
    seqs=None,
) -> None:
    """Install a fresh Context (positional order as in context.py:28-40)."""
    global _CONTEXT
    _CONTEXT = Context(
        is_prefill=is_prefill,
        cu_seqlens_q=cu_seqlens_q,
        cu_seqlens_k=cu_seqlens_k,
        max_seqlen_q=max_seqlen_q,
        max_seqlen_k=max_seqlen_k,
        slot_mapping=slot_mapping,
        extra_slot_mapping=extra_slot_mapping,
        context_lens=context_lens,
        block_tables=block_tables,
        is_diffusion=is_diffusion,
        seqs=seqs,
    )


def reset_context() -> None:
    global _CONTEXT
    _CONTEXT = Context()
