"""Low-confidence remasking step of the diffusion runner on the gfx950 K8 / K9
kernels: the drop-in for ModelRunner._reconstruct_and_sample_optimized_v2
(dllmserve/engine/model_runner.py:756-949, temperature 0).

Per sequence, the reference picks the hidden rows whose tokens may be
unmasked this step (all generated positions without a SparseConfig, the
current block otherwise; :791-818), projects them to logits, takes
``x0_p, x0 = max(softmax(logits))`` (:862-887) and unmasks
``min(ceil(nmask / steps_remain), nmask)`` masked positions of the window in
order of confidence, the block's first position first in the full-attention
state (:895-949).  Here the windows are derived on the host from the
sequences' own state (no device reads), the rows are gathered with one
``index_select``, the LM head stays a library GEMM (``compute_logits``), and
K8 (softmax-max, one read of the logits) and K9 (count, top-k and write-back
for all sequences in one launch) finish the step on the device.  Tokens live
in a device int64 tensor; nothing synchronises with the host.  There is no
CPU path.
"""
from __future__ import annotations

from typing import Callable, Optional, Sequence as Seq

import torch

from .. import _capi

MAX_WINDOW = 8192  # SamplingParams caps gen_length at 8192 (sampling_params.py:18-22)


def _total_steps(seq) -> int:
    sp = getattr(seq, "sampling_params", None)
    return sp.steps if sp is not None else seq.steps


def step_windows(seqs) -> list[tuple[int, int, int, int, int]]:
    """(hidden row of the window's first position, window start position,
    window length, steps_remain, first-token rule) per sequence, for the rows
    the runner fed this step, packed in sequence order: only the current
    block in the reuse-cache state, every position otherwise
    (model_runner.py:240-256).  Reads only what the reference's Sequence and
    PerRequestSparseState expose (num_prompt_tokens, num_tokens,
    current_step, sampling_params.steps, compute_block_boundaries,
    step_in_block, the state properties)."""
    out, row0 = [], 0
    for seq in seqs:
        st = seq.sparse_state
        P, N = seq.num_prompt_tokens, seq.num_tokens
        if st is None:                                    # :797-802, :911-912
            start, n_fed = 0, N
            lo, hi = P, N
            steps_remain = _total_steps(seq) - seq.current_step
            first = 0
        else:                                             # :803-818, :913-915
            lo, n = st.compute_block_boundaries(P, N)
            n = max(0, n)
            hi = lo + n
            start, n_fed = (lo, n) if st.should_reuse_cache else (0, N)
            steps_remain = n - st.step_in_block
            first = int(st.is_full_attention and n > 0)   # :920
        if steps_remain == 0:
            # the reference computes ceil(float(nmask) / steps_remain) (:916)
            raise ZeroDivisionError(f"sequence {seq.seq_id}: no denoising steps remain for its window")
        if not (start <= lo <= hi <= start + n_fed):
            raise ValueError(f"sequence {seq.seq_id}: window [{lo}, {hi}) is not among the fed rows")
        out.append((row0 + lo - start, lo, hi - lo, steps_remain, first))
        row0 += n_fed
    return out


class RemaskSampler:
    """Holds the step's small buffers; call once per denoising step.

    compute_logits(hidden_rows [m, H] bf16) -> logits [m, V] bf16 (the LM
    head, e.g. ``lambda h: h @ lm_head.t()``).  tokens is the device int64
    token store: [B, N_max] (row b = sequence b) or flat with
    ``token_offsets[b]`` giving sequence b's first token."""

    def __init__(self, compute_logits: Callable[[torch.Tensor], torch.Tensor], mask_token_id: int,
                 max_logprobs: Optional[int] = None, seed: int = 0):
        self.compute_logits = compute_logits
        self.mask_token_id = int(mask_token_id)
        self.max_logprobs = max_logprobs  # rows per LM-head chunk (None: all at once)
        self.seed = int(seed)             # base of the per-call noise seeds (temperature > 0)
        self.calls = 0
        self._ws = None

    def _workspace(self, M: int, V: int, device) -> Optional[torch.Tensor]:
        need = _capi.softmax_max_workspace_size(M, V)
        if need == 0:
            return None
        if self._ws is None or self._ws.numel() < need or self._ws.device != device:
            self._ws = torch.empty(max(need, 16), dtype=torch.uint8, device=device)
        return self._ws

    def logits_max(self, rows: torch.Tensor, row_temperature: Optional[torch.Tensor] = None, seed: int = 0):
        """x0 (int64) and x0_p (bf16) of the gathered hidden rows; rows whose
        row_temperature (float64, device) is > 0 are sampled with Gumbel noise
        drawn from (seed, row index)."""
        M = rows.shape[0]
        dev = rows.device
        x0 = torch.empty(M, dtype=torch.int64, device=dev)
        x0_p = torch.empty(M, dtype=torch.bfloat16, device=dev)
        step = M if not self.max_logprobs else self.max_logprobs
        for a in range(0, M, max(step, 1)):
            b = min(M, a + step)
            logits = self.compute_logits(rows[a:b])
            if logits.dtype != torch.bfloat16 or logits.dim() != 2 or logits.stride(-1) != 1:
                raise ValueError("compute_logits must return [rows, vocab] bf16 with a contiguous last dim")
            ws = self._workspace(b - a, logits.shape[1], dev)
            if row_temperature is None:
                _capi.softmax_max(logits, x0[a:b], x0_p[a:b], ws)
            else:
                _capi.softmax_max_sample(logits, row_temperature[a:b], seed, a, x0[a:b], x0_p[a:b], ws)
        return x0, x0_p

    def __call__(self, hidden_states: torch.Tensor, seqs: Seq, tokens: torch.Tensor,
                 token_offsets: Optional[Seq[int]] = None, remasking: str = "low_confidence",
                 temperature: float = 0.0, generator: Optional[torch.Generator] = None) -> torch.Tensor:
        """Unmask this step's tokens in place; returns the per-sequence count
        of unmasked positions (int32 [B], on the device).

        Temperatures come from each sequence's ``sampling_params`` when it
        has them, else from ``temperature`` (one value or one per sequence).
        Rows of a sequence with temperature > 0 get the reference's Gumbel
        noise (add_gumbel_noise, model_runner.py:592-600) with draws from a
        counter-based generator seeded by (seed, call number).  Every such
        sequence gets its noise; the reference's v2 path applies it only to
        the first sequence of each logits chunk (its cu_seqlens there is the
        cumsum of one length, model_runner.py:826-836,859-866)."""
        if remasking not in ("low_confidence", "random"):
            raise NotImplementedError(remasking)               # :908-909
        _capi._require_gpu(hidden_states, tokens)
        if tokens.dtype != torch.int64 or not tokens.is_contiguous():
            raise ValueError("tokens must be a contiguous int64 device tensor")
        dev = hidden_states.device
        win = step_windows(seqs)
        if tokens.dim() == 2:
            if tokens.shape[0] != len(seqs):
                raise ValueError("tokens [B, N] must have one row per sequence")
            offs = [b * tokens.stride(0) for b in range(len(seqs))]
        else:
            if token_offsets is None or len(token_offsets) != len(seqs):
                raise ValueError("a flat token store needs token_offsets, one per sequence")
            offs = [int(o) for o in token_offsets]
        temps = []
        for b, seq in enumerate(seqs):
            sp = getattr(seq, "sampling_params", None)
            if sp is not None:
                temps.append(float(sp.temperature))
            elif isinstance(temperature, (list, tuple)):
                temps.append(float(temperature[b]))
            else:
                temps.append(float(temperature))
        params, idx, row_t, r = [], [], [], 0
        for b, (h0, lo, n, sr, first) in enumerate(win):
            if n > MAX_WINDOW:
                raise ValueError(f"window of {n} positions exceeds {MAX_WINDOW}")
            params.append((offs[b] + lo, n, r, sr, first))
            idx.append(torch.arange(h0, h0 + n, dtype=torch.int64))
            row_t.append(torch.full((n,), max(0.0, temps[b]), dtype=torch.float64))
            r += n
        n_unmasked = torch.zeros(len(seqs), dtype=torch.int32, device=dev)
        if r == 0:
            return n_unmasked
        sel = torch.cat(idx).pin_memory().to(dev, non_blocking=True)
        p = torch.tensor(params, dtype=torch.int32).pin_memory().to(dev, non_blocking=True)
        rt = None
        if any(t > 0 for t in temps):
            rt = torch.cat(row_t).pin_memory().to(dev, non_blocking=True)
        seed = (self.seed * 0x9E3779B97F4A7C15 + self.calls) & 0xFFFFFFFFFFFFFFFF
        self.calls += 1
        x0, x0_p = self.logits_max(hidden_states.index_select(0, sel), rt, seed)
        conf = x0_p
        if remasking == "random":                              # :903-905
            conf = torch.rand(r, device=dev, generator=generator).to(torch.bfloat16)
        _capi.lowconf_unmask(tokens.view(-1), p, len(seqs), max(w[2] for w in win), x0, conf,
                             self.mask_token_id, n_unmasked)
        return n_unmasked


def sample_device_windows(sampler: "RemaskSampler", hidden_states: torch.Tensor, tokens: torch.Tensor,
                          smp_rows: torch.Tensor, smp_params: torch.Tensor, max_win: int) -> torch.Tensor:
    """The sampling step with windows built on the device (dllm_step_build's
    smp_rows / smp_params): nothing is computed or copied on the host."""
    n_seq = smp_params.shape[0]
    n_unmasked = torch.zeros(n_seq, dtype=torch.int32, device=hidden_states.device)
    if smp_rows.numel() == 0:
        return n_unmasked
    x0, x0_p = sampler.logits_max(hidden_states.index_select(0, smp_rows))
    _capi.lowconf_unmask(tokens.view(-1), smp_params, n_seq, max_win, x0, x0_p, sampler.mask_token_id, n_unmasked)
    return n_unmasked


def token_lists(tokens: torch.Tensor, seqs, token_offsets: Optional[Seq[int]] = None) -> list[list[int]]:
    """The reference's return value (one token list per sequence); one copy to the host."""
    host = tokens.cpu()
    if host.dim() == 2:
        return [host[b, :s.num_tokens].tolist() for b, s in enumerate(seqs)]
    return [host[o:o + s.num_tokens].tolist() for o, s in zip(token_offsets, seqs)]
