"""Drop-in ``Attention`` layer and KV-cache helpers on the gfx950 kernels.

Interface of dllmserve/layers/attention.py (``Attention(num_heads,
head_dim, scale, num_kv_heads, causal)``, ``.forward(q, k, v)``,
``store_kvcache``, ``load_kvcache``, the ``k_cache`` / ``v_cache`` /
``layer_id`` attributes a model runner binds).  The diffusion branch
(attention.py:150-306) is reproduced per sequence:

* cache state 0 or no SparseConfig: full bidirectional attention over the
  sequence's rows (K3a);
* state 1: full attention (K3a), and the top-n_keep non-block rows of every
  KV head (``head_select``) or of all heads are written to the sequence's
  cache slots (K5/K6 fused with K1);
* state 2: the block rows attend to [cached rows ; block rows] (K3b), read
  straight from the paged cache by slot, without the reference's gather and
  concatenation copies.

Per step the layer builds one launch plan from ``context.seqs`` (host
integers only, no device synchronisation) and caches it on the Context, so
the 32 layers of a forward reuse it.  Every kernel runs on the caller's
current HIP stream; nothing falls back to the CPU.
"""
from __future__ import annotations

import os
import weakref

import numpy as np
import torch
from torch import nn

from .. import _capi
from ..sparse.state import keep_count
from ..utils.context import get_context


def _token_rows(t: torch.Tensor, heads: int, head_dim: int, name: str):
    """(t, rows, token stride in elements) of q/k/v given as [rows, heads *
    head_dim] or [rows, heads, head_dim] with contiguous heads; any other
    shape goes through the reference's ``view(-1, heads, head_dim)``."""
    sh = t.shape
    if len(sh) == 2 and sh[1] == heads * head_dim:
        st = t.stride()
        if st[1] != 1:
            raise ValueError(f"{name} must have contiguous heads; got shape {tuple(sh)} strides {st}")
        return t, sh[0], st[0]
    if len(sh) != 3 or sh[1] != heads or sh[2] != head_dim:
        t = t.view(-1, heads, head_dim)
        sh = t.shape
    st = t.stride()
    if st[2] != 1 or st[1] != head_dim:
        raise ValueError(f"{name} must be [rows, heads, head_dim] with contiguous heads; got shape "
                         f"{tuple(sh)} strides {st}")
    return t, sh[0], st[0]


def _slot_tensor(slot_mapping, device) -> torch.Tensor:
    if not isinstance(slot_mapping, torch.Tensor):
        slot_mapping = torch.tensor(list(slot_mapping), dtype=torch.int32)
    if slot_mapping.dtype != torch.int32 or slot_mapping.device != device or not slot_mapping.is_contiguous():
        slot_mapping = slot_mapping.to(device=device, dtype=torch.int32).contiguous()
    return slot_mapping


def store_kvcache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                  slot_mapping: torch.Tensor) -> None:
    """k_cache.flat[slot_mapping[i], :] = key[i], same for value (attention.py:33-50)."""
    N, num_heads, head_dim = key.shape
    D = num_heads * head_dim
    assert key.stride(-1) == 1 and value.stride(-1) == 1
    assert key.stride(1) == head_dim and value.stride(1) == head_dim
    assert k_cache.stride(1) == D and v_cache.stride(1) == D
    if slot_mapping.numel() != N:
        print(f"Warning: slot_mapping.numel {slot_mapping.numel()} != N {N}")
    assert slot_mapping.numel() == N
    assert k_cache.is_contiguous() and v_cache.is_contiguous(), "KV cache must be contiguous"
    assert key.dtype == value.dtype == k_cache.dtype == v_cache.dtype == torch.bfloat16, "bf16 tensors expected"
    slot = _slot_tensor(slot_mapping, key.device)
    _capi.store_kvcache(key, value, k_cache, v_cache, slot, N, D)


def load_kvcache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                 slot_mapping: torch.Tensor) -> None:
    """key[i] = k_cache.flat[slot_mapping[i], :], same for value (attention.py:77-92)."""
    N, num_heads, head_dim = key.shape
    D = num_heads * head_dim
    assert key.stride(-1) == 1 and value.stride(-1) == 1
    assert key.stride(1) == head_dim and value.stride(1) == head_dim
    assert k_cache.stride(1) == D and v_cache.stride(1) == D
    assert slot_mapping.numel() == N
    assert k_cache.is_contiguous() and v_cache.is_contiguous(), "KV cache must be contiguous"
    assert key.dtype == value.dtype == k_cache.dtype == v_cache.dtype == torch.bfloat16, "bf16 tensors expected"
    slot = _slot_tensor(slot_mapping, key.device)
    _capi.load_kvcache(key, value, k_cache, v_cache, slot, N, D)


class StepLayout:
    """Host integers of one diffusion step: per-sequence mode (0 full, 1 full
    + select-and-store, 2 block vs cache, -1 unrecognised), fed rows, block
    span and n_keep, and the launch sizes derived from them (attention.py:
    168-265, sequence.py:99-152).  No tensors are created."""

    def __init__(self, seqs):
        if not seqs:
            raise ValueError("diffusion context has no sequences")
        rows, modes, spans, keeps, cfgs = [], [], [], [], []
        for seq in seqs:
            cfg = seq.sparse_state.config if seq.sparse_state is not None else None
            cfgs.append((bool(cfg.head_select), int(cfg.pool_kernel)) if cfg is not None else (False, 1))
            st = seq.sparse_state
            N = seq.num_tokens
            if st is None or st.is_full_attention:
                modes.append(0)
                rows.append(N)
                spans.append((0, 0))
                keeps.append(0)
            elif st.should_compute_cache:
                bs, bl = st.block_span(seq.num_prompt_tokens, N)
                bl = max(0, min(bl, N - bs)) if bs < N else 0
                if bl == 0:
                    raise ValueError(f"sequence {seq.seq_id}: cache state 1 with an empty block "
                                     f"(block start {bs}, {N} tokens)")
                modes.append(1)
                rows.append(N)
                spans.append((bs, bl))
                keeps.append(keep_count(N - bl, st.retention_ratio))
            elif st.should_reuse_cache:
                bs, bl_raw = st.compute_block_boundaries(seq.num_prompt_tokens, N)
                if bl_raw < 0:  # the reference's torch.arange(bs, bs + bl) raises here too
                    raise RuntimeError(f"sequence {seq.seq_id}: block {st.current_block_idx} starts at {bs}, "
                                       f"past the {N} tokens of the sequence")
                bl = bl_raw
                modes.append(2)
                rows.append(bl)
                spans.append((bs, bl))
                keeps.append(seq.current_sparse_token)
            else:
                modes.append(-1)  # unrecognised state: rows stay zero (outputs = zeros_like(q))
                rows.append(N)
                spans.append((0, 0))
                keeps.append(0)
        self.modes, self.rows, self.spans, self.keeps = modes, rows, spans, keeps
        self.cfgs = cfgs  # (head_select, pool_kernel) per sequence; selection jobs carry their own
        self.n_seq = len(seqs)
        self.total_rows = int(sum(rows))
        self.cu = np.zeros(self.n_seq + 1, dtype=np.int64)
        self.cu[1:] = np.cumsum(rows)
        self.any_skipped = any(m == -1 for m in modes)
        # longest first (ties by index): with the XCD interleave of the dense
        # kernel, long segments then start early and short ones fill the tail
        # (16 ragged Dream GQA segments: 3-12 % faster than batch order)
        self.dense = sorted((i for i, m in enumerate(modes) if m in (0, 1)), key=lambda i: (-rows[i], i))
        self.jobs_idx = [i for i, m in enumerate(modes) if m == 1]
        self.cached = [i for i, m in enumerate(modes) if m == 2]
        self.n_dense = len(self.dense)
        self.max_q_dense = max((rows[i] for i in self.dense), default=0)
        self.n_job = len(self.jobs_idx)
        self.max_kc = max((rows[i] - spans[i][1] for i in self.jobs_idx), default=0)
        self.max_keep = max((keeps[i] for i in self.jobs_idx), default=0)
        self.max_blk = max((spans[i][1] for i in self.jobs_idx), default=0)
        self.n_cached = len(self.cached)
        self.max_q_cached = max((rows[i] for i in self.cached), default=0)
        self.max_keys_cached = max((rows[i] + keeps[i] for i in self.cached), default=0)
        self.total_slots = sum(keeps[i] for i in self.cached + self.jobs_idx)
        # a launch over every sequence in batch order gets no id table: the
        # kernels then read a segment's offsets one dependent load earlier
        self.dense_identity = self.dense == list(range(self.n_seq))
        self.cached_identity = self.cached == list(range(self.n_seq))

    def signature(self) -> tuple:
        """Everything a captured step's launches depend on."""
        return (tuple(self.modes), tuple(self.rows), tuple(self.keeps), tuple(s[1] for s in self.spans),
                tuple(self.cfgs[i] for i in self.jobs_idx))


class StepPlan:
    """Launch tables of one diffusion forward (shared by all layers).

    ``StepPlan(context, device, ...)`` builds them from host integers of
    ``context.seqs`` and uploads them with one asynchronous copy;
    ``StepPlan.from_device`` wraps tables the device-side builder wrote."""

    _SCALARS = ("n_seq", "total_rows", "any_skipped", "n_dense", "max_q_dense", "n_job", "max_kc", "max_keep",
                "max_blk", "n_cached", "max_q_cached", "max_keys_cached", "dense_identity", "cached_identity")

    def __init__(self, context, device: torch.device, num_kv_heads: int = 0, head_dim: int = 0, num_heads: int = 0,
                 layout: StepLayout | None = None):
        seqs = context.seqs
        lay = layout if layout is not None else StepLayout(seqs)
        self._take(lay, device)
        rows, spans, keeps, cu = lay.rows, lay.spans, lay.keeps, lay.cu
        dense, jobs_idx, cached = lay.dense, lay.jobs_idx, lay.cached

        # slots of sparse sequences: state-2 sequences first (contiguous, so
        # slot_off below brackets each of them), then state-1 sequences
        slot_mapping = context.slot_mapping if context.slot_mapping is not None else []
        slot_parts, slot_base = [], {}
        off = 0
        for i in cached + jobs_idx:
            if i >= len(slot_mapping):
                raise ValueError(f"context.slot_mapping has no entry for sequence index {i}")
            sm = slot_mapping[i]
            n = sm.numel() if isinstance(sm, torch.Tensor) else len(sm)
            if n != keeps[i]:
                print(f"Warning: slot_mapping.numel {n} != N {keeps[i]}")
            assert n == keeps[i]
            slot_base[i] = off
            off += n
            slot_parts.append(_slot_tensor(sm, device))
        self.slots = torch.cat(slot_parts) if slot_parts else torch.zeros(1, dtype=torch.int32, device=device)

        # selection jobs: row0, n_tok, blk_start, blk_len, n_keep, slot_off, head_select, pool_k
        jobs = np.zeros((max(1, self.n_job), _capi.JOB_COLS), dtype=np.int64)
        for r, i in enumerate(jobs_idx):
            bs, bl = spans[i]
            hs, pk = lay.cfgs[i]
            jobs[r] = (cu[i], rows[i], bs, bl, keeps[i], slot_base[i], int(hs), pk)

        # cached (state 2) segments: slot offsets indexed by position in `cached`
        slot_off = np.zeros(self.n_cached + 1, dtype=np.int64)
        for r, i in enumerate(cached):
            slot_off[r] = slot_base[i]
            slot_off[r + 1] = slot_base[i] + keeps[i]

        # one asynchronous host->device copy (from pinned memory) of every int32 table
        parts = [cu, np.array(dense or [0]), np.array(cached or [0]), slot_off, jobs.reshape(-1)]
        flat = np.concatenate([p.astype(np.int64) for p in parts])
        if flat.size and (flat.max() >= 2**31 or flat.min() < -(2**31)):
            raise ValueError("step tables exceed int32")
        host = torch.from_numpy(flat.astype(np.int32))
        if device.type == "cuda":
            host = host.pin_memory()
        dev = host.to(device, non_blocking=True)
        o = 0
        self.cu = dev[o:o + cu.size]; o += cu.size
        self.dense_ids = dev[o:o + max(1, len(dense))]; o += max(1, len(dense))
        self.cached_ids = dev[o:o + max(1, len(cached))]; o += max(1, len(cached))
        self.slot_off = dev[o:o + slot_off.size]; o += slot_off.size
        self.jobs = dev[o:o + jobs.size]

    def _take(self, lay: StepLayout, device) -> None:
        self.device = device
        for k in self._SCALARS:
            setattr(self, k, getattr(lay, k))
        self._ws = {}
        self._args = {}
        self.last_idx = None

    @classmethod
    def from_device(cls, lay: StepLayout, device, cu, dense_ids, cached_ids, slot_off, jobs, slots) -> "StepPlan":
        """Plan over tables already on the device (written by dllm_step_build)."""
        self = cls.__new__(cls)
        self._take(lay, device)
        self.cu, self.dense_ids, self.cached_ids = cu, dense_ids, cached_ids
        self.slot_off, self.jobs, self.slots = slot_off, jobs, slots
        return self

    def workspace(self, key, nbytes: int) -> torch.Tensor | None:
        """A device buffer of at least ``nbytes`` kept under ``key`` for the
        step.  A larger request under the same key replaces (and frees) the
        earlier buffer, so a caller that keeps an address must key by
        everything the size depends on."""
        if nbytes <= 0:
            return None
        t = self._ws.get(key)
        if t is None or t.numel() < nbytes:
            t = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
            self._ws[key] = t
        return t

    def launch_args(self, Hq: int, Hkv: int, D: int) -> dict:
        """Device addresses of the step's tables and the K3b workspace for
        one head shape, computed once per step for all layers.  The workspace
        is keyed by the head shape and held in the returned dict, so the
        address cached here stays valid while the plan lives, whatever other
        head shapes later ask for."""
        key = (Hq, Hkv, D)
        a = self._args.get(key)
        if a is None:
            ws = self.workspace(("cached",) + key, _capi.block_cached_workspace_size(
                self.n_cached, self.max_q_cached, self.max_keys_cached, Hq, Hkv, D)) if self.n_cached else None
            a = dict(cu=self.cu.data_ptr(), slots=self.slots.data_ptr(), slot_off=self.slot_off.data_ptr(),
                     dense_ids=None if self.dense_identity else self.dense_ids.data_ptr(),
                     cached_ids=None if self.cached_identity else self.cached_ids.data_ptr(),
                     ws=None if ws is None else ws.data_ptr(), ws_bytes=0 if ws is None else ws.numel(),
                     ws_tensor=ws)
            self._args[key] = a
        return a


class Attention(nn.Module):
    """Drop-in for dllmserve.layers.attention.Attention (attention.py:95-119)."""

    keep_indices = os.environ.get("DLLM_KEEP_SELECT_INDICES", "0") == "1"

    def __init__(self, num_heads, head_dim, scale, num_kv_heads, causal=True):
        super().__init__()
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.scale = scale
        self.num_kv_heads = num_kv_heads
        self.causal = causal
        self.k_cache = self.v_cache = torch.tensor([])
        self.layer_id = None
        self.last_select_indices = None
        # (weak references, addresses, sizes, device, result) of the last bound
        # cache that passed _check_cache: weak, so that a cache the runner
        # drops or re-sizes is freed at once, not kept alive by this check
        self._cache_ok = None

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        # q/k/v as [rows, heads * head_dim] or [rows, heads, head_dim] are used
        # without the reference's view (attention.py:108-110); other shapes
        # take that view
        context = get_context()
        if context.is_diffusion:
            return self._mixed_sparse_dense_attention(q, k, v, context)
        raise NotImplementedError(
            "only the diffusion branch (context.is_diffusion=True) is provided; the autoregressive "
            "prefill/decode branch of the reference is unused by diffusion models")

    def _plan(self, context, device) -> StepPlan:
        plan = getattr(context, "_dllm_plan", None)
        if plan is None or plan.device != device:
            plan = StepPlan(context, device, self.num_kv_heads, self.head_dim, self.num_heads)
            context._dllm_plan = plan
        return plan

    def _check_cache(self, device) -> tuple:
        """Check the bound cache and return (k address, v address, slots).
        The kernels address it as flat bf16 rows of Hkv * head_dim elements on
        q's device (the checks store_kvcache makes, attention.py:42-47); a
        cache that passed keeps passing while the same tensors keep their
        addresses and sizes."""
        kc, vc = self.k_cache, self.v_cache
        key = (kc.data_ptr(), vc.data_ptr(), kc.numel(), vc.numel(), device)
        ok = self._cache_ok
        if ok is not None and ok[0]() is kc and ok[1]() is vc and ok[2:7] == key:
            return ok[7]
        for t, n in ((kc, "k_cache"), (vc, "v_cache")):
            if (t.dtype != torch.bfloat16 or not t.is_contiguous() or t.device != device or t.dim() < 2
                    or tuple(t.shape[-2:]) != (self.num_kv_heads, self.head_dim)):
                raise ValueError(f"{n} must be a contiguous bf16 tensor [..., {self.num_kv_heads}, {self.head_dim}] "
                                 f"on {device}; got {t.dtype} {tuple(t.shape)} on {t.device}")
        res = (kc.data_ptr(), vc.data_ptr(), min(kc.numel(), vc.numel()) // (self.num_kv_heads * self.head_dim))
        self._cache_ok = (weakref.ref(kc), weakref.ref(vc)) + key + (res,)
        return res

    def _mixed_sparse_dense_attention(self, q, k, v, context):
        Hq, Hkv, D = self.num_heads, self.num_kv_heads, self.head_dim
        q, nq, q_st = _token_rows(q, Hq, D, "q")
        k, nk, k_st = _token_rows(k, Hkv, D, "k")
        v, nv, v_st = _token_rows(v, Hkv, D, "v")
        if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
            raise TypeError(f"bf16 q/k/v expected, got {q.dtype}/{k.dtype}/{v.dtype}")
        if not (q.is_cuda and k.is_cuda and v.is_cuda):
            raise RuntimeError("Attention runs on the GPU only (no CPU fallback)")
        if not (k.get_device() == v.get_device() == q.get_device()):
            raise ValueError(f"q/k/v are on different devices: {q.device}/{k.device}/{v.device}")
        dev = q.device
        plan = self._plan(context, dev)
        if nq != plan.total_rows or nk != plan.total_rows or nv != plan.total_rows:
            raise ValueError(f"q/k/v have {nq}/{nk}/{nv} rows, the step's sequences feed {plan.total_rows}")
        o = torch.zeros_like(q) if plan.any_skipped else torch.empty_like(q)
        o_st = o.stride(0)
        args = plan.launch_args(Hq, Hkv, D)
        stream = _capi._stream(dev)
        qp, kp, vp, op = q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr()

        if plan.n_dense:
            _capi.attn_varlen_fwd_raw(qp, kp, vp, op, args["cu"], args["dense_ids"], plan.n_dense, plan.max_q_dense,
                                      Hq, Hkv, D, q_st, k_st, v_st, o_st, float(self.scale), stream)

        if plan.n_job:
            if not (self.k_cache.numel() and self.v_cache.numel()):
                raise RuntimeError("cache state 1 needs k_cache/v_cache bound to this layer")
            self._check_cache(dev)
            ws = plan.workspace("select", _capi.select_workspace_size(plan.n_job, plan.max_kc, Hq, Hkv, D))
            idx = None
            if self.keep_indices:
                idx = torch.full((plan.n_job, Hkv, plan.max_keep), -1, dtype=torch.int64, device=dev)
            q3 = q if q.dim() == 3 else q.view(-1, Hq, D)
            k3 = k if k.dim() == 3 else k.view(-1, Hkv, D)
            v3 = v if v.dim() == 3 else v.view(-1, Hkv, D)
            _capi.select_kv_store(q3, k3, v3, plan.jobs, plan.n_job, plan.max_kc, plan.max_keep, np.float32(D ** 0.5),
                                  self.k_cache, self.v_cache, plan.slots, idx, ws)
            self.last_select_indices = idx

        if plan.n_cached:
            if not (self.k_cache.numel() and self.v_cache.numel()):
                raise RuntimeError("cache state 2 needs k_cache/v_cache bound to this layer")
            kc, vc, cache_slots = self._check_cache(dev)
            _capi.attn_block_cached_fwd_raw(qp, kp, vp, op, args["cu"], args["cached_ids"], plan.n_cached,
                                            plan.max_q_cached, plan.max_keys_cached, kc, vc, cache_slots,
                                            args["slots"], args["slot_off"], Hq, Hkv, D, q_st, k_st, v_st, o_st,
                                            float(self.scale), args["ws"], args["ws_bytes"], stream)
        return o if o.dim() == 2 else o.view(-1, Hq * D)
