"""ctypes binding of ``libdllm_attn.so`` (the gfx950 kernels behind the C ABI
declared in ``include/dllm_attn.h``).

The library is built in-tree by ``dllm-serve_amd/csrc/Makefile``.  ``torch``
is imported before the library is loaded so that the library binds to the
HIP runtime torch already loaded (both carry the soname libamdhip64.so.7):
device pointers and streams are then shared.  There is no CPU fallback: when
the library is missing every call raises ``RuntimeError``.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must precede the library load, see module docstring)

LIB_NAME = "libdllm_attn.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

DLLM_OK = 0
DLLM_ERR_INVALID_ARG = -1
DLLM_ERR_UNSUPPORTED = -2
DLLM_ERR_WORKSPACE = -3
DLLM_ERR_HIP = -4

# name -> (restype, argtypes); must match include/dllm_attn.h
_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_F = ctypes.c_float
_SZ = ctypes.c_size_t
SIGNATURES = {
    "dllm_last_error": (ctypes.c_char_p, []),
    "dllm_abi_version": (_I, []),
    "dllm_store_kvcache": (_I, [_P, _I64, _P, _I64, _P, _P, _I64, _P, _I, _I, _P]),
    "dllm_load_kvcache": (_I, [_P, _I64, _P, _I64, _P, _P, _I64, _P, _I, _I, _P]),
    "dllm_attn_varlen_fwd": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I64, _I64, _I64, _I64, _F, _P],
    ),
    "dllm_attn_varlen_launch_shape": (_I, [_I, _I, _I, _I, _I, _I, _P, _P, _P]),
    "dllm_attn_block_cached_workspace_size": (_SZ, [_I, _I, _I, _I, _I, _I]),
    "dllm_attn_block_cached_launch_shape": (_I, [_I, _I, _I, _I, _I, _I, _P, _P, _P]),
    "dllm_attn_block_cached_fwd": (
        _I,
        [_P, _P, _P, _P, _P, _P, _I, _I, _I, _P, _P, _I64, _P, _P, _I, _I, _I,
         _I64, _I64, _I64, _I64, _F, _P, _SZ, _P],
    ),
    "dllm_attn_block_cached_paged_fwd": (
        _I,
        [_P, _P, _P, _P, _P, _P, _I, _I, _I, _P, _P, _I, _P, _I, _P, _I, _I, _I,
         _I64, _I64, _I64, _I64, _F, _P, _SZ, _P],
    ),
    "dllm_attn_block_cached_noalloc_max_workspace": (_SZ, []),
    "dllm_attn_block_cached_fwd_noalloc": (
        _I,
        [_P, _P, _P, _P, _P, _P, _I, _I, _I, _P, _P, _I64, _P, _P, _I, _I, _I,
         _I64, _I64, _I64, _I64, _F, _P],
    ),
    "dllm_select_kv_workspace_size": (_SZ, [_I, _I, _I, _I, _I]),
    "dllm_select_kv_store": (
        _I,
        [_P, _P, _P, _I64, _I64, _I64, _I64, _P, _I, _I, _I, _I, _I, _I, _F,
         _P, _P, _I64, _P, _I64, _P, _P, _SZ, _P],
    ),
    "dllm_rope_neox": (_I, [_P, _I64, _P, _I64, _P, _I64, _P, _I64, _P, _P, _I64, _I, _I, _I, _I, _P]),
    "dllm_softmax_max_workspace_size": (_SZ, [_I, _I]),
    "dllm_softmax_max": (_I, [_P, _I64, _I, _I, _P, _P, _P, _SZ, _P]),
    "dllm_softmax_max_sample": (_I, [_P, _I64, _I, _I, _P, ctypes.c_uint64, _I64, _P, _P, _P, _SZ, _P]),
    "dllm_lowconf_unmask": (_I, [_P, _I64, _P, _I, _I, _P, _P, _I64, _I64, _P, _P]),
    "dllm_step_build": (_I, [_P, _P, _P, _P, _I, _I64, _P, _P, _P, _P, _P, _P, _I, _P, _P, _I, _P, _P, _I, _P, _P]),
    "dllm_step_advance": (_I, [_P, _I, _P]),
    "dllm_mfma_probe_flops": (_I64, [_I, _I]),
    "dllm_mfma_probe": (_I, [_P, _I, _I, _P]),
}

_lib = None
_lock = threading.Lock()


def load(path: str | None = None) -> ctypes.CDLL:
    """Load (once) and return the library; raise RuntimeError if it is absent."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        p = path or LIB_PATH
        if not os.path.exists(p):
            raise RuntimeError(
                f"{LIB_NAME} not found at {p}; build it with `make -C dllm-serve_amd/csrc` "
                "(or __graft_entry__.build()). There is no CPU fallback for this path."
            )
        lib = ctypes.CDLL(p)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def _check(rc: int, what: str) -> None:
    if rc != DLLM_OK:
        msg = load().dllm_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (code {rc}): {msg}")


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


# The raw handle of the device's current stream, without building a
# torch.cuda.Stream object (1.8 -> 0.1 us per kernel call).
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(device: torch.device) -> int:
    if _raw_stream is not None:
        return _raw_stream(device.index if device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(device).cuda_stream


def _require_gpu(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(
                "dllm_serve_amd kernels run on the GPU only; got a tensor on "
                f"{t.device} (there is no CPU fallback)"
            )


# ---------------------------------------------------------------- wrappers ---

def store_kvcache(key, value, k_cache, v_cache, slot_mapping, n_tok, row_elems):
    """K1: cache rows slot_mapping[i] <- key[i], value[i] (bit-exact)."""
    _require_gpu(key, value, k_cache, v_cache, slot_mapping)
    lib = load()
    rc = lib.dllm_store_kvcache(
        key.data_ptr(), key.stride(0), value.data_ptr(), value.stride(0),
        k_cache.data_ptr(), v_cache.data_ptr(), min(k_cache.numel(), v_cache.numel()) // row_elems,
        slot_mapping.data_ptr(), n_tok, row_elems, _stream(key.device))
    _check(rc, "dllm_store_kvcache")


def load_kvcache(key, value, k_cache, v_cache, slot_mapping, n_tok, row_elems):
    """K2: key[i], value[i] <- cache rows slot_mapping[i] (bit-exact)."""
    _require_gpu(key, value, k_cache, v_cache, slot_mapping)
    lib = load()
    rc = lib.dllm_load_kvcache(
        key.data_ptr(), key.stride(0), value.data_ptr(), value.stride(0),
        k_cache.data_ptr(), v_cache.data_ptr(), min(k_cache.numel(), v_cache.numel()) // row_elems,
        slot_mapping.data_ptr(), n_tok, row_elems, _stream(key.device))
    _check(rc, "dllm_load_kvcache")


def attn_varlen_fwd(q, k, v, o, cu_q, cu_k, seg_ids, n_seg, max_seqlen_q, scale, max_seqlen_k=None):
    """K3a: bidirectional varlen attention of segments (q,k,v,o are [rows, H, D])."""
    _require_gpu(q, k, v, o, cu_q, cu_k)
    lib = load()
    if max_seqlen_k is None:
        max_seqlen_k = max_seqlen_q
    rc = lib.dllm_attn_varlen_fwd(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
        cu_q.data_ptr(), cu_k.data_ptr(), _ptr(seg_ids), n_seg, max_seqlen_q, max_seqlen_k,
        q.shape[1], k.shape[1], q.shape[2],
        q.stride(0), k.stride(0), v.stride(0), o.stride(0), float(scale),
        _stream(q.device))
    _check(rc, "dllm_attn_varlen_fwd")


def _lib_now() -> ctypes.CDLL:
    return _lib if _lib is not None else load()


def attn_varlen_fwd_raw(q_ptr, k_ptr, v_ptr, o_ptr, cu_ptr, ids_ptr, n_seg, max_q, Hq, Hkv, D, q_st, k_st, v_st,
                        o_st, scale, stream) -> None:
    """attn_varlen_fwd over device addresses and token strides (elements) the
    caller has already checked; Lq == Lk per segment (cu_q is cu_k)."""
    rc = _lib_now().dllm_attn_varlen_fwd(q_ptr, k_ptr, v_ptr, o_ptr, cu_ptr, cu_ptr, ids_ptr, n_seg, max_q, max_q,
                                         Hq, Hkv, D, q_st, k_st, v_st, o_st, scale, stream)
    if rc != DLLM_OK:
        _check(rc, "dllm_attn_varlen_fwd")


def attn_block_cached_fwd_raw(q_ptr, k_ptr, v_ptr, o_ptr, cu_ptr, ids_ptr, n_seg, max_q, max_keys, kc_ptr, vc_ptr,
                              cache_slots, slots_ptr, slot_off_ptr, Hq, Hkv, D, q_st, k_st, v_st, o_st, scale,
                              ws_ptr, ws_bytes, stream) -> None:
    """attn_block_cached_fwd over device addresses (see attn_varlen_fwd_raw)."""
    rc = _lib_now().dllm_attn_block_cached_fwd(q_ptr, k_ptr, v_ptr, o_ptr, cu_ptr, ids_ptr, n_seg, max_q, max_keys,
                                               kc_ptr, vc_ptr, cache_slots, slots_ptr, slot_off_ptr, Hq, Hkv, D,
                                               q_st, k_st, v_st, o_st, scale, ws_ptr, ws_bytes, stream)
    if rc != DLLM_OK:
        _check(rc, "dllm_attn_block_cached_fwd")


def varlen_launch_shape(n_seg, max_seqlen_q, max_seqlen_k, Hq, Hkv, D) -> dict:
    """Launch shape K3a picks for these sizes (no launch): wavefronts per
    workgroup, keys per tile, grid."""
    vals = [ctypes.c_int(0) for _ in range(3)]
    _check(load().dllm_attn_varlen_launch_shape(n_seg, max_seqlen_q, max_seqlen_k, Hq, Hkv, D,
                                                *[ctypes.byref(x) for x in vals]), "dllm_attn_varlen_launch_shape")
    return dict(wavefronts=vals[0].value, tile_keys=vals[1].value, grid=vals[2].value)


def block_cached_launch_shape(n_seg, max_q, max_keys, Hq, Hkv, D) -> dict:
    """Launch shape K3b picks for these sizes (no launch): row blocks per
    workgroup, key splits, grid."""
    vals = [ctypes.c_int(0) for _ in range(3)]
    _check(load().dllm_attn_block_cached_launch_shape(n_seg, max_q, max_keys, Hq, Hkv, D,
                                                      *[ctypes.byref(x) for x in vals]),
           "dllm_attn_block_cached_launch_shape")
    return dict(row_blocks=vals[0].value, n_split=vals[1].value, grid=vals[2].value)


def block_cached_workspace_size(n_seg, max_q, max_keys, Hq, Hkv, D) -> int:
    return int(load().dllm_attn_block_cached_workspace_size(n_seg, max_q, max_keys, Hq, Hkv, D))


def attn_block_cached_fwd(q, k, v, o, cu, seg_ids, n_seg, max_q, max_keys,
                          k_cache, v_cache, slots, slot_off, scale, workspace):
    """K3b: block rows attend to [cached rows (by slot) ; block rows]."""
    _require_gpu(q, k, v, o, cu, slot_off)
    lib = load()
    Hkv, D = k.shape[1], k.shape[2]
    cache_slots = (min(k_cache.numel(), v_cache.numel()) // (Hkv * D)
                   if k_cache is not None and v_cache is not None and k_cache.numel() else 0)
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    rc = lib.dllm_attn_block_cached_fwd(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
        cu.data_ptr(), _ptr(seg_ids), n_seg, max_q, max_keys,
        _ptr(k_cache) if cache_slots else None, _ptr(v_cache) if cache_slots else None,
        cache_slots, _ptr(slots) if cache_slots else None, slot_off.data_ptr(),
        q.shape[1], Hkv, D,
        q.stride(0), k.stride(0), v.stride(0), o.stride(0), float(scale),
        _ptr(workspace), ws_bytes, _stream(q.device))
    _check(rc, "dllm_attn_block_cached_fwd")


def attn_block_cached_paged_fwd_raw(q_ptr, k_ptr, v_ptr, o_ptr, cu_ptr, ids_ptr, n_seg, max_q, max_keys, kc_ptr,
                                    vc_ptr, num_pages, pt_ptr, max_pages, len_ptr, Hq, Hkv, D, q_st, k_st, v_st, o_st,
                                    scale, ws_ptr, ws_bytes, stream) -> None:
    """attn_block_cached_paged_fwd over device addresses (see attn_varlen_fwd_raw)."""
    rc = _lib_now().dllm_attn_block_cached_paged_fwd(q_ptr, k_ptr, v_ptr, o_ptr, cu_ptr, ids_ptr, n_seg, max_q,
                                                     max_keys, kc_ptr, vc_ptr, num_pages, pt_ptr, max_pages, len_ptr,
                                                     Hq, Hkv, D, q_st, k_st, v_st, o_st, scale, ws_ptr, ws_bytes,
                                                     stream)
    if rc != DLLM_OK:
        _check(rc, "dllm_attn_block_cached_paged_fwd")


def attn_block_cached_paged_fwd(q, k, v, o, cu, seg_ids, n_seg, max_q, max_keys, k_cache, v_cache, page_table,
                                cached_len, scale, workspace):
    """K3b, page-table form: segment s's cached rows are rows r < cached_len[s]
    of its pages page_table[s, r // 256] (256-row pages of the cache, given
    as [num_pages, 256, Hkv, D] or flat rows)."""
    # the kernel reads int32 rows of the table (one per launch segment) and int32 lengths
    if page_table.dtype != torch.int32 or page_table.dim() != 2 or page_table.stride(1) != 1 \
            or page_table.stride(0) != page_table.shape[1] or page_table.shape[0] < n_seg:
        raise ValueError("page_table must be a contiguous int32 [n_seg, max_pages] tensor, one row per launch "
                         f"segment; got {tuple(page_table.shape)} {page_table.dtype}")
    if cached_len.dtype != torch.int32 or not cached_len.is_contiguous() or cached_len.numel() < n_seg:
        raise ValueError(f"cached_len must be a contiguous int32 tensor of n_seg = {n_seg} lengths; "
                         f"got {tuple(cached_len.shape)} {cached_len.dtype}")
    _require_gpu(q, k, v, o, cu, page_table, cached_len)
    lib = load()
    Hkv, D = k.shape[1], k.shape[2]
    rows = (min(k_cache.numel(), v_cache.numel()) // (Hkv * D)
            if k_cache is not None and v_cache is not None and k_cache.numel() else 0)
    num_pages = rows // 256
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    rc = lib.dllm_attn_block_cached_paged_fwd(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), cu.data_ptr(), _ptr(seg_ids), n_seg, max_q,
        max_keys, _ptr(k_cache) if num_pages else None, _ptr(v_cache) if num_pages else None, num_pages,
        page_table.data_ptr(), page_table.shape[1],
        cached_len.data_ptr(), q.shape[1], Hkv, D, q.stride(0), k.stride(0), v.stride(0), o.stride(0), float(scale),
        _ptr(workspace), ws_bytes, _stream(q.device))
    _check(rc, "dllm_attn_block_cached_paged_fwd")


def block_cached_noalloc_max_workspace() -> int:
    return int(load().dllm_attn_block_cached_noalloc_max_workspace())


def attn_block_cached_fwd_noalloc(q, k, v, o, cu, seg_ids, n_seg, max_q, max_keys,
                                  k_cache, v_cache, slots, slot_off, scale):
    """K3b with its split partials in the library's static device scratch
    (allocates nothing; calls that overlap on one GPU race)."""
    _require_gpu(q, k, v, o, cu, slot_off)
    lib = load()
    Hkv, D = k.shape[1], k.shape[2]
    cache_slots = (min(k_cache.numel(), v_cache.numel()) // (Hkv * D)
                   if k_cache is not None and v_cache is not None and k_cache.numel() else 0)
    rc = lib.dllm_attn_block_cached_fwd_noalloc(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
        cu.data_ptr(), _ptr(seg_ids), n_seg, max_q, max_keys,
        _ptr(k_cache) if cache_slots else None, _ptr(v_cache) if cache_slots else None,
        cache_slots, _ptr(slots) if cache_slots else None, slot_off.data_ptr(),
        q.shape[1], Hkv, D,
        q.stride(0), k.stride(0), v.stride(0), o.stride(0), float(scale), _stream(q.device))
    _check(rc, "dllm_attn_block_cached_fwd_noalloc")


JOB_COLS = 8  # row0, n_tok, blk_start, blk_len, n_keep, slot_off, head_select, pool_k


def select_workspace_size(n_job, max_kc, Hq, Hkv, D) -> int:
    return int(load().dllm_select_kv_workspace_size(n_job, max_kc, Hq, Hkv, D))


def select_kv_store(q, k, v, jobs, n_job, max_kc, max_keep, sqrt_d, k_cache, v_cache, slots, idx_out, workspace):
    """K5/K6: selection + fused cache scatter; jobs int32 [n_job, 8] carry each
    sequence's head_select and pool_kernel (see include/dllm_attn.h)."""
    _require_gpu(q, k, v, jobs, k_cache, v_cache, slots)
    lib = load()
    Hq, Hkv, D = q.shape[1], k.shape[1], q.shape[2]
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    rc = lib.dllm_select_kv_store(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), min(q.shape[0], k.shape[0], v.shape[0]),
        q.stride(0), k.stride(0), v.stride(0),
        jobs.data_ptr(), n_job, max_kc, max_keep, Hq, Hkv, D, float(sqrt_d),
        k_cache.data_ptr(), v_cache.data_ptr(), min(k_cache.numel(), v_cache.numel()) // (Hkv * D),
        slots.data_ptr(), slots.numel(), _ptr(idx_out), _ptr(workspace), ws_bytes, _stream(q.device))
    _check(rc, "dllm_select_kv_store")


def rope_neox(q_in, q_out, k_in, k_out, positions, cos_sin_cache, n_tok, Hq, Hkv, D):
    """K7: NeoX rotary embedding of q and k (token-major, last dim contiguous).
    q_out / k_out may be q_in / k_in (in place)."""
    _require_gpu(q_in, q_out, k_in, k_out, positions, cos_sin_cache)
    lib = load()
    rc = lib.dllm_rope_neox(
        _ptr(q_in), q_in.stride(0) if q_in is not None else 0,
        _ptr(q_out), q_out.stride(0) if q_out is not None else 0,
        _ptr(k_in), k_in.stride(0) if k_in is not None else 0,
        _ptr(k_out), k_out.stride(0) if k_out is not None else 0,
        positions.data_ptr(), cos_sin_cache.data_ptr(), cos_sin_cache.shape[0],
        n_tok, Hq, Hkv, D, _stream(positions.device))
    _check(rc, "dllm_rope_neox")


def softmax_max_workspace_size(M, V) -> int:
    return int(load().dllm_softmax_max_workspace_size(M, V))


def softmax_max(logits, x0, x0_p, workspace=None):
    """K8: x0_p, x0 = max(softmax(logits, -1), -1) of bf16 logits [M, V]
    (x0 int64 [M], x0_p bf16 [M]).  workspace is optional (the kernel needs none)."""
    _require_gpu(logits, x0, x0_p, workspace)
    lib = load()
    M, V = logits.shape
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    rc = lib.dllm_softmax_max(logits.data_ptr(), logits.stride(0), M, V, x0.data_ptr(), x0_p.data_ptr(),
                              _ptr(workspace), ws_bytes, _stream(logits.device))
    _check(rc, "dllm_softmax_max")


def softmax_max_sample(logits, row_temperature, seed, row_base, x0, x0_p, workspace=None):
    """K8 with Gumbel noise on the rows whose temperature is > 0
    (row_temperature: float64 [M] on the device, or None)."""
    _require_gpu(logits, row_temperature, x0, x0_p, workspace)
    lib = load()
    M, V = logits.shape
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    rc = lib.dllm_softmax_max_sample(logits.data_ptr(), logits.stride(0), M, V, _ptr(row_temperature),
                                     int(seed) & 0xFFFFFFFFFFFFFFFF, int(row_base), x0.data_ptr(), x0_p.data_ptr(),
                                     _ptr(workspace), ws_bytes, _stream(logits.device))
    _check(rc, "dllm_softmax_max_sample")


def lowconf_unmask(tokens, seq_params, n_seq, max_win, x0, conf, mask_id, n_unmasked=None):
    """K9: one low-confidence unmasking step of n_seq windows of the flat
    int64 token array (seq_params: int32 [n_seq, 5], see include/dllm_attn.h)."""
    _require_gpu(tokens, seq_params, x0, conf, n_unmasked)
    lib = load()
    rc = lib.dllm_lowconf_unmask(tokens.data_ptr(), tokens.numel(), seq_params.data_ptr(), n_seq, max_win,
                                 x0.data_ptr(), conf.data_ptr(), x0.numel(), int(mask_id), _ptr(n_unmasked),
                                 _stream(tokens.device))
    _check(rc, "dllm_lowconf_unmask")


def step_build(state, ratio, pages, page_off, n_seq, tok_stride, cu, dense_ids, cached_ids, slot_off, jobs,
               slots, positions, token_index, smp_params, smp_rows, counts):
    """S1: one step's launch tables, fed-row positions and sampler windows
    from the device state table (see include/dllm_attn.h)."""
    _require_gpu(state, ratio, page_off, cu, counts)
    lib = load()
    rc = lib.dllm_step_build(state.data_ptr(), ratio.data_ptr(), _ptr(pages), page_off.data_ptr(), n_seq,
                             int(tok_stride), cu.data_ptr(), dense_ids.data_ptr(), cached_ids.data_ptr(),
                             slot_off.data_ptr(), jobs.data_ptr(), _ptr(slots), slots.numel(),
                             positions.data_ptr(), token_index.data_ptr(), positions.numel(),
                             smp_params.data_ptr(), smp_rows.data_ptr(), smp_rows.numel(), counts.data_ptr(),
                             _stream(state.device))
    _check(rc, "dllm_step_build")


def step_advance(state, n_seq):
    """S2: advance every sequence's step / block / cache state on the device."""
    _require_gpu(state)
    rc = load().dllm_step_advance(state.data_ptr(), n_seq, _stream(state.device))
    _check(rc, "dllm_step_advance")


def mfma_probe(sink, n_cu: int, iters: int) -> int:
    """Launch the register-only MFMA clock probe on the current stream;
    returns its FLOPs (sink: float32 [n_cu * 512] on the device)."""
    _require_gpu(sink)
    lib = load()
    _check(lib.dllm_mfma_probe(sink.data_ptr(), n_cu, iters, _stream(sink.device)), "dllm_mfma_probe")
    return int(lib.dllm_mfma_probe_flops(n_cu, iters))
