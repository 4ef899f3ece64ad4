"""The C ABI library loads on the host, exports every entry point that
include/dllm_attn.h declares with the arity the ctypes binding uses, and
rejects invalid requests before touching the GPU (no kernel is launched)."""
import ctypes
import os
import re

import pytest

from dllm_serve_amd import _capi

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "dllm_attn.h")


def _declarations():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    decls = {}
    for m in re.finditer(r"\b(dllm_\w+)\s*\(([^;{]*?)\)\s*;", text, flags=re.S):
        params = m.group(2).strip()
        decls[m.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return decls


def test_library_exports_every_declared_symbol():
    lib = _capi.load()
    decls = _declarations()
    assert len(decls) >= 9
    for name, arity in decls.items():
        assert hasattr(lib, name), name
        assert name in _capi.SIGNATURES, name
        assert len(_capi.SIGNATURES[name][1]) == arity, (name, arity)
    assert lib.dllm_abi_version() >= 100


def test_workspace_size_functions():
    # one split: no workspace; few long segments: split over keys
    assert _capi.block_cached_workspace_size(1024, 32, 4000, 32, 32, 128) == 0
    ws = _capi.block_cached_workspace_size(2, 32, 4128, 32, 32, 128)
    assert ws > 0 and ws % 4 == 0
    # raw scores, token-selection partial sums, order keys, selections
    assert _capi.select_workspace_size(4, 1216, 32, 32, 128) >= 4 * 32 * 1216 * (2 + 8 + 2 + 4)
    assert _capi.select_workspace_size(0, 10, 32, 32, 128) == 0
    # beyond the in-LDS sort the radix-sort ping-pong buffers are added
    small = _capi.select_workspace_size(1, 8192, 32, 32, 128)
    assert _capi.select_workspace_size(1, 8193, 32, 32, 128) >= small + 2 * 32 * 8193 * (2 + 4)


def _err(rc):
    return rc, _capi.load().dllm_last_error().decode()


def test_argument_validation_without_gpu():
    lib = _capi.load()
    P = ctypes.c_void_p
    fake = P(4096)  # never dereferenced: every call below fails validation first
    rc, msg = _err(lib.dllm_attn_varlen_fwd(fake, fake, fake, fake, fake, fake, None, 1, 8, 8, 4, 4, 64,
                                            256, 256, 256, 256, 0.125, None))
    assert rc == _capi.DLLM_ERR_UNSUPPORTED and "head_dim" in msg
    rc, msg = _err(lib.dllm_attn_varlen_fwd(fake, fake, fake, fake, fake, fake, None, 1, 8, 8, 6, 4, 128,
                                            768, 512, 512, 768, 0.1, None))
    assert rc == _capi.DLLM_ERR_INVALID_ARG and "multiple" in msg
    rc, msg = _err(lib.dllm_attn_varlen_fwd(P(4098), fake, fake, fake, fake, fake, None, 1, 8, 8, 4, 4, 128,
                                            512, 512, 512, 512, 0.1, None))
    assert rc == _capi.DLLM_ERR_INVALID_ARG and "aligned" in msg
    assert lib.dllm_attn_varlen_fwd(fake, fake, fake, fake, fake, fake, None, 0, 8, 8, 4, 4, 128,
                                    512, 512, 512, 512, 0.1, None) == 0   # nothing to do
    # two 32-row blocks against 4096 cached rows split over the keys and need a workspace
    assert _capi.block_cached_workspace_size(2, 32, 4128, 32, 32, 128) > 0
    rc, msg = _err(lib.dllm_attn_block_cached_fwd(fake, fake, fake, fake, fake, None, 2, 32, 4128, fake, fake,
                                                  4096, fake, fake, 32, 32, 128, 4096, 4096, 4096, 4096, 0.1,
                                                  None, 0, None))
    assert rc == _capi.DLLM_ERR_WORKSPACE
    # selection: no candidate cap any more; the workspace and the group size are checked
    need = _capi.select_workspace_size(1, 9000, 32, 32, 128)
    rc, msg = _err(lib.dllm_select_kv_store(fake, fake, fake, 9064, 4096, 4096, 4096, fake, 1, 9000, 100, 32, 32,
                                            128, 11.3, fake, fake, 4096, fake, 100, None, fake, need - 1, None))
    assert rc == _capi.DLLM_ERR_WORKSPACE
    rc, msg = _err(lib.dllm_select_kv_store(fake, fake, fake, 9064, 65 * 128, 128, 128, fake, 1, 9000, 100, 65, 1,
                                            128, 11.3, fake, fake, 4096, fake, 100, None, fake, 1 << 30, None))
    assert rc == _capi.DLLM_ERR_UNSUPPORTED and "query heads per KV head" in msg
    rc, msg = _err(lib.dllm_select_kv_store(fake, fake, fake, 9064, 4096, 4096, 4096, fake, 1, 90, 100, 32, 32,
                                            128, 11.3, fake, fake, 4096, fake, 100, None, fake, 1 << 30, None))
    assert rc == _capi.DLLM_ERR_INVALID_ARG and "max_keep" in msg
    rc, msg = _err(lib.dllm_store_kvcache(None, 4096, None, 4096, None, None, 10, None, 3, 4096, None))
    assert rc == _capi.DLLM_ERR_INVALID_ARG
    assert lib.dllm_store_kvcache(None, 4096, None, 4096, None, None, 10, None, 0, 4096, None) == 0


def test_paged_block_cached_validation_without_gpu():
    """The page-table form rejects what it cannot address before any launch:
    a cache that is not whole 256-row pages, a missing page table or cached
    lengths, a page-table row length that the launch cannot carry, and a
    missing workspace when the keys are split."""
    lib = _capi.load()
    P = ctypes.c_void_p
    fake = P(4096)

    def call(num_pages=16, pt=fake, max_pages=4, clen=fake, n_seg=2, max_keys=96, ws=None, ws_bytes=0,
             kc=fake, vc=fake):
        return _err(lib.dllm_attn_block_cached_paged_fwd(fake, fake, fake, fake, fake, None, n_seg, 32, max_keys,
                                                         kc, vc, num_pages, pt, max_pages, clen, 32, 32, 128,
                                                         4096, 4096, 4096, 4096, 0.1, ws, ws_bytes, None))

    rc, msg = call(num_pages=-1)
    assert rc == _capi.DLLM_ERR_INVALID_ARG and "num_pages" in msg
    rc, msg = call(clen=None)
    assert rc == _capi.DLLM_ERR_INVALID_ARG and "cached_len" in msg
    rc, msg = call(pt=None)
    assert rc == _capi.DLLM_ERR_INVALID_ARG and "page table" in msg
    rc, msg = call(max_pages=0)
    assert rc == _capi.DLLM_ERR_INVALID_ARG and "max_pages" in msg
    rc, msg = call(max_pages=1 << 26)
    assert rc == _capi.DLLM_ERR_INVALID_ARG and "page table too large" in msg
    rc, msg = call(kc=None)
    assert rc == _capi.DLLM_ERR_INVALID_ARG
    # two 32-row blocks against 4096 cached rows: split over the keys, a workspace is needed
    need = _capi.block_cached_workspace_size(2, 32, 4128, 32, 32, 128)
    assert need > 0
    rc, msg = call(max_keys=4128, max_pages=16)
    assert rc == _capi.DLLM_ERR_WORKSPACE
    # nothing to do: no segments
    assert call(n_seg=0)[0] == 0


def test_paged_wrapper_checks_table_and_lengths():
    """The Python wrapper refuses a page table or lengths the kernel would
    misread (wrong dtype, not one contiguous row per segment, too few rows)."""
    import torch
    q = k = v = o = torch.zeros(4, 2, 128, dtype=torch.bfloat16)
    cu = torch.tensor([0, 2, 4], dtype=torch.int32)
    good_pt = torch.zeros(2, 3, dtype=torch.int32)
    good_len = torch.zeros(2, dtype=torch.int32)
    bad_tables = [torch.zeros(2, 3, dtype=torch.int64), torch.zeros(6, dtype=torch.int32),
                  torch.zeros(3, 2, dtype=torch.int32).t(), torch.zeros(1, 3, dtype=torch.int32)]
    for pt in bad_tables:
        with pytest.raises(ValueError, match="page_table"):
            _capi.attn_block_cached_paged_fwd(q, k, v, o, cu, None, 2, 2, 6, None, None, pt, good_len, 0.1, None)
    for ln in (torch.zeros(2, dtype=torch.int64), torch.zeros(1, dtype=torch.int32)):
        with pytest.raises(ValueError, match="cached_len"):
            _capi.attn_block_cached_paged_fwd(q, k, v, o, cu, None, 2, 2, 6, None, None, good_pt, ln, 0.1, None)
    # well-formed arguments get as far as the GPU check
    with pytest.raises(RuntimeError, match="GPU only"):
        _capi.attn_block_cached_paged_fwd(q, k, v, o, cu, None, 2, 2, 6, None, None, good_pt, good_len, 0.1, None)


def test_missing_library_fails_loudly(tmp_path, monkeypatch):
    monkeypatch.setattr(_capi, "_lib", None)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        _capi.load(str(tmp_path / "absent.so"))


def test_rope_validation_without_gpu():
    lib = _capi.load()
    P = ctypes.c_void_p
    fake = P(4096)
    rc, msg = _err(lib.dllm_rope_neox(fake, 512, fake, 512, fake, 512, fake, 512, fake, fake, 64,
                                      4, 4, 4, 72, None))
    assert rc == _capi.DLLM_ERR_UNSUPPORTED and "head_dim" in msg
    rc, msg = _err(lib.dllm_rope_neox(P(4098), 512, fake, 512, fake, 512, fake, 512, fake, fake, 64,
                                      4, 4, 4, 128, None))
    assert rc == _capi.DLLM_ERR_INVALID_ARG and "aligned" in msg
    rc, msg = _err(lib.dllm_rope_neox(fake, 100, fake, 512, fake, 512, fake, 512, fake, fake, 64,
                                      4, 4, 4, 128, None))
    assert rc == _capi.DLLM_ERR_INVALID_ARG and "stride" in msg
    assert lib.dllm_rope_neox(fake, 512, fake, 512, fake, 512, fake, 512, fake, fake, 64, 0, 4, 4, 128, None) == 0


def test_rope_module_refuses_cpu_tensors():
    import torch
    from dllm_serve_amd.layers.rotary_embedding import RotaryEmbedding, get_rope

    assert get_rope(128, 128, 64, 10000.0) is get_rope(128, 128, 64, 10000.0)
    rope = RotaryEmbedding(128, 128, 64, 10000.0)
    assert rope.cos_sin_cache.shape == (64, 128) and rope.cos_sin_cache.dtype == torch.float32
    q = torch.zeros(4, 2 * 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU only"):
        rope(torch.arange(4), q, q.clone())


def test_sampler_validation_without_gpu():
    lib = _capi.load()
    P = ctypes.c_void_p
    fake = P(4096)
    # one workgroup per row: no workspace at any size, and a null one is accepted
    assert _capi.softmax_max_workspace_size(1024, 126464) == 0
    assert _capi.softmax_max_workspace_size(64, 126464) == 0
    ws = 0
    rc, msg = _err(lib.dllm_softmax_max(fake, 126464, 64, 126460, fake, fake, fake, ws, None))
    assert rc == _capi.DLLM_ERR_UNSUPPORTED and "multiple of 8" in msg
    rc, msg = _err(lib.dllm_softmax_max(fake, 126456, 64, 126464, fake, fake, fake, ws, None))
    assert rc == _capi.DLLM_ERR_INVALID_ARG and "stride" in msg
    rc, msg = _err(lib.dllm_softmax_max(None, 126464, 64, 126464, fake, fake, None, 0, None))
    assert rc == _capi.DLLM_ERR_INVALID_ARG and "null" in msg
    assert lib.dllm_softmax_max(fake, 126464, 0, 126464, fake, fake, None, 0, None) == 0
    rc, msg = _err(lib.dllm_lowconf_unmask(fake, 100, fake, 4, 8193, fake, fake, 100, 126336, None, None))
    assert rc == _capi.DLLM_ERR_UNSUPPORTED and "8192" in msg
    assert lib.dllm_lowconf_unmask(fake, 100, fake, 0, 10, fake, fake, 100, 126336, None, None) == 0


def test_sampler_refuses_cpu_tensors():
    import torch
    from dllm_serve_amd.engine.sampler import RemaskSampler, step_windows
    from dllm_serve_amd.engine.sequence import Sequence
    from dllm_serve_amd.sparse.state import SparseConfig

    seqs = [Sequence([1] * 10, 8, 99, None, device="cpu", steps=4),
            Sequence([2] * 6, 8, 99, SparseConfig(default_block_len=4), device="cpu")]
    # (hidden row, window start, length, steps_remain, first-token rule)
    assert step_windows(seqs) == [(10, 10, 8, 4, 0), (18 + 6, 6, 4, 4, 1)]
    seqs[0].current_step = 4
    with pytest.raises(ZeroDivisionError):
        step_windows(seqs)
    seqs[0].current_step = 0
    s = RemaskSampler(lambda h: h, 99)
    with pytest.raises(RuntimeError, match="GPU only"):
        s(torch.zeros(32, 8, dtype=torch.bfloat16), seqs, torch.zeros(2, 18, dtype=torch.int64))
    with pytest.raises(NotImplementedError):
        s(torch.zeros(32, 8, dtype=torch.bfloat16), seqs, torch.zeros(2, 18, dtype=torch.int64), remasking="topk")


def test_launch_shape_queries():
    """The launch shapes the benchmark workloads run (host-side planning only)."""
    c2 = _capi.varlen_launch_shape(8, 384, 384, 32, 32, 128)
    assert c2 == dict(wavefronts=12, tile_keys=32, grid=256)      # one workgroup per (sequence, head)
    assert _capi.varlen_launch_shape(4, 384, 384, 32, 32, 128)["wavefronts"] == 4   # 128 pairs: < 160
    c4 = _capi.varlen_launch_shape(4, 1280, 1280, 32, 32, 128)
    assert c4["wavefronts"] == 4 and c4["tile_keys"] == 32 and c4["grid"] >= 4 * 32 * 10
    assert _capi.varlen_launch_shape(2, 4096, 4096, 32, 32, 128)["wavefronts"] == 8
    assert _capi.varlen_launch_shape(16, 1245, 1245, 28, 4, 128)["wavefronts"] == 4
    assert _capi.varlen_launch_shape(0, 384, 384, 32, 32, 128)["grid"] == 0
    c5 = _capi.block_cached_launch_shape(32, 32, 4128, 32, 32, 128)
    assert c5["row_blocks"] == 1 and c5["n_split"] == 1 and c5["grid"] >= 32 * 32
    dream = _capi.block_cached_launch_shape(16, 32, 732, 28, 4, 128)   # 7 M tiles per (segment, KV head)
    assert dream["row_blocks"] == 2 and dream["n_split"] == 1
    assert _capi.block_cached_launch_shape(2, 32, 4128, 32, 32, 128)["n_split"] > 1
    with pytest.raises(RuntimeError):
        _capi.varlen_launch_shape(1, 8, 8, 32, 32, 64)
