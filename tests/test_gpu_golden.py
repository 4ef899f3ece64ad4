"""GPU kernels against the committed golden fixtures."""
import os

import numpy as np
import pytest
import torch

from oracle import configs
from dllm_serve_amd import _capi

pytestmark = pytest.mark.gpu
HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def test_c1_attention_fixture(dev):
    """bf16 GPU attention at C1 vs the fp32 fixture sample (bf16 inputs are
    the fixture's fp32 inputs rounded: max-abs 2e-2, mean-abs 2e-3)."""
    print("golden C1", flush=True)
    fx = np.load(os.path.join(HERE, "c1_attention.npz"))
    q, k, v, cu, scale = configs.c1_single_layer()
    qd, kd, vd = (t.to(torch.bfloat16).to(dev) for t in (q, k, v))
    o = torch.empty_like(qd)
    cud = cu.to(dev)
    _capi.attn_varlen_fwd(qd, kd, vd, o, cud, cud, None, 1, 512, scale)
    torch.cuda.synchronize()
    got = o.float().cpu().numpy().reshape(-1)[::int(fx["stride"])]
    err = np.abs(got - fx["out_sample"])
    assert err.max() <= 2e-2 and err.mean() <= 2e-3, (err.max(), err.mean())


def test_select_fixtures(dev):
    print("golden select", flush=True)
    fx = np.load(os.path.join(HERE, "select_cases.npz"))
    for name in ("mha_hs", "gqa_hs", "gqa_tok"):
        Lb, Kc, Hq, Hkv, n_keep, hs, pk = (int(x) for x in fx[f"{name}_params"])
        qb = torch.from_numpy(fx[f"{name}_q"].view(np.int16)).view(torch.bfloat16)
        kb = torch.from_numpy(fx[f"{name}_k"].view(np.int16)).view(torch.bfloat16)
        # sequence = [block rows ; candidate rows] with the block first (blk_start 0)
        n_tok = Lb + Kc
        q = torch.zeros(n_tok, Hq, 128, dtype=torch.bfloat16)
        q[:Lb] = qb
        k = torch.zeros(n_tok, Hkv, 128, dtype=torch.bfloat16)
        k[Lb:] = kb
        v = k.clone()
        jobs = torch.tensor([[0, n_tok, 0, Lb, n_keep, 0]], dtype=torch.int32, device=dev)
        cache = torch.zeros(2, 256, Hkv, 128, dtype=torch.bfloat16, device=dev)
        slots = torch.arange(n_keep, dtype=torch.int32, device=dev)
        n_sel = Hkv if hs else 1
        idx = torch.full((1, n_sel, n_keep), -1, dtype=torch.int64, device=dev)
        ws = torch.empty(_capi.select_workspace_size(1, Kc, Hq, Hkv, 128, hs), dtype=torch.uint8, device=dev)
        _capi.select_kv_store(q.to(dev), k.to(dev), v.to(dev), jobs, 1, Kc, n_keep, Lb, hs, pk,
                              np.float32(128 ** 0.5), cache[0], cache[1], slots, idx, ws)
        torch.cuda.synchronize()
        want = fx[f"{name}_idx"] if hs else fx[f"{name}_idx"][None, :]
        assert np.array_equal(idx.cpu().numpy()[0], want), name
