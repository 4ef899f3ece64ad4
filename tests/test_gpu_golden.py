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
        jobs = torch.tensor([[0, n_tok, 0, Lb, n_keep, 0, hs, pk]], dtype=torch.int32, device=dev)
        cache = torch.zeros(2, 256, Hkv, 128, dtype=torch.bfloat16, device=dev)
        slots = torch.arange(n_keep, dtype=torch.int32, device=dev)
        idx = torch.full((1, Hkv, n_keep), -1, dtype=torch.int64, device=dev)
        ws = torch.empty(_capi.select_workspace_size(1, Kc, Hq, Hkv, 128), dtype=torch.uint8, device=dev)
        _capi.select_kv_store(q.to(dev), k.to(dev), v.to(dev), jobs, 1, Kc, n_keep,
                              np.float32(128 ** 0.5), cache[0], cache[1], slots, idx, ws)
        torch.cuda.synchronize()
        got = idx.cpu().numpy()[0] if hs else idx.cpu().numpy()[0][:1]
        want = fx[f"{name}_idx"] if hs else fx[f"{name}_idx"][None, :]
        assert np.array_equal(got, want), name


def test_rope_fixture(dev):
    print("golden rope", flush=True)
    fx = np.load(os.path.join(HERE, "rope_cases.npz"))
    n, H, D = fx["x"].shape
    table = torch.zeros(int(fx["max_position"]), D, dtype=torch.float32)
    pos = torch.from_numpy(fx["pos"])
    table[pos] = torch.from_numpy(fx["table_rows"])
    x = torch.from_numpy(fx["x"].view(np.int16)).view(torch.bfloat16).to(dev)
    out = torch.empty_like(x)
    k = torch.empty(n, 0, D, dtype=torch.bfloat16, device=dev)
    _capi.rope_neox(x, out, k, k, pos.to(dev), table.to(dev), n, H, 0, D)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().view(torch.int16).numpy().view(np.uint16), fx["out"])


def test_sampler_fixture(dev):
    print("golden sampler", flush=True)
    fx = np.load(os.path.join(HERE, "sampler_cases.npz"))
    logits = torch.from_numpy(fx["logits"].view(np.int16)).view(torch.bfloat16).to(dev)
    M, V = logits.shape
    x0 = torch.empty(M, dtype=torch.int64, device=dev)
    p = torch.empty(M, dtype=torch.bfloat16, device=dev)
    ws = torch.empty(_capi.softmax_max_workspace_size(M, V), dtype=torch.uint8, device=dev)
    _capi.softmax_max(logits, x0, p, ws)
    tok = torch.from_numpy(fx["tokens"]).to(dev)
    params = torch.from_numpy(fx["params"]).to(dev)
    conf = torch.from_numpy(fx["conf"].view(np.int16)).view(torch.bfloat16).to(dev)
    pred = torch.from_numpy(fx["pred"]).to(dev)
    nun = torch.empty(params.shape[0], dtype=torch.int32, device=dev)
    _capi.lowconf_unmask(tok, params, params.shape[0], int(fx["params"][:, 1].max()), pred, conf,
                         int(fx["mask_id"]), nun)
    torch.cuda.synchronize()
    assert np.array_equal(x0.cpu().numpy(), fx["x0"])
    d = np.abs(p.cpu().view(torch.int16).numpy().view(np.uint16).astype(int) - fx["x0_p"].astype(int))
    assert d.max() <= 1 and np.mean(d == 0) >= 0.9
    assert np.array_equal(tok.cpu().numpy(), fx["tokens_out"]) and np.array_equal(nun.cpu().numpy(), fx["n_unmasked"])
