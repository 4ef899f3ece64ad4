"""The oracle reproduces the committed golden fixtures (CPU)."""
import os

import numpy as np

from oracle.bf16 import bf16_bits_to_f32

import importlib.util

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
_spec = importlib.util.spec_from_file_location("make_golden", os.path.join(HERE, "make_golden.py"))
mg = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(mg)


def test_c1_fixture():
    fx = np.load(os.path.join(HERE, "c1_attention.npz"))
    now = mg.c1()
    assert np.allclose(now["input_sums"], fx["input_sums"], rtol=1e-9)
    assert np.abs(now["out_sample"] - fx["out_sample"]).max() < 1e-5
    assert np.allclose(now["head_norms"], fx["head_norms"], rtol=1e-6)


def test_select_fixtures():
    fx = np.load(os.path.join(HERE, "select_cases.npz"))
    for name, Lb, Kc, Hq, Hkv, n_keep, hs, pk, seed in mg.SELECT_CASES:
        qb, kb, idx = mg.select_case(Lb, Kc, Hq, Hkv, n_keep, hs, pk, seed)
        assert np.array_equal(qb, fx[f"{name}_q"]) and np.array_equal(kb, fx[f"{name}_k"])
        assert np.array_equal(idx, fx[f"{name}_idx"]), name


def test_rope_fixture():
    import torch

    from oracle import rope as orope

    fx = np.load(os.path.join(HERE, "rope_cases.npz"))
    n = fx["x"].shape[0]
    # the oracle on the stored table rows (row i of table_rows is position pos[i])
    got = orope.rotate_table(bf16_bits_to_f32(fx["x"]), np.arange(n), fx["table_rows"])
    assert np.array_equal(got, fx["out"])
    # the table rows are the ones the reference's construction gives
    now = mg.rope_case()
    assert np.allclose(now["table_rows"], fx["table_rows"], rtol=0, atol=2e-7)
    # torch's f32 expression on the same rows (the reference's own ops)
    x = torch.from_numpy(bf16_bits_to_f32(fx["x"]))
    cs = torch.from_numpy(fx["table_rows"])[:, None, :]
    x1, x2 = torch.chunk(x, 2, dim=-1)
    y = torch.cat((x1 * cs[..., :64] - x2 * cs[..., 64:], x2 * cs[..., :64] + x1 * cs[..., 64:]), -1)
    assert np.array_equal(y.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16), fx["out"])


def test_sampler_fixture():
    import torch

    from oracle import sampler as osm

    fx = np.load(os.path.join(HERE, "sampler_cases.npz"))
    x0, p = osm.softmax_max(fx["logits"])
    assert np.array_equal(x0, fx["x0"]) and np.array_equal(p, fx["x0_p"])
    t = torch.from_numpy(fx["logits"].view(np.int16)).view(torch.bfloat16)
    tp, ti = torch.max(torch.softmax(t, dim=-1), dim=-1)       # the reference's ops on the CPU
    assert np.array_equal(ti.numpy(), fx["x0"])
    assert np.all(np.abs(tp.view(torch.int16).numpy().view(np.uint16).astype(int) - fx["x0_p"].astype(int)) <= 1)
    assert fx["x0"][35] == 3 and fx["x0"][36] == 40 and fx["x0"][37] == 0 and fx["x0"][39] == 4095
    out, nun = osm.unmask_step(fx["tokens"], fx["params"], fx["pred"], fx["conf"], int(fx["mask_id"]))
    assert np.array_equal(out, fx["tokens_out"]) and np.array_equal(nun, fx["n_unmasked"])
