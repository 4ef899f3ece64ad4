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
