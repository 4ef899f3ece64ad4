"""Writes the golden fixtures of the attention path (run from the repo root):

    python tests/golden/make_golden.py

The reference ships no numeric fixtures for this path and cannot be
imported here (its package needs flash_attn), so the fixtures are produced
by the oracle (oracle/) and serve as regression anchors for both the oracle
and the GPU kernels:

  c1_attention.npz  C1 configuration (one LLaDA-8B layer, 512 tokens, RoPE
                    theta 5e5, seed 0): input checksums, a strided sample of
                    the fp32 output and per-head output norms.
  select_cases.npz  three selection cases (head_select with MHA, head_select
                    with GQA group 4, token selection with GQA): bf16 inputs
                    as uint16 bit patterns and the selected indices.
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import attention as oatt  # noqa: E402
from oracle import configs  # noqa: E402
from oracle import select as osel  # noqa: E402
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
C1_STRIDE = 97
SELECT_CASES = [
    # name, Lb, Kc, Hq, Hkv, n_keep, head_select, pool_k, seed
    ("mha_hs", 16, 120, 4, 4, 60, True, 3, 101),
    ("gqa_hs", 8, 100, 8, 2, 33, True, 3, 102),
    ("gqa_tok", 8, 100, 4, 2, 25, False, 2, 103),
]


def c1():
    q, k, v, cu, scale = configs.c1_single_layer()
    qn, kn, vn = q.numpy(), k.numpy(), v.numpy()
    out = oatt.varlen(qn, kn, vn, cu.numpy(), cu.numpy(), scale, dtype=np.float32)
    sums = np.array([[t.astype(np.float64).sum(), (t.astype(np.float64) ** 2).sum()] for t in (qn, kn, vn)])
    return dict(input_sums=sums, out_sample=out.reshape(-1)[::C1_STRIDE].copy(),
                head_norms=np.linalg.norm(out.astype(np.float64), axis=(0, 2)), stride=np.int64(C1_STRIDE))


def select_case(Lb, Kc, Hq, Hkv, n_keep, head_select, pool_k, seed):
    rng = np.random.default_rng(seed)
    qb = f32_to_bf16_bits(rng.standard_normal((Lb, Hq, 128)).astype(np.float32))
    kb = f32_to_bf16_bits(rng.standard_normal((Kc, Hkv, 128)).astype(np.float32))
    idx = osel.select(bf16_bits_to_f32(qb), bf16_bits_to_f32(kb), n_keep, head_select, pool_k,
                      np.float32(128 ** 0.5))
    return qb, kb, idx


def main():
    np.savez_compressed(os.path.join(HERE, "c1_attention.npz"), **c1())
    arrs = {}
    for name, Lb, Kc, Hq, Hkv, n_keep, hs, pk, seed in SELECT_CASES:
        qb, kb, idx = select_case(Lb, Kc, Hq, Hkv, n_keep, hs, pk, seed)
        arrs[f"{name}_q"] = qb
        arrs[f"{name}_k"] = kb
        arrs[f"{name}_idx"] = idx
        arrs[f"{name}_params"] = np.array([Lb, Kc, Hq, Hkv, n_keep, int(hs), pk], dtype=np.int64)
    np.savez_compressed(os.path.join(HERE, "select_cases.npz"), **arrs)
    print("wrote", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    main()
