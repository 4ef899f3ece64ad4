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
  rope_cases.npz    NeoX RoPE (theta 5e5, table of 4096 positions built as
                    the reference builds it): bf16 inputs, positions, the
                    table rows they use and the rotated bf16 outputs.
  sampler_cases.npz softmax-max of 40 logit rows of 4096 words (scales 0.3
                    to 4, planted exact and rounding ties) with x0 / x0_p,
                    and one unmasking step of 12 windows with its tokens,
                    parameters, confidences and results.
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import attention as oatt  # noqa: E402
from oracle import configs  # noqa: E402
from oracle import rope as orope  # noqa: E402
from oracle import sampler as osm  # noqa: E402
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


def rope_case():
    import torch

    rng = np.random.default_rng(7)
    D, n, H = 128, 64, 3
    inv = 1.0 / (500000.0 ** (torch.arange(0, D, 2, dtype=torch.float) / D))
    t = torch.arange(4096, dtype=torch.float)
    freqs = torch.einsum("i,j -> ij", t, inv)
    table = torch.cat((freqs.cos(), freqs.sin()), dim=-1).numpy()
    x = f32_to_bf16_bits(rng.standard_normal((n, H, D)).astype(np.float32) * 2)
    pos = rng.integers(0, 4096, n).astype(np.int64)
    out = orope.rotate_table(bf16_bits_to_f32(x), pos, table)
    return dict(x=x, pos=pos, table_rows=table[pos], max_position=np.int64(4096), out=out)


def sampler_case():
    rng = np.random.default_rng(11)
    V = 4096
    rows = []
    for sigma in (0.3, 0.7, 1.3, 2.0, 4.0):
        rows.append(rng.standard_normal((7, V)).astype(np.float32) * sigma)
    extra = np.full((5, V), 0.28125, np.float32)
    extra[0, 3], extra[0, 10] = 1.0 - 2 ** -8, 1.0             # rounding tie: index 3
    extra[1] = rng.standard_normal(V) * 1.5
    extra[1, [40, 4000, 1000]] = 7.0                            # exact ties: index 40
    extra[2] = 0.5                                              # uniform row: index 0
    extra[3] = rng.standard_normal(V)
    extra[3, ::2] = -np.inf
    extra[4] = rng.standard_normal(V)
    extra[4, V - 1] = 9.0
    logits = f32_to_bf16_bits(np.concatenate(rows + [extra]))
    x0, x0p = osm.softmax_max(logits)
    # one unmasking step of 12 windows
    mask = 126336
    tokens, params, r = [], [], 0
    for b in range(12):
        n = int(rng.integers(0, 40))
        tok = rng.integers(0, 1000, n + 2)
        tok[2:][rng.random(n) < 0.7] = mask
        params.append((len(tokens) + 2, n, r, int(rng.integers(1, 6)), int(b % 3 == 0)))
        tokens.extend(tok.tolist())
        r += n
    tokens = np.array(tokens, np.int64)
    conf = f32_to_bf16_bits(np.round(rng.random(r) * 16) / 16)
    pred = rng.integers(1000, 126000, r).astype(np.int64)
    out, nun = osm.unmask_step(tokens, params, pred, conf, mask)
    return dict(logits=logits, x0=x0, x0_p=x0p, tokens=tokens, params=np.array(params, np.int32), conf=conf,
                pred=pred, tokens_out=out, n_unmasked=nun, mask_id=np.int64(mask))


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
    np.savez_compressed(os.path.join(HERE, "rope_cases.npz"), **rope_case())
    np.savez_compressed(os.path.join(HERE, "sampler_cases.npz"), **sampler_case())
    print("wrote", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    main()
