"""Low-confidence remasking sampler (the step after the model's forward).

TEST INFRASTRUCTURE ONLY: expected results for the K8 / K9 kernels.

Restates dllmserve/engine/model_runner.py:756-949
(_reconstruct_and_sample_optimized_v2, temperature 0):
  softmax_max   probs = F.softmax(bf16 logits, -1) (f32 inside, bf16 out);
                x0_p, x0 = torch.max(probs, -1)                     (:862-863, :886-887)
  softmax_max_sample  the same after add_gumbel_noise (:592-600) on rows of
                temperature > 0, with the counter-based SplitMix64 draws the
                K8 kernel uses
  unmask_step   per sequence: mask test over the window, steps_remain,
                num_to_unmask = min(ceil(nmask / steps_remain), nmask), the
                is_full_attention first-token rule, torch.topk over the
                confidences and the token write-back                (:895-949)
Parity pins: tests/test_oracle_sampler.py (torch CPU softmax + max on the
same bf16 rows, closed forms, planted exact and rounding ties; torch.topk on
tie-free confidences, counting invariants, the first-token rule).
"""
from __future__ import annotations

import numpy as np

from .bf16 import bf16_bits_to_f32, f32_to_bf16_bits, f64_to_bf16_bits

GAMMA = 0x9E3779B97F4A7C15


def softmax_max(logit_bits: np.ndarray, s_scale: float = 1.0) -> tuple[np.ndarray, np.ndarray]:
    """Rows of bf16 logits (uint16 bits, [M, V]) -> (x0 int64 [M], x0_p bf16 bits [M]).

    In f32: m = max l, e = exp(l - m), s = sum e, P = bf16(e / s); x0_p is
    max P and x0 the first index attaining it (torch.max's documented rule).
    s_scale multiplies s: tests use it to find the rows whose result does not
    depend on the summation order of s."""
    l = bf16_bits_to_f32(np.asarray(logit_bits, dtype=np.uint16)).astype(np.float32)
    l = l.reshape(-1, l.shape[-1])
    m = l.max(axis=1, keepdims=True)
    e = np.exp(l - m, dtype=np.float32)
    s = e.sum(axis=1, dtype=np.float32, keepdims=True) * np.float32(s_scale)
    p = f32_to_bf16_bits(e / s)
    pv = bf16_bits_to_f32(p)
    x0 = pv.argmax(axis=1).astype(np.int64)  # first maximal index
    return x0, p[np.arange(p.shape[0]), x0]


def splitmix64_at(seed: int, c: np.ndarray) -> np.ndarray:
    """SplitMix64 output for counters c (Steele, Lea & Flood 2014): mix of
    seed + (c + 1) * golden gamma, with wrap-around uint64 arithmetic."""
    c = np.asarray(c, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + (c + np.uint64(1)) * np.uint64(GAMMA)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def uniforms(seed: int, row: int, V: int) -> np.ndarray:
    """The f64 draws u_j in [0, 1) of logits row `row` (global index)."""
    c = np.uint64(row) * np.uint64(V) + np.arange(V, dtype=np.uint64)
    return (splitmix64_at(seed, c) >> np.uint64(11)).astype(np.float64) * 2.0 ** -53


def gumbel_transform(logit_bits: np.ndarray, T: float, u: np.ndarray) -> np.ndarray:
    """add_gumbel_noise (model_runner.py:592-600) on one bf16 row, stored
    back as bf16 (f64 -> f32 -> bf16, the conversion of the bf16 assignment
    at :833-835 / :864-866)."""
    l = bf16_bits_to_f32(np.asarray(logit_bits, dtype=np.uint16)).astype(np.float64)
    with np.errstate(divide="ignore"):
        nl = -np.log(u)
    g = nl if T == 1.0 else np.power(nl, T)
    with np.errstate(divide="ignore", invalid="ignore"):
        v = np.exp(l) / g
    return f64_to_bf16_bits(v)


def softmax_max_sample(logit_bits: np.ndarray, row_temperature, seed: int, row_base: int = 0):
    """softmax_max after the Gumbel transform of every row whose temperature
    is > 0 (draws from `uniforms(seed, row_base + r, V)`)."""
    b = np.array(logit_bits, dtype=np.uint16, copy=True).reshape(-1, np.asarray(logit_bits).shape[-1])
    V = b.shape[1]
    for r, T in enumerate(np.asarray(row_temperature, dtype=np.float64)):
        if T > 0:
            b[r] = gumbel_transform(b[r], float(T), uniforms(seed, row_base + r, V))
    return softmax_max(b)


def conf_order(bits: np.ndarray) -> np.ndarray:
    """bf16 bits -> uint32 keys ordered like the values (-0 == +0)."""
    b = np.asarray(bits, dtype=np.uint32) & 0xFFFF
    b = np.where(b == 0x8000, 0, b)
    return np.where(b & 0x8000, (~b) & 0xFFFF, b | 0x8000).astype(np.uint32)


def unmask_step(tokens: np.ndarray, params, x0: np.ndarray, conf_bits: np.ndarray, mask_id: int):
    """One denoising step of every sequence.

    tokens: flat int64 array, updated in a copy that is returned.
    params: rows (tok_off, win_len, row_off, steps_remain, first_rule).
    x0 / conf_bits: the per-row predictions and bf16 confidences.
    Returns (tokens, n_unmasked per sequence)."""
    out = np.array(tokens, dtype=np.int64, copy=True)
    n_unmasked = []
    for tok_off, n, r0, sr, first in params:
        tok_off, n, r0, sr, first = int(tok_off), int(n), int(r0), int(sr), bool(first)
        win = out[tok_off:tok_off + n]                # a view: writes land in `out`
        masked = win == mask_id
        nmask = int(masked.sum())
        # math.ceil(float(nmask) / steps_remain), min with nmask (:916-917)
        k = min(-(-nmask // sr), nmask) if sr > 0 else 0
        n_unmasked.append(k)
        if n == 0 or k == 0:
            continue
        pred = x0[r0:r0 + n]
        cand = masked.copy()
        if first and masked[0]:                       # :920-935
            win[0] = pred[0]
            cand[0] = False
            k -= 1
        if k > 0:
            key = conf_order(conf_bits[r0:r0 + n])
            j = np.nonzero(cand)[0]
            # highest confidence first, ties to the lower position
            order = j[np.lexsort((j, -key[j].astype(np.int64)))]
            sel = order[:k]
            win[sel] = pred[sel]
    return out, np.array(n_unmasked, dtype=np.int32)
