"""Oracle pins for the low-confidence remasking sampler (CPU only).

softmax_max is checked against torch's own CPU softmax + max on the same
bf16 rows (the library routines the reference calls), against closed forms
(uniform rows, one dominant logit, planted exact ties) and on a planted
rounding tie, where a lower-index logit below the maximum rounds to the same
bf16 probability and torch.max returns it.  unmask_step is checked against
torch.topk on tie-free confidences and against counting invariants, the
steps_remain rule and the first-token rule."""
import math

import numpy as np
import pytest
import torch

from oracle import sampler as osm
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits

MASK = 126336


def _bits(x):
    return f32_to_bf16_bits(np.asarray(x, np.float32))


def _torch_softmax_max(bits):
    t = torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16)
    p, i = torch.max(torch.softmax(t, dim=-1), dim=-1)
    return i.numpy(), p.view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("M,V,sigma", [(16, 126464, 1.3), (8, 4096, 3.0), (32, 1000, 0.4)])
def test_softmax_max_matches_torch_cpu(M, V, sigma):
    rng = np.random.default_rng(M + V)
    bits = _bits(rng.standard_normal((M, V)) * sigma)
    x0, p = osm.softmax_max(bits)
    tx0, tp = _torch_softmax_max(bits)
    assert np.array_equal(x0, tx0)
    # summation order may move bf16(1/s) by one unit in rare rows
    assert np.all(np.abs(p.astype(np.int32) - tp.astype(np.int32)) <= 1)
    assert np.mean(p == tp) >= 0.9


def test_softmax_max_closed_forms():
    V = 4096
    # uniform row: every probability is bf16(1/V), the first index wins
    x0, p = osm.softmax_max(_bits(np.full((1, V), 0.75)))
    assert x0[0] == 0 and p[0] == _bits(1.0 / V)
    # one dominant logit L at j, zeros elsewhere: s = 1 + (V-1) e^-L
    L, j = 6.0, 1234
    row = np.zeros(V, np.float32)
    row[j] = L
    x0, p = osm.softmax_max(_bits(row[None]))
    assert x0[0] == j
    assert abs(int(p[0]) - int(_bits([1.0 / (1.0 + (V - 1) * math.exp(-L))])[0])) <= 1
    # exact ties of the maximal logit: the first one wins
    row = np.random.default_rng(1).standard_normal(V).astype(np.float32)
    row[[77, 500, 3000]] = 5.0
    x0, _ = osm.softmax_max(_bits(row[None]))
    assert x0[0] == 77


def test_softmax_max_rounding_tie_takes_lower_index():
    """logit 1 - 2^-8 at index 3 and 1.0 at index 10: with this filler both
    probabilities round to the same bf16 (0.18 % inside the bucket), so the
    result is index 3 although index 10 holds the larger logit."""
    V = 4096
    row = np.full(V, 0.28125, np.float32)
    row[3], row[10] = 1.0 - 2 ** -8, 1.0
    bits = _bits(row[None])
    x0, p = osm.softmax_max(bits)
    tx0, tp = _torch_softmax_max(bits)
    assert x0[0] == 3 and tx0[0] == 3 and p[0] == tp[0]


def _params_case(rng, n_seq, max_win, first_frac=0.5):
    tokens, params, rows = [], [], 0
    for b in range(n_seq):
        n = int(rng.integers(0, max_win + 1))
        pad = int(rng.integers(0, 5))
        tok = rng.integers(0, 1000, n + pad)
        tok[pad:][rng.random(n) < rng.random()] = MASK
        params.append((len(tokens) + pad, n, rows, int(rng.integers(-1, 6)), int(rng.random() < first_frac)))
        tokens.extend(tok.tolist())
        rows += n
    return np.array(tokens, np.int64), params, rows


def test_unmask_matches_torch_topk_on_distinct_confidences():
    rng = np.random.default_rng(5)
    tokens, params, rows = _params_case(rng, 40, 300)
    # confidences distinct within each window: distinct bf16 patterns of (0, 1)
    conf = np.zeros(rows, np.uint16)
    for off, n, r0, sr, first in params:
        conf[r0:r0 + n] = rng.choice(np.arange(0x3000, 0x3F80, dtype=np.uint16), size=n, replace=False)
    x0 = rng.integers(1000, 2000, rows)
    out, nun = osm.unmask_step(tokens, params, x0, conf, MASK)
    for b, (off, n, r0, sr, first) in enumerate(params):
        tok = torch.from_numpy(tokens[off:off + n].copy())
        c = torch.from_numpy(bf16_bits_to_f32(conf[r0:r0 + n]))
        pred = torch.from_numpy(x0[r0:r0 + n])
        mask = tok == MASK
        conf_t = torch.where(mask, c, torch.tensor(-np.inf))
        nmask = int(mask.sum())
        k = min(math.ceil(nmask / sr), nmask) if sr > 0 else 0
        assert nun[b] == k
        if first and n > 0 and k > 0 and bool(mask[0]):
            tok[0] = pred[0]
            if k > 1:
                rem = conf_t.clone()
                rem[0] = -np.inf
                top = torch.topk(rem, k=min(k - 1, nmask - 1)).indices
                tok[top] = pred[top]
        elif k > 0:
            top = torch.topk(conf_t, k=k).indices
            tok[top] = pred[top]
        assert np.array_equal(out[off:off + n], tok.numpy()), f"sequence {b}"
    # positions outside every window are untouched
    inside = np.zeros(len(tokens), bool)
    for off, n, *_ in params:
        inside[off:off + n] = True
    assert np.array_equal(out[~inside], tokens[~inside])


def test_unmask_invariants_with_ties():
    rng = np.random.default_rng(9)
    n = 512
    tokens = np.where(rng.random(n) < 0.7, MASK, rng.integers(0, 1000, n))
    conf = _bits(np.round(rng.random(n) * 8) / 8)   # heavy ties
    x0 = rng.integers(1000, 2000, n)
    for sr in (1, 2, 3, 7, 1000):
        out, nun = osm.unmask_step(tokens, [(0, n, 0, sr, 0)], x0, conf, MASK)
        masked = tokens == MASK
        changed = out != tokens
        nmask = int(masked.sum())
        k = min(-(-nmask // sr), nmask)
        assert nun[0] == k and changed.sum() == k
        assert np.all(masked[changed]) and np.array_equal(out[changed], x0[changed])
        cv = bf16_bits_to_f32(conf)
        still = masked & ~changed
        if still.any() and changed.any():
            lo_sel = cv[changed].min()
            assert lo_sel >= cv[still].max()
            # among equal confidences at the threshold, lower positions go first
            at = np.nonzero(np.isclose(cv, lo_sel) & masked)[0]
            sel_at = at[changed[at]]
            assert np.array_equal(sel_at, at[:len(sel_at)])
    # steps_remain == 1 unmasks every masked position
    out, _ = osm.unmask_step(tokens, [(0, n, 0, 1, 0)], x0, conf, MASK)
    assert not np.any(out == MASK)


def test_unmask_first_token_rule():
    n = 8
    tokens = np.array([MASK] * n, np.int64)
    conf = _bits(np.linspace(0.1, 0.9, n))          # position 0 has the lowest confidence
    x0 = np.arange(100, 100 + n)
    out, nun = osm.unmask_step(tokens, [(0, n, 0, 4, 1)], x0, conf, MASK)  # k = 2
    assert nun[0] == 2 and out[0] == 100 and out[7] == 107
    assert np.sum(out != MASK) == 2
    out, _ = osm.unmask_step(tokens, [(0, n, 0, 4, 0)], x0, conf, MASK)    # rule off
    assert out[0] == MASK and out[6] == 106 and out[7] == 107
    t2 = tokens.copy()
    t2[0] = 5                                        # first position already known
    out, nun = osm.unmask_step(t2, [(0, n, 0, 4, 1)], x0, conf, MASK)      # nmask 7, k = 2
    assert nun[0] == 2 and out[0] == 5 and out[6] == 106 and out[7] == 107


def test_splitmix64_known_answers():
    # first outputs of SplitMix64 seeded with 0 (the published reference sequence)
    got = [int(x) for x in osm.splitmix64_at(0, np.arange(3, dtype=np.uint64))]
    assert got == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]
    u = osm.uniforms(1234, 5, 100000)
    assert u.min() >= 0.0 and u.max() < 1.0 and abs(u.mean() - 0.5) < 0.005
    # a row's draws depend on its global index only
    assert np.array_equal(osm.uniforms(7, 3, 64), osm.uniforms(7, 3, 64))
    assert not np.array_equal(osm.uniforms(7, 3, 64), osm.uniforms(7, 4, 64))


@pytest.mark.parametrize("T", [1.0, 0.5, 2.0])
def test_gumbel_transform_matches_the_reference_ops(T):
    """add_gumbel_noise's torch ops (model_runner.py:592-600) on the same draws,
    stored back into a bf16 tensor as the reference's slice assignment does."""
    rng = np.random.default_rng(int(T * 10))
    V = 4096
    bits = _bits(rng.standard_normal(V) * 3)
    u = osm.uniforms(99, 2, V)
    got = osm.gumbel_transform(bits, T, u)
    lg = torch.from_numpy(bf16_bits_to_f32(bits)).to(torch.float64)
    noise = torch.from_numpy(u)
    want = lg.exp() / (-torch.log(noise)) ** T
    dst = torch.empty(V, dtype=torch.bfloat16)
    dst[:] = want
    assert np.array_equal(got, dst.view(torch.int16).numpy().view(np.uint16))


def test_gumbel_sampling_follows_softmax():
    """Gumbel-max: at T = 1 the sampled index is distributed as softmax(l)."""
    V, n = 8, 40000
    l = np.log(np.array([1, 2, 3, 4, 6, 8, 12, 16], np.float64))
    bits = np.tile(_bits(l.astype(np.float32)), (n, 1))
    x0, p = osm.softmax_max_sample(bits, np.ones(n), seed=2024)
    freq = np.bincount(x0, minlength=V) / n
    want = np.exp(bf16_bits_to_f32(bits[0]).astype(np.float64))
    want /= want.sum()
    assert np.abs(freq - want).max() < 0.01, (freq, want)
    # temperature 0 rows are plain softmax-max
    x0b, pb = osm.softmax_max_sample(bits[:4], np.zeros(4), seed=1)
    xa, pa = osm.softmax_max(bits[:4])
    assert np.array_equal(x0b, xa) and np.array_equal(pb, pa)
