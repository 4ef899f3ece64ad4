"""Oracle pins: bf16 rounding, KV store/load, RoPE (CPU only)."""
import numpy as np
import torch

from oracle import bf16 as ob
from oracle import configs
from oracle import kvcache as okv
from oracle import rope as orope


def test_bf16_rounding_matches_torch():
    """f32 -> bf16 round-to-nearest-even equals torch's CPU conversion,
    including exact ties, signed zeros, infinities and subnormals."""
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2**32, size=200_000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[np.isfinite(x)]
    ties = np.array([1.00390625, 1.01171875, -1.00390625, 3.0e-39, -0.0, 0.0, np.inf, -np.inf], dtype=np.float32)
    x = np.concatenate([x, ties])
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ob.f32_to_bf16_bits(x), ref)
    assert ob.f32_to_bf16_bits(np.array([np.nan], np.float32))[0] == 0x7FC0
    back = ob.bf16_bits_to_f32(ref)
    assert np.array_equal(back, torch.from_numpy(x).to(torch.bfloat16).float().numpy())


def test_f64_two_step_rounding():
    """The documented two-step rule f64 -> f32 -> bf16 (the GPU converts the
    same way) on values where one step and two steps can differ."""
    vals = np.array([1 + 2**-8 + 2**-30, 1 + 2**-8 - 2**-30, -(1 + 2**-8), 0.1], dtype=np.float64)
    got = ob.f64_to_bf16_bits(vals)
    want = ob.f32_to_bf16_bits(vals.astype(np.float32))
    assert np.array_equal(got, want)
    # 1 + 2^-8 + 2^-30 is exactly representable? no: f32 rounds it to the tie 1 + 2^-8, which rounds to even (1.0)
    assert got[0] == 0x3F80 and got[1] == 0x3F80


def test_store_load_bruteforce_and_roundtrip():
    rng = np.random.default_rng(1)
    n, row, slots_n = 37, 24, 64
    key = rng.standard_normal((n, row)).astype(np.float32)
    val = rng.standard_normal((n, row)).astype(np.float32)
    slots = rng.permutation(slots_n)[:n]
    slots[5] = -1          # skipped
    slots[9] = slots_n     # skipped (== capacity)
    kc = np.full((slots_n, row), 7.0, np.float32)
    vc = np.full((slots_n, row), 7.0, np.float32)
    okv.store(key, val, kc, vc, slots)
    kref = np.full((slots_n, row), 7.0, np.float32)
    for i in range(n):
        if 0 <= slots[i] < slots_n:
            kref[slots[i]] = key[i]
    assert np.array_equal(kc, kref)
    untouched = np.setdiff1d(np.arange(slots_n), slots[(slots >= 0) & (slots < slots_n)])
    assert np.all(kc[untouched] == 7.0) and np.all(vc[untouched] == 7.0)
    k2 = np.zeros_like(key)
    v2 = np.zeros_like(val)
    okv.load(k2, v2, kc, vc, slots)
    ok = (slots >= 0) & (slots < slots_n)
    assert np.array_equal(k2[ok], key[ok]) and np.array_equal(v2[ok], val[ok])
    assert np.all(k2[~ok] == 0)


def test_rope_invariants_and_torch_agreement():
    rng = np.random.default_rng(2)
    N, H, D = 64, 3, 128
    x = rng.standard_normal((N, H, D)).astype(np.float32)
    pos = np.arange(N)
    y = orope.apply(x, pos, 500000.0)
    # position 0 is the identity
    assert np.allclose(y[0], x[0], atol=0)
    # each (i, i + D/2) pair is rotated: its norm is preserved
    nx = x[..., :D // 2] ** 2 + x[..., D // 2:] ** 2
    ny = y[..., :D // 2] ** 2 + y[..., D // 2:] ** 2
    assert np.allclose(nx, ny, rtol=1e-5, atol=1e-5)
    # relative position: <R(p)q, R(p')k> depends on p - p' only
    q = rng.standard_normal((1, 1, D)).astype(np.float32)
    k = rng.standard_normal((1, 1, D)).astype(np.float32)
    def dot(p, pp):
        return float((orope.apply(q, [p], 1e4) * orope.apply(k, [pp], 1e4)).sum())
    assert abs(dot(5, 2) - dot(103, 100)) < 1e-3 and abs(dot(0, 7) - dot(50, 57)) < 1e-3
    # torch formulation used for the benchmark inputs agrees
    yt = configs.rope_torch(torch.from_numpy(x), torch.from_numpy(pos), 500000.0).numpy()
    assert np.abs(yt - y).max() < 1e-4


def _bf16_values(rng, shape):
    from oracle.bf16 import round_bf16
    return round_bf16(rng.standard_normal(shape).astype(np.float32))


def test_rope_table_turns_are_exact():
    """Quarter turn (cos 0, sin 1) swaps the halves with a sign, half turn
    negates, cos 1 / sin 0 is the identity -- exactly, so a transposed half, a
    wrong sign or an interleaved (GPT-J) pairing fails."""
    from oracle.bf16 import f32_to_bf16_bits
    rng = np.random.default_rng(3)
    N, H, D = 6, 2, 64
    h = D // 2
    x = _bf16_values(rng, (N, H, D))
    table = np.zeros((3, D), np.float32)
    table[0, :h] = 1.0                      # identity
    table[1, h:] = 1.0                      # quarter turn
    table[2, :h] = -1.0                     # half turn
    pos = np.array([0, 1, 2, 1, 0, 2])
    y = orope.rotate_table(x, pos, table)
    for i, p in enumerate(pos):
        if p == 0:
            want = x[i]
        elif p == 1:
            want = np.concatenate([-x[i, :, h:], x[i, :, :h]], axis=-1)
        else:
            want = -x[i]
        assert np.array_equal(y[i], f32_to_bf16_bits(want)), (i, p)


def test_rope_table_matches_apply_and_torch_ops():
    """With the f32 table of the module construction the table rotation equals
    orope.apply rounded to bf16, and torch's f32 ops evaluated one by one."""
    from oracle.bf16 import f32_to_bf16_bits
    rng = np.random.default_rng(4)
    N, H, D = 40, 3, 128
    x = _bf16_values(rng, (N, H, D))
    pos = rng.integers(0, 4096, N)
    c, s = orope.cos_sin(np.arange(4096), D, 500000.0)
    table = np.concatenate([c, s], axis=-1)
    y = orope.rotate_table(x, pos, table)
    assert np.array_equal(y, f32_to_bf16_bits(orope.apply(x, pos, 500000.0)))
    xt = torch.from_numpy(x)
    tt = torch.from_numpy(table)[torch.from_numpy(pos)]
    ct, st = tt[:, None, :D // 2], tt[:, None, D // 2:]
    x1, x2 = xt[..., :D // 2], xt[..., D // 2:]
    yt = torch.cat((x1 * ct - x2 * st, x2 * ct + x1 * st), dim=-1).to(torch.bfloat16)
    assert np.array_equal(y, yt.view(torch.int16).numpy().view(np.uint16))
