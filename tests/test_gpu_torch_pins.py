"""Rounding steps of the reference that torch itself executes, pinned against
torch on the MI355X.

- Scores / sqrt(D): the reference divides a bf16 score tensor by the Python
  float D ** 0.5 (dllmserve/layers/attention.py:376,381-383).  On the GPU,
  torch evaluates a tensor divided by a host scalar as a multiply by the f32
  reciprocal, not as an IEEE division.  oracle.select.scale_scores (and the
  selection kernels) use the f32 division bf16(f32(x) / f32(sqrt D)); over
  every one of the 65536 bf16 patterns the two must give the same bf16 bits.
- RoPE: the reference's RotaryEmbedding.forward runs under @torch.compile
  (dllmserve/layers/rotary_embedding.py:40-57).  K7 rounds the f32
  expression x1*cos - x2*sin / x2*cos + x1*sin op by op (no fused
  multiply-add), which is bit-exact against eager torch; the compiled form
  contracts multiply-adds into fused ones.  Here the expression is compiled
  by torch (inductor) on the box and compared with K7: every element within
  what a contraction can move (2^-22 of the products' magnitude, plus one
  bf16 unit of the result), and the count of differing elements printed."""
import numpy as np
import pytest
import torch

from oracle import select as osel
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits
from dllm_serve_amd.layers.rotary_embedding import RotaryEmbedding

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("D", [128, 64])
def test_score_scaling_matches_torch_gpu_division(dev, D):
    print(f"torch pin: bf16 tensor / {D} ** 0.5 on the GPU, all 65536 patterns", flush=True)
    pat = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    x = torch.from_numpy(pat.view(np.int16)).view(torch.bfloat16).to(dev)
    y = (x / (D ** 0.5)).cpu().view(torch.int16).numpy().view(np.uint16)
    want = f32_to_bf16_bits(osel.scale_scores(bf16_bits_to_f32(pat), np.float32(D ** 0.5)).astype(np.float32))
    xf = bf16_bits_to_f32(pat)
    nan_in = np.isnan(xf)
    assert np.isnan(bf16_bits_to_f32(y))[nan_in].all()
    diff = np.flatnonzero((y != want) & ~nan_in)
    assert diff.size == 0, f"{diff.size} patterns differ, first {pat[diff[:8]]}"


def _rope_expr(positions, query, key, table, head_size):
    """The reference's forward expression (rotary_embedding.py:6-17,41-57)."""
    n = positions.size(0)
    cos, sin = table[positions].chunk(2, dim=-1)
    cos, sin = cos.unsqueeze(-2), sin.unsqueeze(-2)
    out = []
    for x in (query, key):
        shape = x.shape
        x = x.view(n, -1, head_size)
        x1, x2 = torch.chunk(x.to(torch.float32), 2, dim=-1)
        y = torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), dim=-1).to(x.dtype)
        out.append(y.view(shape))
    return out[0], out[1]


@pytest.mark.parametrize("Hq,Hkv,theta", [(32, 32, 500000.0), (28, 4, 1e6)])
def test_rope_against_torch_compile(dev, Hq, Hkv, theta):
    print(f"torch pin: RoPE under torch.compile vs K7, {Hq}/{Hkv} heads", flush=True)
    D, n = 128, 512
    rope = RotaryEmbedding(D, D, 4096, theta).to(dev)
    g = torch.Generator(device=dev).manual_seed(3)
    q = (torch.randn(n, Hq * D, generator=g, device=dev) * 3).to(torch.bfloat16)
    k = (torch.randn(n, Hkv * D, generator=g, device=dev) * 3).to(torch.bfloat16)
    pos = torch.randint(0, 4096, (n,), generator=g, device=dev)
    try:
        compiled = torch.compile(_rope_expr, dynamic=False)
        qc, kc = compiled(pos, q, k, rope.cos_sin_cache, D)
        torch.cuda.synchronize()
    except Exception as e:  # inductor / its kernel compiler unavailable on this box
        pytest.skip(f"torch.compile unavailable: {type(e).__name__}: {e}")
    qe, ke = _rope_expr(pos, q, k, rope.cos_sin_cache, D)
    q7, k7 = rope(pos, q, k)
    torch.cuda.synchronize()
    cos, sin = rope.cos_sin_cache[pos].double().chunk(2, dim=-1)
    cos, sin = cos.unsqueeze(-2), sin.unsqueeze(-2)
    for name, x, c, e, ours in (("q", q, qc, qe, q7), ("k", k, kc, ke, k7)):
        assert torch.equal(ours.view(torch.int16), e.view(torch.int16)), f"K7 {name} differs from eager torch"
        x1, x2 = x.view(n, -1, D).double().chunk(2, dim=-1)
        # magnitude of the two products of each output: a fused multiply-add
        # moves the f32 result by at most 2^-23 of it (plus the f32 rounding
        # the eager form makes), before the bf16 rounding
        mag = torch.cat(((x1 * cos).abs() + (x2 * sin).abs(), (x2 * cos).abs() + (x1 * sin).abs()), dim=-1)
        cv, ov = c.view(n, -1, D).double(), ours.view(n, -1, D).double()
        big = torch.maximum(cv.abs(), ov.abs())
        ulp = torch.where(big > 0, torch.exp2(torch.floor(torch.log2(big.clamp_min(1e-300))) - 7), torch.zeros_like(big))
        diff = (cv - ov).abs()
        ndiff = int((diff > 0).sum())
        print(f"  {name}: {ndiff} of {diff.numel()} elements differ from the compiled expression", flush=True)
        assert bool((diff <= mag * 2.0 ** -22 + ulp).all()), f"{name}: compiled RoPE beyond the contraction bound"
