"""Pins the oracle's RoPE (attention.py:277-288) and the cos/sin tables (rope.py:10-27).

The reference ships no RoPE test, so the oracle is held to what the mathematics
fixes:
  - each pair (x[d], x[d + D/2]) is rotated as the complex product
    (x[d] + i x[d + D/2]) * (cos + i sin): checked against float64 to bf16
    accuracy, which fails on a swapped half, a wrong sign or a shifted index;
  - the rounding is torch's op-by-op bf16 (product, product, sum, each rounded
    to nearest-even): checked bit for bit against an explicit numpy rounding of
    each op, and shown to differ from a single rounding of the fp32 result
    on some elements, so the per-op rounding is really there;
  - cos_cached/sin_cached equal cos/sin(t * base^(-2i/D)) for both halves.
"""
import numpy as np
import torch

from oracle import paged_ref
from needle_amd.layers.rope import RotaryEmbedding


def _rne_bf16(x: np.ndarray) -> np.ndarray:
    """Round float32 -> bfloat16 (nearest-even) and back to float32, finite inputs."""
    b = x.astype(np.float32).view(np.uint32).astype(np.uint64)
    b = (b + 0x7FFF + ((b >> 16) & 1)) >> 16
    return (b.astype(np.uint32) << 16).view(np.float32)


def _case(t=37, h=3, d=64, seed=0, base=1e6):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn((t, h, d), generator=g) * 3).to(torch.bfloat16)
    rope = RotaryEmbedding(d, 4096, base).to(torch.bfloat16)
    pos = torch.randint(0, 4096, (t,), generator=g)
    cos, sin = rope.get_cos_sin(pos)
    return x, cos, sin


def test_rope_is_the_complex_rotation():
    for d in (64, 128):
        x, cos, sin = _case(d=d, seed=d)
        y, _ = paged_ref.apply_rope(x, x[:, :1], cos, sin)
        half = d // 2
        xc = x[..., :half].double() + 1j * x[..., half:].double()
        c = cos[:, None, :half].double()
        s = sin[:, None, :half].double()
        assert torch.equal(cos[:, :half], cos[:, half:]) and torch.equal(sin[:, :half], sin[:, half:])
        want = xc * (c + 1j * s)
        got = y[..., :half].double() + 1j * y[..., half:].double()
        err = (got - want).abs()
        # three bf16 roundings of values bounded by |x|: a few ulp of |x|
        bound = 3 * 2.0 ** -8 * (xc.abs() + 1e-30) + 1e-6
        assert bool((err <= bound).all()), float((err - bound).max())


def test_rope_rounds_each_op_in_bf16():
    x, cos, sin = _case(t=64, h=4, d=128, seed=5)
    y, _ = paged_ref.apply_rope(x, x[:, :1], cos, sin)
    xf = x.float().numpy()
    c = cos.float().numpy()[:, None, :]
    s = sin.float().numpy()[:, None, :]
    half = 128 // 2
    rot = np.concatenate([-xf[..., half:], xf[..., :half]], axis=-1)
    per_op = _rne_bf16(_rne_bf16(xf * c) + _rne_bf16(rot * s))
    assert np.array_equal(y.float().numpy().view(np.uint32), per_op.view(np.uint32))
    single = _rne_bf16(xf * c + rot * s)
    assert (single != per_op).sum() > 0


def test_cos_sin_tables_match_closed_form():
    d, base, n = 128, 500000.0, 8192
    rope = RotaryEmbedding(d, n, base)
    t = np.arange(n, dtype=np.float64)[:, None]
    inv = base ** (-np.arange(0, d, 2, dtype=np.float64) / d)
    ang = t * inv
    for table, fn in ((rope.cos_cached, np.cos), (rope.sin_cached, np.sin)):
        got = table.double().numpy()
        want = fn(ang)
        # fp32 angle t*inv_freq carries a relative error of ~1e-7 at t < 8192
        assert np.abs(got[:, : d // 2] - want).max() < 2e-3
        assert np.array_equal(got[:, : d // 2], got[:, d // 2:])
