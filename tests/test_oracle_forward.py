"""Pins oracle.paged_ref.attention_forward (reference needle/layers/attention.py:83-96).

With projection weights that are selection matrices (W[i, sel[i]] = 1, so F.linear(x, W)
is x[:, sel] exactly in bf16) and a bias, the forward must reduce exactly to: the selected
columns plus the bias as q, k and v, the rotary embedding, the prefill or decode seam, and
the output's columns selected by o_proj.  Each selection is a different, non-involutive
one, so swapped projections (k for v), a transposed weight, a dropped bias, a missing RoPE
or a skipped o_proj all fail; the seams and apply_rope are pinned on their own in the other
oracle tests.
"""
import torch

from oracle import paged_ref

H, HKV, D = 4, 2, 16
HIDDEN = H * D


def _selection(sel, n_in):
    w = torch.zeros((len(sel), n_in), dtype=torch.bfloat16)
    w[torch.arange(len(sel)), torch.tensor(sel)] = 1
    return w


def _setup(seed, t):
    g = torch.Generator().manual_seed(seed)
    perm = lambda n: torch.randperm(n, generator=g).tolist()       # noqa: E731
    sel = {"q": perm(HIDDEN), "k": perm(HIDDEN)[:HKV * D], "v": perm(HIDDEN)[:HKV * D],
           "o": perm(H * D)}
    weights = {f"{n}_proj.weight": _selection(sel[n], HIDDEN if n != "o" else H * D)
               for n in "qkvo"}
    for n, width in (("q", H * D), ("k", HKV * D), ("v", HKV * D)):
        weights[f"{n}_proj.bias"] = (torch.randn(width, generator=g) * 0.5).to(torch.bfloat16)
    x = torch.randn((t, HIDDEN), generator=g).to(torch.bfloat16)
    ang = torch.rand((t, D // 2), generator=g) * 6.28
    cos = torch.cat([ang.cos(), ang.cos()], -1).to(torch.bfloat16)
    sin = torch.cat([ang.sin(), ang.sin()], -1).to(torch.bfloat16)
    return sel, weights, x, cos, sin


def _expected(sel, weights, x, cos, sin, seam):
    t = x.shape[0]
    q = (x[:, sel["q"]] + weights["q_proj.bias"]).view(t, H, D)
    k = (x[:, sel["k"]] + weights["k_proj.bias"]).view(t, HKV, D)
    v = (x[:, sel["v"]] + weights["v_proj.bias"]).view(t, HKV, D)
    q, k = paged_ref.apply_rope(q, k, cos, sin)
    return seam(q, k, v).reshape(t, H * D)[:, sel["o"]]


def test_selection_projections_reduce_to_rope_and_the_prefill_seam():
    sel, weights, x, cos, sin = _setup(0, 40)
    cu = torch.tensor([0, 7, 25, 40], dtype=torch.int32)
    ctx = torch.zeros(3, dtype=torch.int32)
    table = torch.tensor([[5, 0], [1, 2], [3, 4]], dtype=torch.int32)
    pool_a = torch.randn((2, 6, HKV, 16, D)).to(torch.bfloat16)
    pool_b = pool_a.clone()
    got = paged_ref.attention_forward(weights, x, pool_a, table, cu, ctx, True, cos, sin,
                                      H, HKV, D)
    want = _expected(sel, weights, x, cos, sin, lambda q, k, v: paged_ref.prefill(
        q, k, v, pool_b, table, cu, ctx, H, HKV))
    assert torch.equal(got, want)
    assert torch.equal(pool_a.view(torch.int16), pool_b.view(torch.int16))


def test_selection_projections_reduce_to_rope_and_the_decode_seam():
    sel, weights, x, cos, sin = _setup(1, 3)
    ctx = torch.tensor([4, 20, 0], dtype=torch.int32)
    table = torch.tensor([[2, 5], [0, 1], [3, 5]], dtype=torch.int32)
    pool_a = torch.randn((2, 6, HKV, 16, D)).to(torch.bfloat16)
    pool_b = pool_a.clone()
    got = paged_ref.attention_forward(weights, x, pool_a, table, None, ctx, False, cos, sin,
                                      H, HKV, D)
    want = _expected(sel, weights, x, cos, sin, lambda q, k, v: paged_ref.decode(
        q, k, v, pool_b, table, ctx, 1.0 / D ** 0.5, H, HKV, D))
    assert torch.equal(got, want)
    assert torch.equal(pool_a.view(torch.int16), pool_b.view(torch.int16))


def test_a_planted_slip_is_caught():
    """The same check fails when the forward is given k's weights for v (a swapped
    projection) or loses a bias: the pin is not vacuous."""
    sel, weights, x, cos, sin = _setup(2, 3)
    ctx = torch.tensor([4, 20, 9], dtype=torch.int32)
    table = torch.tensor([[2, 5], [0, 1], [3, 4]], dtype=torch.int32)
    pool = torch.randn((2, 6, HKV, 16, D)).to(torch.bfloat16)

    def run(w):
        return paged_ref.attention_forward(w, x, pool.clone(), table, None, ctx, False, cos,
                                           sin, H, HKV, D)
    want = _expected(sel, weights, x, cos, sin, lambda q, k, v: paged_ref.decode(
        q, k, v, pool.clone(), table, ctx, 1.0 / D ** 0.5, H, HKV, D))
    assert torch.equal(run(weights), want)
    swapped = dict(weights, **{"v_proj.weight": weights["k_proj.weight"],
                               "v_proj.bias": weights["k_proj.bias"]})
    assert not torch.equal(run(swapped), want)
    no_bias = {k: v for k, v in weights.items() if k != "q_proj.bias"}
    assert not torch.equal(run(no_bias), want)
