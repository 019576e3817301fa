"""GPU parity of ndl_rope_paged_decode_append: RoPE, append and decode attention in one launch.

Attention.forward's decode step from RoPE on (attention.py:88, then _decode :141-159).  The
one launch must return the same output bits and leave the same pool bits as
ndl_rope_kv_append (decode form) followed by ndl_paged_decode on the rotated q, for every
split, and match the oracle (the reference's torch RoPE, append and _decode_pytorch):
pool bytes exact, output within |gpu - ref| <= 2e-2 + 1e-2 |ref|.  cos/sin come from the
model's rotary table at each sequence's position (rope_theta 1e6 and 1e4) and, to exercise
the general formula, from random values.
"""
import numpy as np
import pytest
import torch

from oracle import paged_ref
from needle_amd import ops, workloads as wl
from needle_amd.layers.rope import RotaryEmbedding

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _bits(t):
    return t.view(torch.int16)


def _cos_sin(case, base):
    if base is None:
        g = torch.Generator().manual_seed(5)
        shape = (case.num_seqs, case.shape.head_dim)
        return (torch.randn(shape, generator=g).to(torch.bfloat16),
                torch.randn(shape, generator=g).to(torch.bfloat16))
    rope = RotaryEmbedding(case.shape.head_dim, 1 << 17, base).to(torch.bfloat16)
    return rope.get_cos_sin(torch.as_tensor(case.ctx, dtype=torch.long))


def _fused(case, cos, sin, part):
    s = case.shape
    g = case.to(DEV)
    out = ops.paged_decode(g.q, g.kv_cache, g.block_table, g.context_lens, s.scale,
                           s.num_heads, s.num_kv_heads, s.head_dim, partition_tokens=part,
                           new_k=g.k, new_v=g.v, cos=cos.to(DEV), sin=sin.to(DEV))
    torch.cuda.synchronize()
    return out.cpu(), g.kv_cache.cpu()


def _two_launches(case, cos, sin, part):
    s = case.shape
    g = case.to(DEV)
    qr = ops.rope_kv_append(g.q, g.k, g.v, cos.to(DEV), sin.to(DEV), g.kv_cache,
                            g.block_table, g.context_lens)
    out = ops.paged_decode(qr, g.kv_cache, g.block_table, g.context_lens, s.scale,
                           s.num_heads, s.num_kv_heads, s.head_dim, partition_tokens=part)
    torch.cuda.synchronize()
    return out.cpu(), g.kv_cache.cpu()


def _check(case, base, part):
    cos, sin = _cos_sin(case, base)
    out_f, pool_f = _fused(case, cos, sin, part)
    out_t, pool_t = _two_launches(case, cos, sin, part)
    assert torch.equal(_bits(pool_f), _bits(pool_t)), "pool differs from rope_kv_append"
    assert torch.equal(_bits(out_f), _bits(out_t)), "output differs from the two launches"
    s = case.shape
    qr, kr = paged_ref.apply_rope(case.q, case.k, cos, sin)
    pool = case.kv_cache.clone()
    want = paged_ref.decode(qr, kr, case.v, pool, case.block_table, case.context_lens, s.scale,
                            s.num_heads, s.num_kv_heads, s.head_dim).float()
    assert torch.equal(_bits(pool_f), _bits(pool)), "pool differs from the oracle"
    got = out_f.float().numpy().astype(np.float64)
    ref = want.numpy().astype(np.float64)
    assert np.isfinite(got).all()
    assert (np.abs(got - ref) - (2e-2 + 1e-2 * np.abs(ref))).max() <= 0


@pytest.mark.parametrize("part", [0, -1, 256])
@pytest.mark.parametrize("cfg", ["qwen2-0.5b-decode", "llama3-8b-decode"])
@pytest.mark.parametrize("base", [1e6, None])
def test_rope_fused_decode_named_cases(cfg, part, base):
    _check(wl.config_case(cfg), base, part)


@pytest.mark.parametrize("part", [-1, 16, 64])
@pytest.mark.parametrize("shape", [wl.HeadShape(28, 4, 128), wl.HeadShape(14, 2, 64),
                                   wl.HeadShape(8, 8, 64), wl.HeadShape(16, 1, 128)])
def test_rope_fused_decode_edges(shape, part):
    # the new token at rows 0 and 15, at a fresh block, at position 0; rope_theta 1e4
    case = wl.decode_case(shape, [0, 15, 16, 255, 256, 1023, 3000], seed=411)
    _check(case, 1e4, part)
