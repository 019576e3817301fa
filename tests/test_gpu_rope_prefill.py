"""GPU parity of ndl_rope_varlen_prefill: the rotary embedding of q inside the prefill.

The drop-in layer's prefill (reference needle/layers/attention.py:88 then :102-107) runs
as two launches: ndl_rope_kv_append with q = NULL (k rotated and appended, v appended),
then ndl_rope_varlen_prefill on the raw q, which rotates each query row as it reads it.
It must equal, bit for bit, the form that writes the rotated q to memory and reads it
back: ndl_rope_kv_append (q_out) followed by ndl_varlen_prefill (both checked against the
oracle by their own tests).  Output and the whole pool are compared as bits, at the
Qwen2-7B prefill workload (28/4 heads, head_dim 128, 16 prompts U[128, 2048]), at the
end-to-end model's attention shape (14/2 heads, head_dim 64, prompts U[64, 1024]), for
group sizes 1-16 with arbitrary cos/sin rows, cached prefixes, empty prompts and strided
q views.  The Qwen2-7B case is also held to the oracle (RoPE as the reference's torch ops,
then write_kv and per-prompt SDPA) within |gpu - ref| <= 2e-2 + 1e-2 |ref|.
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


def _positions(case):
    pos = []
    for c, n in zip(case.ctx, case.new_lens):
        pos += list(range(c, c + n))
    return pos


def _table_cos_sin(case, base):
    rope = RotaryEmbedding(case.shape.head_dim, 1 << 16, base).to(torch.bfloat16)
    return rope.get_cos_sin(torch.as_tensor(_positions(case), dtype=torch.long))


def _random_cos_sin(case, seed):
    g = torch.Generator().manual_seed(seed)
    t, d = case.q.shape[0], case.shape.head_dim
    return (torch.randn((t, d), generator=g).to(torch.bfloat16),
            torch.randn((t, d), generator=g).to(torch.bfloat16))


def _both_forms(case, cos, sin, q=None):
    """(out, pool) of the two-launch form with the rotated q in memory, and of the form
    with q rotated inside the prefill."""
    s = case.shape
    q = case.q if q is None else q
    res = []
    for fused in (False, True):
        g = case.to(DEV)
        qd, cd, sd = q.to(DEV), cos.to(DEV), sin.to(DEV)
        if fused:
            assert ops.rope_kv_append(None, g.k, g.v, cd, sd, g.kv_cache, g.block_table,
                                      g.context_lens, g.cu_seqlens) is None
            out = ops.varlen_prefill(qd, g.kv_cache, g.block_table, g.cu_seqlens,
                                     g.context_lens, case.max_seqlen, s.scale, s.num_heads,
                                     s.num_kv_heads, s.head_dim,
                                     max_context_len=max(case.ctx), cos=cd, sin=sd)
        else:
            qr = ops.rope_kv_append(qd, g.k, g.v, cd, sd, g.kv_cache, g.block_table,
                                    g.context_lens, g.cu_seqlens)
            out = ops.varlen_prefill(qr, g.kv_cache, g.block_table, g.cu_seqlens,
                                     g.context_lens, case.max_seqlen, s.scale, s.num_heads,
                                     s.num_kv_heads, s.head_dim, max_context_len=max(case.ctx))
        torch.cuda.synchronize()
        res.append((out.cpu(), g.kv_cache.cpu()))
    return res


def _identical(case, cos, sin, q=None):
    (out_a, pool_a), (out_b, pool_b) = _both_forms(case, cos, sin, q)
    assert torch.equal(_bits(pool_a), _bits(pool_b)), "pools differ"
    assert torch.equal(_bits(out_a), _bits(out_b)), \
        f"outputs differ (max |diff| {(out_a.float() - out_b.float()).abs().max():.3g})"
    return out_b, pool_b


def test_qwen2_7b_prefill_bit_identical_and_vs_oracle():
    case = wl.config_case("qwen2-7b-prefill")
    cos, sin = _table_cos_sin(case, 1e6)
    got, pool = _identical(case, cos, sin)
    s = case.shape
    qr, kr = paged_ref.apply_rope(case.q, case.k, cos, sin)
    want_pool = case.kv_cache.clone()
    want = paged_ref.prefill(qr, kr, case.v, want_pool, case.block_table, case.cu_seqlens,
                             case.context_lens, s.num_heads, s.num_kv_heads)
    assert torch.equal(_bits(pool), _bits(want_pool))
    got, want = got.double().numpy(), want.double().numpy()
    assert np.isfinite(got).all()
    assert (np.abs(got - want) - (2e-2 + 1e-2 * np.abs(want))).max() <= 0


def test_e2e_model_attention_shape_bit_identical():
    """Qwen2-0.5B's attention (14/2 heads, head_dim 64): 16 prompts U[64, 1024]."""
    lens = np.random.default_rng(41).integers(64, 1025, size=16).tolist()
    case = wl.prefill_case(wl.QWEN2_05B, lens, seed=41)
    _identical(case, *_table_cos_sin(case, 1e6))


@pytest.mark.parametrize("group", [1, 3, 4, 7, 8, 16])
@pytest.mark.parametrize("head_dim", [64, 128])
def test_group_sizes_with_arbitrary_cos_sin(group, head_dim):
    shape = wl.HeadShape(2 * group, 2, head_dim)
    case = wl.prefill_case(shape, [1, 31, 32, 33, 100, 257], seed=400 + group + head_dim)
    _identical(case, *_random_cos_sin(case, group))


def test_cached_prefixes_and_empty_prompts():
    case = wl.prefill_case(wl.QWEN2_7B, [5, 0, 33, 17, 1, 0, 300], seed=410,
                           ctx_lens=[0, 3, 14, 16, 100, 0, 700])
    _identical(case, *_table_cos_sin(case, 1e6))


def test_strided_q_view_of_a_fused_projection():
    shape = wl.LLAMA3_8B
    case = wl.prefill_case(shape, [7, 40, 16, 129], seed=411)
    t, h, d = case.q.shape
    hkv = case.k.shape[1]
    fused = torch.randn((t, (h + 2 * hkv) * d)).to(torch.bfloat16)
    q = fused[:, :h * d].view(t, h, d)
    _identical(case, *_table_cos_sin(case, 500000.0), q=q)
