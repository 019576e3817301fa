"""GPU parity of the float16 kernels (the reference's --dtype float16, needle/args.py:80-84).

The model, its pools and its attention run in whatever dtype the reference is started with
(needle/model/runner.py:31-34, 75-78); the torch path of needle/layers/attention.py then works
in float16 op for op.  The oracle runs the same restatement in float16 on the CPU.  Bars, as
for bf16:
  * pools and rotated q: bit-exact (RoPE's roundings are float16's here), except after the
    drop-in layer's own projections, which differ by GEMM and are held to the tolerance;
  * attention outputs: |gpu - ref| <= 2e-2 + 1e-2 |ref| against the float16 oracle and
    against the fp64 closed form;
  * the forms of one operation (fused and separate launches, RoPE in the prefill or before
    it): bit-identical to each other.
Shapes: the Qwen2-0.5B and Llama-3-8B decode workloads (8 x 14/2 x 64 and 64 x 32/8 x 128),
the Qwen2-7B prompts (16 x 28/4 x 128), group sizes 1-16 and both head dims.
"""
import numpy as np
import pytest
import torch

from oracle import closed_form, paged_ref
from needle_amd import ops, workloads as wl
from needle_amd.layers.rope import RotaryEmbedding

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
F16 = torch.float16


def _bits(t):
    return t.view(torch.int16)


def _np(x):
    return np.asarray(x.float().cpu() if torch.is_tensor(x) else x, dtype=np.float64)


def assert_close(got, want):
    got, want = _np(got), _np(want)
    assert got.shape == want.shape and np.isfinite(got).all()
    excess = np.abs(got - want) - (2e-2 + 1e-2 * np.abs(want))
    assert excess.max() <= 0, f"max |diff| {np.abs(got - want).max():.4g}"


def _cos_sin(case, base):
    rope = RotaryEmbedding(case.shape.head_dim, 1 << 16, base).to(F16)
    if case.cu_seqlens is None:
        pos = list(case.ctx)
    else:
        pos = [c + i for c, n in zip(case.ctx, case.new_lens) for i in range(n)]
    return rope.get_cos_sin(torch.as_tensor(pos, dtype=torch.long))


def _decode_oracle(case, qr=None, kr=None):
    s = case.shape
    pool = case.kv_cache.clone()
    out = paged_ref.decode(case.q if qr is None else qr, case.k if kr is None else kr, case.v,
                           pool, case.block_table, case.context_lens, s.scale, s.num_heads,
                           s.num_kv_heads, s.head_dim)
    return out, pool


@pytest.mark.parametrize("part", [0, -1, 256])
@pytest.mark.parametrize("cfg", ["qwen2-0.5b-decode", "llama3-8b-decode"])
def test_fused_decode_vs_oracle_and_fp64(cfg, part):
    shape = wl.QWEN2_05B if cfg.startswith("qwen") else wl.LLAMA3_8B
    ctx = wl.qwen05b_decode_ctx() if cfg.startswith("qwen") else wl.llama8b_decode_ctx()
    case = wl.decode_case(shape, ctx, seed=700, dtype=F16,
                          num_blocks=512 if cfg.startswith("qwen") else None)
    s = case.shape
    g = case.to(DEV)
    got = ops.paged_decode(g.q, g.kv_cache, g.block_table, g.context_lens, s.scale, s.num_heads,
                           s.num_kv_heads, s.head_dim, new_k=g.k, new_v=g.v,
                           partition_tokens=part)
    sep = case.to(DEV)
    ops.kv_append(sep.k, sep.v, sep.kv_cache, sep.block_table, sep.context_lens)
    got_sep = ops.paged_decode(sep.q, sep.kv_cache, sep.block_table, sep.context_lens, s.scale,
                               s.num_heads, s.num_kv_heads, s.head_dim, partition_tokens=part)
    torch.cuda.synchronize()
    assert got.dtype == F16
    want, pool = _decode_oracle(case)
    assert torch.equal(_bits(g.kv_cache.cpu()), _bits(pool))
    assert torch.equal(_bits(sep.kv_cache.cpu()), _bits(pool))
    assert torch.equal(_bits(got.cpu()), _bits(got_sep.cpu()))
    assert_close(got, want)
    assert_close(got, closed_form.decode_fp64(case.q, pool, case.block_table, case.context_lens,
                                              s.scale, s.num_heads, s.num_kv_heads))


@pytest.mark.parametrize("shape", [wl.HeadShape(8, 8, 128), wl.HeadShape(28, 4, 128),
                                   wl.HeadShape(16, 1, 128), wl.HeadShape(4, 4, 64),
                                   wl.HeadShape(14, 2, 64), wl.HeadShape(32, 2, 64)])
@pytest.mark.parametrize("part", [-1, 64])
def test_decode_group_sizes(shape, part):
    case = wl.decode_case(shape, [0, 15, 16, 100, 777, 2049], seed=701, dtype=F16)
    s = case.shape
    g = case.to(DEV)
    got = ops.paged_decode(g.q, g.kv_cache, g.block_table, g.context_lens, s.scale, s.num_heads,
                           s.num_kv_heads, s.head_dim, new_k=g.k, new_v=g.v,
                           partition_tokens=part)
    torch.cuda.synchronize()
    want, pool = _decode_oracle(case)
    assert torch.equal(_bits(g.kv_cache.cpu()), _bits(pool))
    assert_close(got, want)


@pytest.mark.parametrize("cfg", ["qwen2-0.5b-decode", "llama3-8b-decode"])
def test_rope_fused_decode(cfg):
    """RoPE folded into the decode launch: q rotated, the new k row rotated into the pool."""
    shape = wl.QWEN2_05B if cfg.startswith("qwen") else wl.LLAMA3_8B
    ctx = wl.qwen05b_decode_ctx() if cfg.startswith("qwen") else wl.llama8b_decode_ctx()
    case = wl.decode_case(shape, ctx, seed=702, dtype=F16)
    s = case.shape
    cos, sin = _cos_sin(case, 1e6 if cfg.startswith("qwen") else 500000.0)
    g = case.to(DEV)
    got = ops.paged_decode(g.q, g.kv_cache, g.block_table, g.context_lens, s.scale, s.num_heads,
                           s.num_kv_heads, s.head_dim, new_k=g.k, new_v=g.v, cos=cos.to(DEV),
                           sin=sin.to(DEV))
    torch.cuda.synchronize()
    qr, kr = paged_ref.apply_rope(case.q, case.k, cos, sin)
    want, pool = _decode_oracle(case, qr, kr)
    assert torch.equal(_bits(g.kv_cache.cpu()), _bits(pool))
    assert_close(got, want)


def test_rope_append_bit_exact():
    case = wl.prefill_case(wl.QWEN2_7B, [5, 0, 33, 17, 300], seed=703, dtype=F16,
                           ctx_lens=[0, 3, 14, 16, 0])
    cos, sin = _cos_sin(case, 1e6)
    qr, kr = paged_ref.apply_rope(case.q, case.k, cos, sin)
    want = case.kv_cache.clone()
    paged_ref.write_kv(kr, case.v, want, case.block_table, case.cu_seqlens, case.context_lens)
    for with_q in (True, False):
        g = case.to(DEV)
        qo = ops.rope_kv_append(g.q if with_q else None, g.k, g.v, cos.to(DEV), sin.to(DEV),
                                g.kv_cache, g.block_table, g.context_lens, g.cu_seqlens)
        torch.cuda.synchronize()
        if with_q:
            assert torch.equal(_bits(qo.cpu()), _bits(qr.contiguous()))
        assert torch.equal(_bits(g.kv_cache.cpu()), _bits(want))


def _prefill(g, case, q, cos=None, sin=None):
    s = case.shape
    return ops.varlen_prefill(q, g.kv_cache, g.block_table, g.cu_seqlens, g.context_lens,
                              case.max_seqlen, s.scale, s.num_heads, s.num_kv_heads, s.head_dim,
                              max_context_len=max(case.ctx), cos=cos, sin=sin)


def test_qwen2_7b_prefill_vs_oracle_and_rope_forms():
    lens = wl.qwen7b_prefill_lens()
    case = wl.prefill_case(wl.QWEN2_7B, lens, seed=704, dtype=F16)
    s = case.shape
    # plain: write_kv + prefill against the float16 oracle (per-prompt SDPA)
    g = case.to(DEV)
    ops.write_kv(g.k, g.v, g.kv_cache, g.block_table, g.cu_seqlens, g.context_lens)
    got = _prefill(g, case, g.q)
    torch.cuda.synchronize()
    pool = case.kv_cache.clone()
    want = paged_ref.prefill(case.q, case.k, case.v, pool, case.block_table, case.cu_seqlens,
                             case.context_lens, s.num_heads, s.num_kv_heads)
    assert torch.equal(_bits(g.kv_cache.cpu()), _bits(pool))
    assert_close(got, want)
    # RoPE: the rotated q in memory against the rotation inside the prefill, bit for bit
    cos, sin = _cos_sin(case, 1e6)
    a = case.to(DEV)
    qr = ops.rope_kv_append(a.q, a.k, a.v, cos.to(DEV), sin.to(DEV), a.kv_cache, a.block_table,
                            a.context_lens, a.cu_seqlens)
    out_a = _prefill(a, case, qr)
    b = case.to(DEV)
    ops.rope_kv_append(None, b.k, b.v, cos.to(DEV), sin.to(DEV), b.kv_cache, b.block_table,
                       b.context_lens, b.cu_seqlens)
    out_b = _prefill(b, case, b.q, cos.to(DEV), sin.to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(_bits(a.kv_cache.cpu()), _bits(b.kv_cache.cpu()))
    assert torch.equal(_bits(out_a.cpu()), _bits(out_b.cpu()))


@pytest.mark.parametrize("group", [1, 4, 7, 16])
@pytest.mark.parametrize("head_dim", [64, 128])
def test_prefill_group_sizes_and_prefix_vs_fp64(group, head_dim):
    shape = wl.HeadShape(2 * group, 2, head_dim)
    case = wl.prefill_case(shape, [1, 31, 33, 100, 257], seed=705 + group, dtype=F16,
                           ctx_lens=[0, 0, 17, 5, 40])
    s = case.shape
    g = case.to(DEV)
    ops.write_kv(g.k, g.v, g.kv_cache, g.block_table, g.cu_seqlens, g.context_lens)
    got = _prefill(g, case, g.q)
    torch.cuda.synchronize()
    pool = g.kv_cache.cpu()
    want = closed_form.prefill_fp64(case.q, pool, case.block_table, case.cu_seqlens,
                                    case.context_lens, s.scale, s.num_heads, s.num_kv_heads)
    assert_close(got, want)


@torch.no_grad()
def test_attention_layer_in_float16():
    """The drop-in layer built in float16 through a prefill and a decode step against the
    oracle's attention_forward in float16 (projections F.linear, RoPE, seams).  The pools
    agree to the tolerance, not bit for bit: the k/v projections run through different GEMM
    implementations on the GPU and the CPU (the append and RoPE are bit-exact above)."""
    from needle_amd.layers.attention import Attention
    from needle_amd.model.config import ModelConfig
    cfg = ModelConfig(model_type="qwen2", hidden_size=896, num_hidden_layers=1,
                      num_attention_heads=14, num_key_value_heads=2, intermediate_size=64,
                      vocab_size=32, max_position_embeddings=4096, rope_theta=1e6)
    torch.manual_seed(0)
    att = Attention(cfg, 0, qkv_bias=True)
    for p in att.parameters():
        p.data.normal_(0, 0.02)
    weights = {k: v.to(F16) for k, v in att.state_dict().items()}
    att = att.to(device=DEV, dtype=F16)
    rope = RotaryEmbedding(cfg.head_dim, 4096, 1e6).to(F16)
    lens = [7, 130, 33]
    nb = 64
    pool = torch.zeros((2, nb, 2, 16, cfg.head_dim), dtype=F16)
    tables = [[5, 9, 11, 2, 40, 41, 42, 43, 44, 45, 46], [1, 3, 6, 7, 8, 10, 12, 13, 14, 15, 16],
              [20, 21, 22, 23, 24, 25, 26, 27, 28, 29, 30]]
    bt = torch.tensor(tables, dtype=torch.int32)
    cu = torch.tensor([0, 7, 137, 170], dtype=torch.int32)
    ctx = torch.zeros(3, dtype=torch.int32)
    x = (torch.randn((sum(lens), cfg.hidden_size)) * 0.5).to(F16)
    pos = torch.cat([torch.arange(n) for n in lens])
    cos, sin = rope.get_cos_sin(pos)
    pool_ref = pool.clone()
    want = paged_ref.attention_forward(weights, x, pool_ref, bt, cu, ctx, True, cos, sin, 14, 2,
                                       cfg.head_dim)
    pool_gpu = pool.to(DEV)
    got = att(x.to(DEV), pos.to(DEV), pool_gpu, bt.to(DEV), cu.to(DEV), ctx.to(DEV), max(lens),
              True, cos.to(DEV), sin.to(DEV))
    torch.cuda.synchronize()
    assert_close(pool_gpu, pool_ref)
    assert_close(got, want)
    # one decode step: the next token of each sequence
    xd = (torch.randn((3, cfg.hidden_size)) * 0.5).to(F16)
    ctx_d = torch.tensor(lens, dtype=torch.int32)
    cos_d, sin_d = rope.get_cos_sin(ctx_d.long())
    want_d = paged_ref.attention_forward(weights, xd, pool_ref, bt, None, ctx_d, False, cos_d,
                                         sin_d, 14, 2, cfg.head_dim)
    got_d = att(xd.to(DEV), ctx_d.long().to(DEV), pool_gpu, bt.to(DEV),
                torch.arange(4, dtype=torch.int32, device=DEV), ctx_d.to(DEV), 1, False,
                cos_d.to(DEV), sin_d.to(DEV))
    torch.cuda.synchronize()
    assert_close(pool_gpu, pool_ref)
    assert_close(got_d, want_d)
