"""GPU parity of the float32 kernels (the reference's --dtype float32, needle/args.py:80-84,
resolved at :143-153).

A float32 model keeps its pools, activations and attention in float32
(needle/model/runner.py:31-34, 75-78), and the torch path of needle/layers/attention.py then
runs every op in float32.  The oracle runs the same restatement in float32 on the CPU.  Bars:
  * pools and rotated q: bit-exact (RoPE's products and sum rounded to float32, as torch's
    three elementwise ops do), except after the drop-in layer's own projections, which
    differ by GEMM and are held to the tolerance below;
  * attention outputs: |gpu - ref| <= 1e-4 + 1e-4 |ref| against the float32 oracle and
    against the fp64 closed form (float32 products and sums in another order, the
    hardware's exp2: errors of a few 1e-6 here);
  * the forms of one operation (fused and separate launches, RoPE in the prefill or before
    it, the allocation-free entry point): bit-identical to each other.
Shapes: the Qwen2-0.5B and Llama-3-8B decode workloads, the Qwen2-7B prompts, group sizes
1-16, both head dims, blocks of 16 and 64 tokens, garbage (NaN and inf bits included) in
every slot no sequence owns.
"""
import numpy as np
import pytest
import torch

from oracle import closed_form, paged_ref
from needle_amd import _lib, ops, workloads as wl
from needle_amd.layers.rope import RotaryEmbedding

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
F32 = torch.float32
ATOL, RTOL = 1e-4, 1e-4


def _bits(t):
    return t.contiguous().view(torch.int32)


def _np(x):
    return np.asarray(x.double().cpu() if torch.is_tensor(x) else x, dtype=np.float64)


def assert_close(got, want, atol=ATOL, rtol=RTOL):
    got, want = _np(got), _np(want)
    assert got.shape == want.shape and np.isfinite(got).all()
    excess = np.abs(got - want) - (atol + rtol * np.abs(want))
    assert excess.max() <= 0, f"max |diff| {np.abs(got - want).max():.4g}"


def _cos_sin(case, base):
    rope = RotaryEmbedding(case.shape.head_dim, 1 << 16, base)
    if case.cu_seqlens is None:
        pos = list(case.ctx)
    else:
        pos = [c + i for c, n in zip(case.ctx, case.new_lens) for i in range(n)]
    cos, sin = rope.get_cos_sin(torch.as_tensor(pos, dtype=torch.long))
    return cos.to(F32), sin.to(F32)


def _decode_oracle(case, qr=None, kr=None):
    s = case.shape
    pool = case.kv_cache.clone()
    out = paged_ref.decode(case.q if qr is None else qr, case.k if kr is None else kr, case.v,
                           pool, case.block_table, case.context_lens, s.scale, s.num_heads,
                           s.num_kv_heads, s.head_dim)
    return out, pool


@pytest.mark.parametrize("part", [0, -1])
@pytest.mark.parametrize("cfg", ["qwen2-0.5b-decode", "llama3-8b-decode"])
def test_decode_fused_and_separate_vs_oracle_and_fp64(cfg, part):
    shape = wl.QWEN2_05B if cfg.startswith("qwen") else wl.LLAMA3_8B
    ctx = wl.qwen05b_decode_ctx() if cfg.startswith("qwen") else wl.llama8b_decode_ctx()
    case = wl.decode_case(shape, ctx, seed=800, dtype=F32,
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
    assert got.dtype == F32
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
def test_decode_group_sizes_and_lengths(shape):
    """Contexts of 0 .. 2049 tokens (a wave with no tiles, partial tiles, a sequence longer
    than 64 tiles per wave), group sizes 1-16."""
    case = wl.decode_case(shape, [0, 15, 16, 100, 777, 2049, 8200], seed=801, dtype=F32)
    s = case.shape
    g = case.to(DEV)
    got = ops.paged_decode(g.q, g.kv_cache, g.block_table, g.context_lens, s.scale, s.num_heads,
                           s.num_kv_heads, s.head_dim, new_k=g.k, new_v=g.v)
    torch.cuda.synchronize()
    want, pool = _decode_oracle(case)
    assert torch.equal(_bits(g.kv_cache.cpu()), _bits(pool))
    assert_close(got, want)


@pytest.mark.parametrize("cfg", ["qwen2-0.5b-decode", "llama3-8b-decode"])
def test_rope_fused_decode(cfg):
    """RoPE in the decode call: q rotated as it is read, the new k row rotated into the pool;
    the same bits as the rotated rows through the plain fused decode."""
    shape = wl.QWEN2_05B if cfg.startswith("qwen") else wl.LLAMA3_8B
    ctx = wl.qwen05b_decode_ctx() if cfg.startswith("qwen") else wl.llama8b_decode_ctx()
    case = wl.decode_case(shape, ctx, seed=802, dtype=F32)
    s = case.shape
    cos, sin = _cos_sin(case, 1e6 if cfg.startswith("qwen") else 500000.0)
    g = case.to(DEV)
    got = ops.paged_decode(g.q, g.kv_cache, g.block_table, g.context_lens, s.scale, s.num_heads,
                           s.num_kv_heads, s.head_dim, new_k=g.k, new_v=g.v, cos=cos.to(DEV),
                           sin=sin.to(DEV))
    qr, kr = paged_ref.apply_rope(case.q, case.k, cos, sin)
    h = case.to(DEV)
    got_rot = ops.paged_decode(qr.contiguous().to(DEV), h.kv_cache, h.block_table,
                               h.context_lens, s.scale, s.num_heads, s.num_kv_heads, s.head_dim,
                               new_k=kr.contiguous().to(DEV), new_v=h.v)
    torch.cuda.synchronize()
    want, pool = _decode_oracle(case, qr, kr)
    assert torch.equal(_bits(g.kv_cache.cpu()), _bits(pool))
    assert torch.equal(_bits(got.cpu()), _bits(got_rot.cpu()))
    assert_close(got, want)


def test_rope_append_bit_exact():
    case = wl.prefill_case(wl.QWEN2_7B, [5, 0, 33, 17, 300], seed=803, dtype=F32,
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
            assert torch.equal(_bits(qo.cpu()), _bits(qr))
        assert torch.equal(_bits(g.kv_cache.cpu()), _bits(want))


def test_append_bit_exact_vs_bruteforce():
    case = wl.prefill_case(wl.QWEN2_05B, [1, 16, 17, 200, 0, 33], seed=804, dtype=F32,
                           ctx_lens=[0, 5, 31, 0, 7, 16])
    g = case.to(DEV)
    ops.write_kv(g.k, g.v, g.kv_cache, g.block_table, g.cu_seqlens, g.context_lens)
    torch.cuda.synchronize()
    want = closed_form.append_bruteforce(case.k, case.v, case.kv_cache, case.block_table,
                                         case.cu_seqlens, case.context_lens)
    assert torch.equal(_bits(g.kv_cache.cpu()), _bits(want))


def _prefill(g, case, q, cos=None, sin=None):
    s = case.shape
    return ops.varlen_prefill(q, g.kv_cache, g.block_table, g.cu_seqlens, g.context_lens,
                              case.max_seqlen, s.scale, s.num_heads, s.num_kv_heads, s.head_dim,
                              max_context_len=max(case.ctx), cos=cos, sin=sin)


def test_qwen2_7b_prefill_vs_oracle_and_rope_forms():
    lens = wl.qwen7b_prefill_lens()
    case = wl.prefill_case(wl.QWEN2_7B, lens, seed=805, dtype=F32)
    s = case.shape
    g = case.to(DEV)
    ops.write_kv(g.k, g.v, g.kv_cache, g.block_table, g.cu_seqlens, g.context_lens)
    got = _prefill(g, case, g.q)
    torch.cuda.synchronize()
    pool = case.kv_cache.clone()
    want = paged_ref.prefill(case.q, case.k, case.v, pool, case.block_table, case.cu_seqlens,
                             case.context_lens, s.num_heads, s.num_kv_heads)
    assert got.dtype == F32
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
    case = wl.prefill_case(shape, [1, 31, 33, 100, 257, 0], seed=806 + group, dtype=F32,
                           ctx_lens=[0, 0, 17, 5, 40, 9])
    s = case.shape
    g = case.to(DEV)
    ops.write_kv(g.k, g.v, g.kv_cache, g.block_table, g.cu_seqlens, g.context_lens)
    got = _prefill(g, case, g.q)
    torch.cuda.synchronize()
    pool = g.kv_cache.cpu()
    want = closed_form.prefill_fp64(case.q, pool, case.block_table, case.cu_seqlens,
                                    case.context_lens, s.scale, s.num_heads, s.num_kv_heads)
    assert_close(got, want)


@pytest.mark.parametrize("bs", [64])
def test_block_size_64(bs):
    """Blocks of 64 tokens (four 16-token tiles each): append, decode and prefill."""
    shape = wl.HeadShape(14, 2, 64, block_size=bs)
    dcase = wl.decode_case(shape, [3, 63, 64, 200, 1000], seed=807, dtype=F32)
    s = dcase.shape
    g = dcase.to(DEV)
    got = ops.paged_decode(g.q, g.kv_cache, g.block_table, g.context_lens, s.scale, s.num_heads,
                           s.num_kv_heads, s.head_dim, new_k=g.k, new_v=g.v)
    torch.cuda.synchronize()
    want, pool = _decode_oracle(dcase)
    assert torch.equal(_bits(g.kv_cache.cpu()), _bits(pool))
    assert_close(got, want)
    pcase = wl.prefill_case(shape, [1, 65, 130, 7], seed=808, dtype=F32, ctx_lens=[0, 63, 5, 64])
    gp = pcase.to(DEV)
    ops.write_kv(gp.k, gp.v, gp.kv_cache, gp.block_table, gp.cu_seqlens, gp.context_lens)
    outp = _prefill(gp, pcase, gp.q)
    torch.cuda.synchronize()
    wantp = closed_form.prefill_fp64(pcase.q, gp.kv_cache.cpu(), pcase.block_table,
                                     pcase.cu_seqlens, pcase.context_lens, s.scale, s.num_heads,
                                     s.num_kv_heads)
    assert_close(outp, wantp)


def test_block_copy_and_allocation_free_decode():
    """The swap copy moves float32 blocks bit for bit; the allocation-free decode gives the
    workspace entry point's bits."""
    case = wl.decode_case(wl.QWEN2_05B, wl.qwen05b_decode_ctx(), seed=809, dtype=F32,
                          num_blocks=512)
    g = case.to(DEV)
    dst = torch.zeros_like(g.kv_cache)
    ids = torch.arange(0, 512, 3, dtype=torch.int32, device=DEV)
    ops.kv_block_copy([dst], [g.kv_cache], ids, ids)
    torch.cuda.synchronize()
    idx = ids.long()
    assert torch.equal(_bits(dst[:, idx].cpu()), _bits(g.kv_cache[:, idx].cpu()))
    s = case.shape
    a = case.to(DEV)
    want = ops.paged_decode(a.q, a.kv_cache, a.block_table, a.context_lens, s.scale,
                            s.num_heads, s.num_kv_heads, s.head_dim, new_k=a.k, new_v=a.v)
    b = case.to(DEV)
    out = torch.empty_like(want)
    lib = _lib.load()
    _, nb, hkv, bs, d = b.kv_cache.shape
    rc = lib.ndl_paged_decode_append_noalloc(
        out.data_ptr(), b.q.data_ptr(), b.q.stride(0), b.k.data_ptr(), b.k.stride(0),
        b.v.data_ptr(), b.v.stride(0), b.kv_cache.data_ptr(), nb, b.block_table.data_ptr(),
        b.block_table.stride(0), b.block_table.shape[1], b.context_lens.data_ptr(),
        b.block_table.shape[0], s.num_heads, s.num_kv_heads, d, bs, _lib.NDL_DTYPE_F32,
        float(s.scale), 0, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == 0, rc
    assert torch.equal(_bits(out.cpu()), _bits(want.cpu()))
    assert torch.equal(_bits(a.kv_cache.cpu()), _bits(b.kv_cache.cpu()))


@torch.no_grad()
def test_attention_layer_in_float32():
    """The drop-in layer built in float32 through a prefill and a decode step against the
    oracle's attention_forward in float32 (projections F.linear, RoPE, seams).  The GPU and
    CPU GEMMs of the projections differ in summation order, so pools and outputs agree to the
    float32 tolerance (5e-4 here, after two GEMMs), not bit for bit."""
    from needle_amd.layers.attention import Attention
    from needle_amd.model.config import ModelConfig
    cfg = ModelConfig(model_type="qwen2", hidden_size=896, num_hidden_layers=1,
                      num_attention_heads=14, num_key_value_heads=2, intermediate_size=64,
                      vocab_size=32, max_position_embeddings=4096, rope_theta=1e6)
    torch.manual_seed(0)
    att = Attention(cfg, 0, qkv_bias=True)
    for p in att.parameters():
        p.data.normal_(0, 0.02)
    weights = {k: v.to(F32) for k, v in att.state_dict().items()}
    att = att.to(device=DEV, dtype=F32)
    rope = RotaryEmbedding(cfg.head_dim, 4096, 1e6)
    lens = [7, 130, 33]
    nb = 64
    pool = torch.zeros((2, nb, 2, 16, cfg.head_dim), dtype=F32)
    tables = [[5, 9, 11, 2, 40, 41, 42, 43, 44, 45, 46], [1, 3, 6, 7, 8, 10, 12, 13, 14, 15, 16],
              [20, 21, 22, 23, 24, 25, 26, 27, 28, 29, 30]]
    bt = torch.tensor(tables, dtype=torch.int32)
    cu = torch.tensor([0, 7, 137, 170], dtype=torch.int32)
    ctx = torch.zeros(3, dtype=torch.int32)
    x = torch.randn((sum(lens), cfg.hidden_size)) * 0.5
    pos = torch.cat([torch.arange(n) for n in lens])
    cos, sin = rope.get_cos_sin(pos)
    pool_ref = pool.clone()
    want = paged_ref.attention_forward(weights, x, pool_ref, bt, cu, ctx, True, cos, sin, 14, 2,
                                       cfg.head_dim)
    pool_gpu = pool.to(DEV)
    got = att(x.to(DEV), pos.to(DEV), pool_gpu, bt.to(DEV), cu.to(DEV), ctx.to(DEV), max(lens),
              True, cos.to(DEV), sin.to(DEV))
    torch.cuda.synchronize()
    assert_close(pool_gpu, pool_ref, 5e-4, 5e-4)
    assert_close(got, want, 5e-4, 5e-4)
    xd = torch.randn((3, cfg.hidden_size)) * 0.5
    ctx_d = torch.tensor(lens, dtype=torch.int32)
    cos_d, sin_d = rope.get_cos_sin(ctx_d.long())
    want_d = paged_ref.attention_forward(weights, xd, pool_ref, bt, None, ctx_d, False, cos_d,
                                         sin_d, 14, 2, cfg.head_dim)
    got_d = att(xd.to(DEV), ctx_d.long().to(DEV), pool_gpu, bt.to(DEV),
                torch.arange(4, dtype=torch.int32, device=DEV), ctx_d.to(DEV), 1, False,
                cos_d.to(DEV), sin_d.to(DEV))
    torch.cuda.synchronize()
    assert_close(pool_gpu, pool_ref, 5e-4, 5e-4)
    assert_close(got_d, want_d, 5e-4, 5e-4)
