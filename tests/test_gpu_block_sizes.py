"""GPU parity at block sizes other than 16: the reference's --page-size (needle/args.py:31,
97-101), the block_size of its ModelRunner pools and BlockAllocator
(needle/backend/engine.py:29-69, needle/model/runner.py:65-94).

Pools are [2, NB, Hkv, bs, D] for bs = 32 .. 256; the attention kernels read them as
16-token tiles (tile t of a sequence is rows 16 (t mod bs/16) .. + 16 of table column
t // (bs/16)).  Bars as at bs = 16: pools byte-equal to the oracle's (append, fused append,
RoPE), attention |gpu - ref| <= 2e-2 + 1e-2 |ref| against the bf16 oracle and the fp64
closed form, and the fused and separate forms of one operation bit-identical.  The table
clamp is covered where it matters most for larger blocks: a context past the table row
whose appended row lands in a middle tile of the last block, not in the last tile.
"""
import numpy as np
import pytest
import torch

from oracle import closed_form, paged_ref
from needle_amd import ops, workloads as wl
from needle_amd.layers.rope import RotaryEmbedding

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
ATOL, RTOL = 2e-2, 1e-2
BLOCK_SIZES = [32, 64, 128, 256]


def _np(x):
    return np.asarray(x.float().cpu() if torch.is_tensor(x) else x, dtype=np.float64)


def assert_close(got, want):
    got, want = _np(got), _np(want)
    assert got.shape == want.shape and np.isfinite(got).all()
    excess = np.abs(got - want) - (ATOL + RTOL * np.abs(want))
    assert excess.max() <= 0, f"max |diff| {np.abs(got - want).max():.4g}"


def _bits(t):
    return t.view(torch.int16)


def _shape(base, bs):
    return wl.HeadShape(base.num_heads, base.num_kv_heads, base.head_dim, bs)


def _decode(g, s, part=0, **kw):
    return ops.paged_decode(g.q, g.kv_cache, g.block_table, g.context_lens, s.scale, s.num_heads,
                            s.num_kv_heads, s.head_dim, partition_tokens=part, **kw)


def _check_decode(case, part):
    """Fused append + attention against the separate launches (bit for bit), the oracle's
    append + decode (pool bytes, tolerance) and the fp64 closed form."""
    s = case.shape
    a = case.to(DEV)
    ops.kv_append(a.k, a.v, a.kv_cache, a.block_table, a.context_lens)
    out_a = _decode(a, s, part)
    b = case.to(DEV)
    out_b = _decode(b, s, part, new_k=b.k, new_v=b.v)
    torch.cuda.synchronize()
    pool = case.kv_cache.clone()
    want = paged_ref.decode(case.q, case.k, case.v, pool, case.block_table, case.context_lens,
                            s.scale, s.num_heads, s.num_kv_heads, s.head_dim)
    assert torch.equal(_bits(a.kv_cache.cpu()), _bits(pool))
    assert torch.equal(_bits(b.kv_cache.cpu()), _bits(pool))
    assert torch.equal(_bits(out_a.cpu()), _bits(out_b.cpu()))
    assert_close(out_b, want)
    assert_close(out_b, closed_form.decode_fp64(case.q, pool, case.block_table,
                                                case.context_lens, s.scale, s.num_heads,
                                                s.num_kv_heads))


@pytest.mark.parametrize("bs", BLOCK_SIZES)
def test_append_decode_and_varlen(bs):
    shape = _shape(wl.QWEN2_7B, bs)
    case = wl.prefill_case(shape, [5, 0, 40, 17, 300, 1], seed=800 + bs,
                           ctx_lens=[0, 3, 100, bs - 1, 0, 2 * bs])
    g = case.to(DEV)
    ops.write_kv(g.k, g.v, g.kv_cache, g.block_table, g.cu_seqlens, g.context_lens)
    want = case.kv_cache.clone()
    paged_ref.write_kv(case.k, case.v, want, case.block_table, case.cu_seqlens,
                       case.context_lens)
    torch.cuda.synchronize()
    assert torch.equal(_bits(g.kv_cache.cpu()), _bits(want))
    dcase = wl.decode_case(_shape(wl.LLAMA3_8B, bs), [0, bs - 1, bs, 3 * bs + 7, 500],
                           seed=810 + bs)
    d = dcase.to(DEV)
    ops.kv_append(d.k, d.v, d.kv_cache, d.block_table, d.context_lens)
    want = dcase.kv_cache.clone()
    paged_ref.decode_append(dcase.k, dcase.v, want, dcase.block_table, dcase.context_lens)
    torch.cuda.synchronize()
    assert torch.equal(_bits(d.kv_cache.cpu()), _bits(want))


@pytest.mark.parametrize("part", [0, -1, 64])
@pytest.mark.parametrize("base", [wl.QWEN2_05B, wl.LLAMA3_8B], ids=["qwen-shape", "llama-shape"])
@pytest.mark.parametrize("bs", BLOCK_SIZES)
def test_decode(bs, base, part):
    ctx = np.random.default_rng(820 + bs).integers(0, 1500, size=12).tolist()
    ctx[:4] = [0, bs - 1, bs, 15]
    _check_decode(wl.decode_case(_shape(base, bs), ctx, seed=830 + bs), part)


@pytest.mark.parametrize("part", [0, -1, 16])
@pytest.mark.parametrize("bs", [32, 64, 256])
def test_decode_table_clamp_mid_block(bs, part):
    """Contexts past a two-column table: the append lands in column 1 at row ctx % bs, a
    middle tile of that block (not the last attended tile); attention covers 2 bs tokens."""
    shape = _shape(wl.LLAMA3_8B, bs)
    case = wl.decode_case(shape, [bs + 3, bs + 10, 5], seed=840 + bs, garbage=False)
    ctx = [2 * bs + 20, 3 * bs + bs // 2 + 1, 5]   # rows 20 and bs/2 + 1 of column 1
    case.context_lens = torch.tensor(ctx, dtype=torch.int32)
    case.ctx = ctx
    _check_decode(case, part)


@pytest.mark.parametrize("bs", [32, 128])
def test_rope_fused_decode(bs):
    shape = _shape(wl.QWEN2_05B, bs)
    case = wl.decode_case(shape, [33, 700, 0, bs * 3 - 1, 250], seed=850 + bs)
    s = case.shape
    rope = RotaryEmbedding(s.head_dim, 4096, 1e6).to(torch.bfloat16)
    cos, sin = rope.get_cos_sin(torch.tensor(case.ctx, dtype=torch.long))
    for part in (0, -1, 64):
        a = case.to(DEV)
        qr = ops.rope_kv_append(a.q, a.k, a.v, cos.to(DEV), sin.to(DEV), a.kv_cache,
                                a.block_table, a.context_lens)
        out_a = ops.paged_decode(qr, a.kv_cache, a.block_table, a.context_lens, s.scale,
                                 s.num_heads, s.num_kv_heads, s.head_dim, partition_tokens=part)
        b = case.to(DEV)
        out_b = _decode(b, s, part, new_k=b.k, new_v=b.v, cos=cos.to(DEV), sin=sin.to(DEV))
        torch.cuda.synchronize()
        assert torch.equal(_bits(a.kv_cache.cpu()), _bits(b.kv_cache.cpu()))
        assert torch.equal(_bits(out_a.cpu()), _bits(out_b.cpu()))
    qr, kr = paged_ref.apply_rope(case.q, case.k, cos, sin)
    pool = case.kv_cache.clone()
    want = paged_ref.decode(qr, kr, case.v, pool, case.block_table, case.context_lens, s.scale,
                            s.num_heads, s.num_kv_heads, s.head_dim)
    assert torch.equal(_bits(b.kv_cache.cpu()), _bits(pool))
    assert_close(out_b, want)


def _prefill(g, case, q, cos=None, sin=None):
    s = case.shape
    return ops.varlen_prefill(q, g.kv_cache, g.block_table, g.cu_seqlens, g.context_lens,
                              case.max_seqlen, s.scale, s.num_heads, s.num_kv_heads, s.head_dim,
                              max_context_len=max(case.ctx), cos=cos, sin=sin)


@pytest.mark.parametrize("base", [wl.QWEN2_7B, wl.QWEN2_05B], ids=["d128", "d64"])
@pytest.mark.parametrize("bs", BLOCK_SIZES)
def test_prefill_with_prefixes(bs, base):
    shape = _shape(base, bs)
    lens = [1, 31, 33, 100, 257, 1100]        # 1100: past one 64-tile window of the table
    ctxs = [0, 0, 17, bs, 40, 3 * bs + 5]
    case = wl.prefill_case(shape, lens, seed=860 + bs, ctx_lens=ctxs)
    s = case.shape
    g = case.to(DEV)
    ops.write_kv(g.k, g.v, g.kv_cache, g.block_table, g.cu_seqlens, g.context_lens)
    got = _prefill(g, case, g.q)
    torch.cuda.synchronize()
    pool = g.kv_cache.cpu()
    want = closed_form.prefill_fp64(case.q, pool, case.block_table, case.cu_seqlens,
                                    case.context_lens, s.scale, s.num_heads, s.num_kv_heads)
    assert_close(got, want)


@pytest.mark.parametrize("bs", [32, 64])
def test_prefill_against_the_oracle_and_rope_forms(bs):
    """No prefix (the reference's runner): against the bf16 oracle; then q's RoPE inside the
    prefill against the rotated q written by the RoPE append, bit for bit."""
    shape = _shape(wl.QWEN2_7B, bs)
    lens = np.random.default_rng(870 + bs).integers(128, 2048, size=6).tolist()
    case = wl.prefill_case(shape, lens, seed=870 + bs)
    s = case.shape
    g = case.to(DEV)
    ops.write_kv(g.k, g.v, g.kv_cache, g.block_table, g.cu_seqlens, g.context_lens)
    got = _prefill(g, case, g.q)
    torch.cuda.synchronize()
    pool = case.kv_cache.clone()
    want = paged_ref.prefill(case.q, case.k, case.v, pool, case.block_table, case.cu_seqlens,
                             case.context_lens, s.num_heads, s.num_kv_heads)
    assert torch.equal(_bits(g.kv_cache.cpu()), _bits(pool))
    assert_close(got, want)
    rope = RotaryEmbedding(s.head_dim, 4096, 1e6).to(torch.bfloat16)
    pos = [i for n in lens for i in range(n)]
    cos, sin = rope.get_cos_sin(torch.tensor(pos, dtype=torch.long))
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


def _masked_fp64(q, pool, bt, nb, scale, group, rows):
    """fp64 attention of each (row, head) over positions 0 .. last read through bt (column
    min(p // bs, W - 1), row p % bs), keys in blocks outside [0, nb) dropped; a row with no
    key left is zero.  rows: (sequence, query row of q, last position attended)."""
    kvn = pool.double().numpy()
    qn = q.double().numpy()
    bs, w = pool.shape[3], bt.shape[1]
    btn = bt.numpy()
    want = np.zeros((len(rows), q.shape[1], q.shape[2]))
    gathered = {}
    for o, (i, t, last) in enumerate(rows):
        if i not in gathered:
            top = max(r[2] for r in rows if r[0] == i)
            pos = np.arange(top + 1)
            blk = btn[i][np.minimum(pos // bs, w - 1)]
            ok = (blk >= 0) & (blk < nb)
            safe = np.where(ok, blk, 0)
            gathered[i] = (kvn[0, safe, :, pos % bs], kvn[1, safe, :, pos % bs], ok)
        k_all, v_all, ok = gathered[i]
        m = ok[:last + 1]
        if not m.any():
            continue
        kr, vr = k_all[:last + 1][m], v_all[:last + 1][m]       # [keys, Hkv, D]
        for h in range(q.shape[1]):
            sc = kr[:, h // group] @ qn[t, h] * scale
            pr = np.exp(sc - sc.max())
            want[o, h] = pr @ vr[:, h // group] / pr.sum()
    return want


@pytest.mark.parametrize("bs", [32, 128])
def test_invalid_block_ids(bs):
    """Ids outside [0, num_blocks) are never dereferenced: their keys are dropped, in the
    decode (both splits) and the prefill, at every tile of such a block."""
    shape = _shape(wl.LLAMA3_8B, bs)
    case = wl.decode_case(shape, [3 * bs + 5, 2 * bs + 1], seed=880 + bs, garbage=False)
    nb = case.kv_cache.shape[1]
    bt = case.block_table.clone()
    bt[0, 1] = -4
    bt[1, 0] = nb + 3
    case.block_table = bt
    s = case.shape
    for part in (0, -1, 16):
        g = case.to(DEV)
        out = _decode(g, s, part)
        torch.cuda.synchronize()
        rows = [(i, i, c) for i, c in enumerate(case.ctx)]
        assert_close(out.cpu(), _masked_fp64(case.q, case.kv_cache, bt, nb, s.scale, s.group,
                                             rows))
    pshape = _shape(wl.QWEN2_7B, bs)
    pcase = wl.prefill_case(pshape, [3 * bs + 9, 2 * bs], seed=890 + bs)
    pnb = pcase.kv_cache.shape[1]
    pbt = pcase.block_table.clone()
    pbt[0, 1] = -2
    pbt[1, 0] = pnb + 1
    pcase.block_table = pbt
    g = pcase.to(DEV)
    ops.write_kv(g.k, g.v, g.kv_cache, g.block_table, g.cu_seqlens, g.context_lens)
    got = _prefill(g, pcase, g.q)
    torch.cuda.synchronize()
    cu = pcase.cu_seqlens.tolist()
    rows = [(i, t, t - cu[i]) for i in range(len(cu) - 1) for t in range(cu[i], cu[i + 1])]
    assert_close(got.cpu(), _masked_fp64(pcase.q, g.kv_cache.cpu(), pbt, pnb, pshape.scale,
                                         pshape.group, rows))


def test_attention_layer_at_block_size_64():
    """The drop-in layer with 64-token pages through a prefill and a decode step against the
    oracle's attention_forward (projections F.linear, RoPE, seams)."""
    from needle_amd.layers.attention import Attention
    from needle_amd.model.config import ModelConfig
    cfg = ModelConfig(model_type="qwen2", hidden_size=896, num_hidden_layers=1,
                      num_attention_heads=14, num_key_value_heads=2, intermediate_size=64,
                      vocab_size=32, max_position_embeddings=4096, rope_theta=1e6)
    torch.manual_seed(1)
    att = Attention(cfg, 0, qkv_bias=True)
    for p in att.parameters():
        p.data.normal_(0, 0.02)
    weights = {k: v.to(torch.bfloat16) for k, v in att.state_dict().items()}
    att = att.to(device=DEV, dtype=torch.bfloat16)
    rope = RotaryEmbedding(cfg.head_dim, 4096, 1e6).to(torch.bfloat16)
    bs, lens = 64, [7, 130, 64]
    pool = torch.zeros((2, 24, 2, bs, cfg.head_dim), dtype=torch.bfloat16)
    bt = torch.tensor([[5, 9, 11], [1, 3, 6], [20, 21, 22]], dtype=torch.int32)
    cu = torch.tensor([0, 7, 137, 201], dtype=torch.int32)
    ctx = torch.zeros(3, dtype=torch.int32)
    x = (torch.randn((sum(lens), cfg.hidden_size)) * 0.5).to(torch.bfloat16)
    pos = torch.cat([torch.arange(n) for n in lens])
    cos, sin = rope.get_cos_sin(pos)
    pool_ref = pool.clone()
    with torch.no_grad():
        want = paged_ref.attention_forward(weights, x, pool_ref, bt, cu, ctx, True, cos, sin, 14,
                                           2, cfg.head_dim)
        pool_gpu = pool.to(DEV)
        got = att(x.to(DEV), pos.to(DEV), pool_gpu, bt.to(DEV), cu.to(DEV), ctx.to(DEV),
                  max(lens), True, cos.to(DEV), sin.to(DEV))
        torch.cuda.synchronize()
        assert_close(pool_gpu, pool_ref)
        assert_close(got, want)
        xd = (torch.randn((3, cfg.hidden_size)) * 0.5).to(torch.bfloat16)
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
