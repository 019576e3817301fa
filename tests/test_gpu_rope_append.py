"""GPU parity of ndl_rope_kv_append: rotated q and the whole pool, bit for bit.

The oracle applies RoPE as the reference does (attention.py:277-288, torch bf16
ops) and then appends (attention.py:141-154 for decode, :204-246 for varlen).
The fused launch must produce the same q bits and leave the same pool bits,
including the random bit patterns outside the owned slots.  The k-only form (q = NULL,
which the drop-in prefill uses before ndl_rope_varlen_prefill; it runs the append
kernel's rotating variant) must leave the same pool bits too.
"""
import pytest
import torch

from oracle import paged_ref
from needle_amd import ops, workloads as wl
from needle_amd.layers.rope import RotaryEmbedding

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _bits(t):
    return t.view(torch.int16)


def _cos_sin(case, positions, base):
    rope = RotaryEmbedding(case.shape.head_dim, 1 << 17, base).to(torch.bfloat16)
    return rope.get_cos_sin(torch.as_tensor(positions, dtype=torch.long))


def _positions(case):
    if case.cu_seqlens is None:
        return list(case.ctx)
    pos = []
    for c, n in zip(case.ctx, case.new_lens):
        pos += list(range(c, c + n))
    return pos


def _parity(case, base=1e6, q=None, k=None, v=None, with_q=True):
    q = case.q if q is None else q
    k = case.k if k is None else k
    v = case.v if v is None else v
    cos, sin = _cos_sin(case, _positions(case), base)
    qr, kr = paged_ref.apply_rope(q, k, cos, sin)
    want = case.kv_cache.clone()
    if case.cu_seqlens is None:
        paged_ref.decode_append(kr, v, want, case.block_table, case.context_lens)
    else:
        paged_ref.write_kv(kr, v, want, case.block_table, case.cu_seqlens, case.context_lens)
    g = case.to(DEV)
    qo = ops.rope_kv_append(q.to(DEV) if with_q else None, k.to(DEV), v.to(DEV), cos.to(DEV),
                            sin.to(DEV), g.kv_cache, g.block_table, g.context_lens, g.cu_seqlens)
    torch.cuda.synchronize()
    if with_q:
        assert torch.equal(_bits(qo.cpu()), _bits(qr.contiguous()))
    else:
        assert qo is None
    assert torch.equal(_bits(g.kv_cache.cpu()), _bits(want))


@pytest.mark.parametrize("cfg", ["qwen2-0.5b-decode", "llama3-8b-decode"])
def test_decode_rope_append_named_cases(cfg):
    _parity(wl.config_case(cfg), base=1e6 if cfg.startswith("qwen") else 500000.0)


def test_varlen_rope_append_qwen2_7b_prefill():
    _parity(wl.config_case("qwen2-7b-prefill"))


def test_rope_append_block_edges_and_long_positions():
    _parity(wl.decode_case(wl.LLAMA3_8B, [0, 15, 16, 17, 31, 32, 1000, 20000], seed=201),
            base=500000.0)
    _parity(wl.decode_case(wl.QWEN2_05B, [0, 15, 16, 17, 31, 32, 1000], seed=202))


def test_varlen_rope_append_prefix_and_empty_seqs():
    _parity(wl.prefill_case(wl.QWEN2_7B, [5, 0, 33, 17, 1, 0], seed=203,
                            ctx_lens=[0, 3, 14, 16, 100, 0]))


def test_varlen_rope_append_clamp_overflow():
    case = wl.prefill_case(wl.QWEN2_05B, [3, 5], seed=204, ctx_lens=[16, 40])
    case.block_table = case.block_table[:, :1].contiguous()
    _parity(case)


def test_rope_append_fused_projection_views():
    # q, k and v as views into one fused projection output [T, (H + 2 Hkv) * D]
    shape = wl.LLAMA3_8B
    case = wl.prefill_case(shape, [7, 40, 16], seed=205)
    t, h, d = case.q.shape
    hkv = case.k.shape[1]
    fused = torch.randn((t, (h + 2 * hkv) * d)).to(torch.bfloat16)
    q = fused[:, :h * d].view(t, h, d)
    k = fused[:, h * d:(h + hkv) * d].view(t, hkv, d)
    v = fused[:, (h + hkv) * d:].view(t, hkv, d)
    _parity(case, base=500000.0, q=q, k=k, v=v)


def test_rope_append_single_token():
    _parity(wl.decode_case(wl.QWEN2_7B, [77], seed=206))


@pytest.mark.parametrize("cfg", ["qwen2-0.5b-decode", "llama3-8b-decode", "qwen2-7b-prefill"])
def test_k_only_form_named_cases(cfg):
    _parity(wl.config_case(cfg), base=500000.0 if cfg.startswith("llama") else 1e6,
            with_q=False)


def test_k_only_form_edges():
    # prefixes and empty prompts; the column clamp; more than 63 prompts (the binary-search
    # lookup); one token; strided k/v views; head_dim 64
    _parity(wl.prefill_case(wl.QWEN2_7B, [5, 0, 33, 17, 1, 0], seed=207,
                            ctx_lens=[0, 3, 14, 16, 100, 0]), with_q=False)
    case = wl.prefill_case(wl.QWEN2_05B, [3, 5], seed=208, ctx_lens=[16, 40])
    case.block_table = case.block_table[:, :1].contiguous()
    _parity(case, with_q=False)
    lens = [1 + (7 * i) % 23 for i in range(80)]
    _parity(wl.prefill_case(wl.QWEN2_05B, lens, seed=209), with_q=False)
    _parity(wl.decode_case(wl.QWEN2_7B, [77], seed=210), with_q=False)
    case = wl.prefill_case(wl.LLAMA3_8B, [7, 40, 16], seed=211)
    t, h, d = case.q.shape
    hkv = case.k.shape[1]
    fused = torch.randn((t, (h + 2 * hkv) * d)).to(torch.bfloat16)
    _parity(case, base=500000.0, k=fused[:, h * d:(h + hkv) * d].view(t, hkv, d),
            v=fused[:, (h + hkv) * d:].view(t, hkv, d), with_q=False)
