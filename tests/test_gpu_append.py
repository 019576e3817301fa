"""GPU parity of ndl_kv_append: the whole pool must equal the oracle's, bit for bit.

The pool is pre-filled with random bit patterns outside the owned slots, so a
stray write anywhere shows up in the byte compare.
"""
import numpy as np
import pytest
import torch

from oracle import paged_ref
from needle_amd import ops, workloads as wl

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _bits(t):
    return t.view(torch.int16) if t.element_size() == 2 else t.view(torch.int32)


def _decode_parity(case):
    want = case.kv_cache.clone()
    paged_ref.decode_append(case.k, case.v, want, case.block_table, case.context_lens)
    g = case.to(DEV)
    ops.kv_append(g.k, g.v, g.kv_cache, g.block_table, g.context_lens)
    torch.cuda.synchronize()
    assert torch.equal(_bits(g.kv_cache.cpu()), _bits(want))


def _varlen_parity(case):
    want = case.kv_cache.clone()
    paged_ref.write_kv(case.k, case.v, want, case.block_table, case.cu_seqlens, case.context_lens)
    g = case.to(DEV)
    ops.write_kv(g.k, g.v, g.kv_cache, g.block_table, g.cu_seqlens, g.context_lens)
    torch.cuda.synchronize()
    assert torch.equal(_bits(g.kv_cache.cpu()), _bits(want))


@pytest.mark.parametrize("cfg", ["qwen2-0.5b-decode", "llama3-8b-decode"])
def test_decode_append_named_cases(cfg):
    _decode_parity(wl.config_case(cfg))


def test_decode_append_block_edges():
    # positions 0, 15, 16, 17, 31, 32 straddle block boundaries
    _decode_parity(wl.decode_case(wl.LLAMA3_8B, [0, 15, 16, 17, 31, 32, 1000], seed=101))
    _decode_parity(wl.decode_case(wl.QWEN2_05B, [0, 15, 16, 17, 31, 32, 1000], seed=102))


def test_varlen_append_qwen2_7b_prefill():
    _varlen_parity(wl.config_case("qwen2-7b-prefill"))


def test_varlen_append_prefix_and_empty_seqs():
    case = wl.prefill_case(wl.QWEN2_7B, [5, 0, 33, 17, 1, 0], seed=103,
                           ctx_lens=[0, 3, 14, 16, 100, 0])
    _varlen_parity(case)


def test_varlen_append_clamp_overflow():
    # One-column tables: positions past W*bs fold into the last column (attention.py:235).
    # Contexts are chosen so the folded slots are distinct (the reference leaves the
    # order of duplicate-slot writes unspecified).
    case = wl.prefill_case(wl.QWEN2_05B, [3, 5], seed=104, ctx_lens=[16, 40])
    case.block_table = case.block_table[:, :1].contiguous()
    _varlen_parity(case)


def test_append_strided_kv_views():
    # k and v as views into one fused projection output [T, 3 * Hkv * D]
    shape = wl.LLAMA3_8B
    case = wl.prefill_case(shape, [7, 40, 16], seed=105)
    t, hkv, d = case.k.shape
    fused = torch.randn((t, 3 * hkv * d)).to(torch.bfloat16)
    k = fused[:, hkv * d:2 * hkv * d].view(t, hkv, d)
    v = fused[:, 2 * hkv * d:].view(t, hkv, d)
    want = case.kv_cache.clone()
    paged_ref.write_kv(k, v, want, case.block_table, case.cu_seqlens, case.context_lens)
    g = case.to(DEV)
    fg = fused.to(DEV)
    kg = fg[:, hkv * d:2 * hkv * d].view(t, hkv, d)
    vg = fg[:, 2 * hkv * d:].view(t, hkv, d)
    ops.write_kv(kg, vg, g.kv_cache, g.block_table, g.cu_seqlens, g.context_lens)
    torch.cuda.synchronize()
    assert torch.equal(_bits(g.kv_cache.cpu()), _bits(want))


def test_append_fp16_pool():
    case = wl.prefill_case(wl.QWEN2_05B, [12, 30], seed=106, dtype=torch.float16)
    _varlen_parity(case)


def test_decode_append_allocator_tables():
    ctx = [1024, 5000, 77, 2049, 16, 3000]
    _decode_parity(wl.decode_case(wl.LLAMA3_8B, ctx, seed=107, table="allocator"))


def test_varlen_append_many_tokens_odd_rows_and_skips():
    """Enough tokens for 4 tokens per wave: 3 kv heads of head_dim 72 (27 16-byte chunks
    per row, 81 per token: not a multiple of the 64 lanes), a cached prefix, an empty
    sequence, two invalid block ids (their tokens are skipped, as the decode kernels skip
    such blocks) and 7 rows after the packed batch (never written)."""
    shape = wl.HeadShape(6, 3, 72)
    case = wl.prefill_case(shape, [1500, 0, 2049, 777, 3], seed=108,
                           ctx_lens=[0, 5, 17, 1024, 0])
    nb = case.kv_cache.shape[1]
    bt = case.block_table.clone()
    bt[0, 10] = -3
    bt[2, 50] = nb + 7
    t, hkv, d = case.k.shape
    assert t >= 4096
    extra_k = torch.randn((7, hkv, d)).to(case.k.dtype)
    extra_v = torch.randn((7, hkv, d)).to(case.v.dtype)
    want = case.kv_cache.clone()
    phys, off = paged_ref.slot_of_tokens(bt, case.cu_seqlens, case.context_lens, 16)
    ok = (phys >= 0) & (phys < nb)
    assert int((~ok).sum()) == 32
    for h in range(hkv):
        want[0, phys[ok], h, off[ok]] = case.k[ok, h]
        want[1, phys[ok], h, off[ok]] = case.v[ok, h]
    g = case.to(DEV)
    kg = torch.cat([g.k, extra_k.to(DEV)])
    vg = torch.cat([g.v, extra_v.to(DEV)])
    ops.write_kv(kg, vg, g.kv_cache, bt.to(DEV), g.cu_seqlens, g.context_lens)
    torch.cuda.synchronize()
    assert torch.equal(_bits(g.kv_cache.cpu()), _bits(want))


@pytest.mark.parametrize("num_seqs", [63, 64, 150])
def test_varlen_append_batch_sizes_around_the_ballot_lookup(num_seqs):
    """Up to 63 packed sequences find their tokens' sequences with one vector load of
    cu_seqlens and a ballot; 64 and more take the binary search.  Empty prompts and cached
    prefixes sit at the ends and in the middle of the batch."""
    rng = np.random.default_rng(110 + num_seqs)
    lens = rng.integers(0, 40, size=num_seqs)
    lens[[0, num_seqs // 2, num_seqs - 1]] = [0, 0, 0]
    ctx = rng.integers(0, 50, size=num_seqs)
    case = wl.prefill_case(wl.QWEN2_7B, lens.tolist(), seed=110 + num_seqs, ctx_lens=ctx.tolist())
    _varlen_parity(case)
