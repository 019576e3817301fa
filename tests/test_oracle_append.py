"""Pins the oracle's append (slot rule + scatter) on the CPU.

Checks: brute-force element loop, hand-computed known answers, the column
clamp (attention.py:144, :235), empty sequences, and that no slot outside
the written ones changes.
"""
import torch

from oracle import closed_form, paged_ref
from needle_amd import workloads as wl


def _tiny_pool(nb=9, hkv=2, bs=16, d=8, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn((2, nb, hkv, bs, d), generator=g).to(torch.bfloat16)


def test_known_answer_decode_slot():
    # block_table row [5, 2], ctx 17 -> position 17 -> column 1 -> block 2, offset 1.
    pool = _tiny_pool()
    before = pool.clone()
    k = torch.full((1, 2, 8), 3.0, dtype=torch.bfloat16)
    v = torch.full((1, 2, 8), -7.0, dtype=torch.bfloat16)
    bt = torch.tensor([[5, 2]], dtype=torch.int32)
    paged_ref.decode_append(k, v, pool, bt, torch.tensor([17], dtype=torch.int32))
    assert torch.equal(pool[0, 2, :, 1], k[0])
    assert torch.equal(pool[1, 2, :, 1], v[0])
    changed = (pool.view(torch.int16) != before.view(torch.int16)).any(dim=-1)
    assert int(changed.sum()) == 2 * 2  # 2 planes x 2 kv heads, nothing else


def test_known_answer_clamp():
    # W = 1 and ctx 20: column min(20 // 16, 0) = 0 -> block 3, offset 20 % 16 = 4.
    pool = _tiny_pool()
    k = torch.full((1, 2, 8), 1.5, dtype=torch.bfloat16)
    v = torch.full((1, 2, 8), 2.5, dtype=torch.bfloat16)
    bt = torch.tensor([[3]], dtype=torch.int32)
    paged_ref.decode_append(k, v, pool, bt, torch.tensor([20], dtype=torch.int32))
    assert torch.equal(pool[0, 3, :, 4], k[0]) and torch.equal(pool[1, 3, :, 4], v[0])


def test_varlen_matches_bruteforce():
    g = torch.Generator().manual_seed(3)
    hkv, d, nb, bs = 2, 8, 40, 16
    pool = _tiny_pool(nb=nb, hkv=hkv, d=d, seed=4)
    seq_lens = [5, 0, 33, 17]
    ctx = [0, 3, 14, 16]
    blocks = [max(1, (c + n + bs - 1) // bs) for c, n in zip(ctx, seq_lens)]
    tables = wl.tables_by_permutation(blocks, nb, seed=5)
    bt = wl.pad_tables(tables, nb)
    t = sum(seq_lens)
    k = torch.randn((t, hkv, d), generator=g).to(torch.bfloat16)
    v = torch.randn((t, hkv, d), generator=g).to(torch.bfloat16)
    cu = torch.tensor([0, 5, 5, 38, 55], dtype=torch.int32)
    ctx_t = torch.tensor(ctx, dtype=torch.int32)
    want = closed_form.append_bruteforce(k, v, pool, bt, cu, ctx_t)
    got = pool.clone()
    paged_ref.write_kv(k, v, got, bt, cu, ctx_t)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_varlen_clamped_overflow_matches_bruteforce():
    # A one-column table: positions 16..18 fold into offsets 0..2 of the only block.
    hkv, d, nb = 1, 8, 6
    pool = _tiny_pool(nb=nb, hkv=hkv, d=d, seed=6)
    g = torch.Generator().manual_seed(7)
    k = torch.randn((3, hkv, d), generator=g).to(torch.bfloat16)
    v = torch.randn((3, hkv, d), generator=g).to(torch.bfloat16)
    bt = torch.tensor([[4]], dtype=torch.int32)
    cu = torch.tensor([0, 3], dtype=torch.int32)
    ctx = torch.tensor([16], dtype=torch.int32)
    want = closed_form.append_bruteforce(k, v, pool, bt, cu, ctx)
    got = pool.clone()
    paged_ref.write_kv(k, v, got, bt, cu, ctx)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    assert torch.equal(got[0, 4, 0, 0], k[0, 0]) and torch.equal(got[1, 4, 0, 2], v[2, 0])


def test_decode_append_matches_bruteforce():
    case = wl.decode_case(wl.QWEN2_05B, [32, 0, 15, 16, 511, 100], seed=11, num_blocks=80)
    want = closed_form.append_bruteforce(case.k, case.v, case.kv_cache, case.block_table, None,
                                         case.context_lens)
    got = case.kv_cache.clone()
    paged_ref.decode_append(case.k, case.v, got, case.block_table, case.context_lens)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_slot_rule_agrees_between_forms():
    # decode append == write_kv with cu_seqlens = arange(B + 1)
    case = wl.decode_case(wl.LLAMA3_8B, [7, 64, 1000, 15], seed=12)
    a = case.kv_cache.clone()
    b = case.kv_cache.clone()
    paged_ref.decode_append(case.k, case.v, a, case.block_table, case.context_lens)
    cu = torch.arange(case.num_seqs + 1, dtype=torch.int32)
    paged_ref.write_kv(case.k, case.v, b, case.block_table, cu, case.context_lens)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
