"""GPU parity of ndl_varlen_prefill (after ndl_kv_append) against the oracle.

Tolerance (bf16 in/out, fp32 accumulation): |gpu - ref| <= 2e-2 + 1e-2 |ref|.
With context 0 the reference is _prefill_pytorch (attention.py:120-134, torch
SDPA on the fresh k/v); with a cached prefix the reference has no counterpart
(it ignores the prefix), so that case is checked against the fp64 closed form
that reads every position through block_table.
"""
import numpy as np
import pytest
import torch

from oracle import closed_form, paged_ref
from needle_amd import ops, workloads as wl

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
ATOL, RTOL = 2e-2, 1e-2


def assert_close(got, want, atol=ATOL, rtol=RTOL):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape
    assert np.isfinite(got).all()
    excess = np.abs(got - want) - (atol + rtol * np.abs(want))
    worst = np.unravel_index(np.argmax(excess), excess.shape)
    assert excess.max() <= 0, (
        f"max |diff| {np.abs(got - want).max():.4g} at {worst}: "
        f"got {got[worst]:.5g} want {want[worst]:.5g}")


def run_gpu(case, max_ctx=0):
    g = case.to(DEV)
    s = case.shape
    ops.write_kv(g.k, g.v, g.kv_cache, g.block_table, g.cu_seqlens, g.context_lens)
    out = ops.varlen_prefill(g.q, g.kv_cache, g.block_table, g.cu_seqlens, g.context_lens,
                             case.max_seqlen, s.scale, s.num_heads, s.num_kv_heads, s.head_dim,
                             max_context_len=max_ctx)
    torch.cuda.synchronize()
    return out.float().cpu(), g.kv_cache.cpu()


def oracle(case):
    s = case.shape
    pool = case.kv_cache.clone()
    out = paged_ref.prefill(case.q, case.k, case.v, pool, case.block_table, case.cu_seqlens,
                            case.context_lens, s.num_heads, s.num_kv_heads)
    return out.float(), pool


def test_qwen2_7b_prefill_vs_oracle():
    case = wl.config_case("qwen2-7b-prefill")
    got, pool = run_gpu(case)
    want, want_pool = oracle(case)
    assert torch.equal(pool.view(torch.int16), want_pool.view(torch.int16))
    assert_close(got, want)


def test_qwen2_7b_prefill_sampled_rows_vs_fp64():
    case = wl.config_case("qwen2-7b-prefill")
    got, pool = run_gpu(case)
    s = case.shape
    # fp64 closed form on a sample of sequences: the two shortest and two longest prompts
    order = np.argsort(case.new_lens)
    pick = sorted(set(order[:2].tolist() + order[-2:].tolist()))
    cu = case.cu_seqlens.tolist()
    for i in pick:
        sub = slice(cu[i], cu[i + 1])
        sub_cu = torch.tensor([0, cu[i + 1] - cu[i]], dtype=torch.int32)
        want = closed_form.prefill_fp64(case.q[sub], pool, case.block_table[i:i + 1], sub_cu,
                                        case.context_lens[i:i + 1], s.scale, s.num_heads,
                                        s.num_kv_heads)
        assert_close(got[sub], want)


@pytest.mark.parametrize("shape", [
    wl.QWEN2_7B, wl.LLAMA3_8B, wl.QWEN2_05B, wl.HeadShape(8, 8, 128), wl.HeadShape(16, 2, 128),
    wl.HeadShape(8, 1, 64), wl.HeadShape(12, 4, 64), wl.HeadShape(16, 1, 128),
    wl.HeadShape(18, 2, 64)])
def test_shapes_and_edge_lengths(shape):
    lens = [1, 15, 16, 17, 31, 32, 33, 127, 128, 129, 300]
    case = wl.prefill_case(shape, lens, seed=301)
    got, _ = run_gpu(case)
    want, _ = oracle(case)
    assert_close(got, want)


def test_single_token_prompts_return_value_rows():
    shape = wl.QWEN2_7B
    case = wl.prefill_case(shape, [1, 1, 1], seed=302)
    got, _ = run_gpu(case)
    g = shape.group
    for h in range(shape.num_heads):
        assert torch.equal(got[:, h], case.v[:, h // g].float())


def test_cached_prefix_vs_fp64():
    shape = wl.QWEN2_7B
    lens, ctx = [5, 40, 130, 1], [16, 3, 100, 250]
    case = wl.prefill_case(shape, lens, seed=303, ctx_lens=ctx)
    got, pool = run_gpu(case, max_ctx=max(ctx))
    s = case.shape
    want = closed_form.prefill_fp64(case.q, pool, case.block_table, case.cu_seqlens,
                                    case.context_lens, s.scale, s.num_heads, s.num_kv_heads)
    assert_close(got, want)


def test_allocator_tables_and_many_prompts():
    shape = wl.QWEN2_05B
    lens = np.random.default_rng(304).integers(1, 400, size=40).tolist()
    case = wl.prefill_case(shape, lens, seed=304, table="allocator")
    got, _ = run_gpu(case)
    want, _ = oracle(case)
    assert_close(got, want)


def test_invalid_block_ids_are_masked():
    """A block id outside [0, num_blocks) is never dereferenced: append skips its rows and
    attention drops its keys (a row left with no valid key returns zeros)."""
    shape = wl.QWEN2_7B
    case = wl.prefill_case(shape, [40, 70, 20], seed=305)
    nb = case.kv_cache.shape[1]
    bt = case.block_table.clone()
    bt[0, 1] = -3          # positions 16..31 of prompt 0
    bt[1, 2] = nb + 7      # positions 32..47 of prompt 1
    bt[2, 0] = -1          # positions 0..15 of prompt 2: rows 0..15 see no valid key
    case.block_table = bt
    got, pool = run_gpu(case)
    s = case.shape
    g = s.group
    kvn = pool.double().numpy()
    qn = case.q.double().numpy()
    btl = bt.tolist()
    cu = case.cu_seqlens.tolist()
    want = np.zeros(got.shape)
    for i in range(len(cu) - 1):
        w = len(btl[i])
        for t in range(cu[i], cu[i + 1]):
            p = t - cu[i]
            keys = [j for j in range(p + 1) if 0 <= btl[i][min(j // 16, w - 1)] < nb]
            for h in range(s.num_heads):
                if not keys:
                    continue
                kvh = h // g
                kr = np.stack([kvn[0, btl[i][min(j // 16, w - 1)], kvh, j % 16] for j in keys])
                vr = np.stack([kvn[1, btl[i][min(j // 16, w - 1)], kvh, j % 16] for j in keys])
                sc = kr @ qn[t, h] * s.scale
                pr = np.exp(sc - sc.max())
                want[t, h] = pr @ vr / pr.sum()
    assert_close(got, want)
