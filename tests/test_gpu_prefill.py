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


# Group sizes 1..9 and 16: a workgroup's eight (head, 32-row subtile) jobs span one subtile
# (g = 8, 16), two (g = 4 .. 7, 9) or more (g = 1, 2, 3), with subtile boundaries at every
# offset inside the eight.
@pytest.mark.parametrize("shape", [
    wl.QWEN2_7B, wl.LLAMA3_8B, wl.QWEN2_05B, wl.HeadShape(8, 8, 128), wl.HeadShape(16, 2, 128),
    wl.HeadShape(8, 1, 64), wl.HeadShape(12, 4, 64), wl.HeadShape(16, 1, 128),
    wl.HeadShape(18, 2, 64), wl.HeadShape(4, 2, 128), wl.HeadShape(10, 2, 128),
    wl.HeadShape(12, 2, 64)])
def test_shapes_and_edge_lengths(shape):
    lens = [1, 15, 16, 17, 31, 32, 33, 127, 128, 129, 300]
    case = wl.prefill_case(shape, lens, seed=301)
    got, _ = run_gpu(case)
    want, _ = oracle(case)
    assert_close(got, want)


@pytest.mark.parametrize("shape", [wl.QWEN2_7B, wl.QWEN2_05B])
def test_empty_prompts_between_real_ones(shape):
    """Zero-length prompts (equal consecutive cu_seqlens entries) at the start, in the middle
    and at the end of the batch own no rows and no tile; the prompts around them attend only
    their own blocks, and the pool matches the oracle's append byte for byte."""
    case = wl.prefill_case(shape, [0, 17, 0, 0, 300, 0, 33, 0], seed=310)
    got, pool = run_gpu(case)
    want, want_pool = oracle(case)
    assert torch.equal(pool.view(torch.int16), want_pool.view(torch.int16))
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


def masked_prefill_fp64(case, bt, pool):
    """fp64 causal attention reading every position of pool (after the append) through bt;
    keys in a block whose id is outside [0, num_blocks) are dropped (a row with no key left
    is zero).  Vectorised per (sequence, kv head), for the longer and more numerous prompts
    below; it agrees with closed_form.prefill_fp64 to 1e-15 where both apply."""
    s = case.shape
    pool = pool.double().numpy()
    nb = pool.shape[1]
    qn = case.q.double().numpy()
    btl = bt.tolist()
    cu = case.cu_seqlens.tolist()
    ctx = case.context_lens.tolist()
    out = np.zeros(qn.shape)
    for i in range(len(cu) - 1):
        n, c = cu[i + 1] - cu[i], ctx[i]
        if n == 0:
            continue
        w = len(btl[i])
        pos = np.arange(c + n)
        ids = np.array([btl[i][min(p // 16, w - 1)] for p in range(c + n)])
        valid = (ids >= 0) & (ids < nb)
        safe = np.where(valid, ids, 0)
        mask = (pos[None, :] <= (c + np.arange(n))[:, None]) & valid[None, :]
        for kvh in range(s.num_kv_heads):
            kr = pool[0, safe, kvh, pos % 16]
            vr = pool[1, safe, kvh, pos % 16]
            for h in range(kvh * s.group, (kvh + 1) * s.group):
                sc = qn[cu[i]:cu[i + 1], h] @ kr.T * s.scale
                sc = np.where(mask, sc, -np.inf)
                mx = sc.max(axis=1, keepdims=True)
                pr = np.where(mask, np.exp(sc - np.where(np.isfinite(mx), mx, 0.0)), 0.0)
                den = pr.sum(axis=1, keepdims=True)
                out[cu[i]:cu[i + 1], h] = np.where(den > 0, (pr @ vr) / np.where(den > 0, den, 1), 0)
    return out


@pytest.mark.parametrize("shape", [wl.QWEN2_7B, wl.LLAMA3_8B])
def test_long_prompts_after_cached_prefixes_vs_fp64(shape):
    """Long cached prefixes (not multiples of the 32-key step) in front of long prompts: the
    unmasked steady-state trips start at the context, cross several 64-block table windows
    and hand over to the masked steps at each tile's diagonal."""
    lens, ctx = [300, 77, 33, 129], [1000, 2100, 31, 0]
    case = wl.prefill_case(shape, lens, seed=306, ctx_lens=ctx)
    got, pool = run_gpu(case, max_ctx=max(ctx))
    _, want_pool = oracle(case)
    assert torch.equal(pool.view(torch.int16), want_pool.view(torch.int16))
    assert_close(got, masked_prefill_fp64(case, case.block_table, pool))


def test_invalid_block_deep_in_long_prompts():
    """An invalid id far into a long prompt (after a table-window refill) ends the steady-state
    trips; one early in another prompt keeps them from starting.  Keys in those blocks drop
    out; every other key is attended."""
    shape = wl.QWEN2_7B
    case = wl.prefill_case(shape, [1500, 600, 1100], seed=307)
    nb = case.kv_cache.shape[1]
    bt = case.block_table.clone()
    bt[0, 70] = -5          # positions 1120..1135 (table window 1)
    bt[1, 5] = nb + 3       # positions 80..95
    bt[2, 64] = -1          # positions 1024..1039: the first block of window 1
    case.block_table = bt
    got, pool = run_gpu(case)
    assert_close(got, masked_prefill_fp64(case, bt, pool))


@pytest.mark.parametrize("shape", [wl.QWEN2_7B, wl.QWEN2_05B])
def test_many_prompts_tile_walk(shape):
    """150 prompts: the persistent walk's sequence search spans three 64-lane chunks."""
    lens = np.random.default_rng(308).integers(1, 120, size=150).tolist()
    case = wl.prefill_case(shape, lens, seed=308)
    got, pool = run_gpu(case)
    assert_close(got, masked_prefill_fp64(case, case.block_table, pool))


def test_one_workgroup_per_tile_beyond_the_tile_list():
    """More than 8192 prompts: the tile list would not fit in LDS, so the kernel launches one
    workgroup per tile instead of the persistent walk."""
    shape = wl.HeadShape(8, 1, 64)
    lens = np.random.default_rng(309).integers(1, 4, size=8200).tolist()
    case = wl.prefill_case(shape, lens, seed=309)
    got, pool = run_gpu(case)
    _, want_pool = oracle(case)
    assert torch.equal(pool.view(torch.int16), want_pool.view(torch.int16))
    assert_close(got, masked_prefill_fp64(case, case.block_table, pool))
