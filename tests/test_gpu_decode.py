"""GPU parity of ndl_paged_decode against the oracle.

Tolerance (bf16 in/out, fp32 accumulation): |gpu - ref| <= 2e-2 + 1e-2 |ref|,
against both the reference restatement (bf16 op for op) and the fp64 closed
form.  The append that precedes attention in _decode (attention.py:141-154)
runs first on both sides.
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


def run_gpu(case, partition_tokens=0):
    g = case.to(DEV)
    s = case.shape
    ops.kv_append(g.k, g.v, g.kv_cache, g.block_table, g.context_lens)
    out = ops.paged_decode(g.q, g.kv_cache, g.block_table, g.context_lens, s.scale,
                           s.num_heads, s.num_kv_heads, s.head_dim,
                           partition_tokens=partition_tokens)
    torch.cuda.synchronize()
    return out.float().cpu(), g


def run_oracle(case):
    s = case.shape
    pool = case.kv_cache.clone()
    out = paged_ref.decode(case.q, case.k, case.v, pool, case.block_table, case.context_lens,
                           s.scale, s.num_heads, s.num_kv_heads, s.head_dim)
    return out.float(), pool


# partition_tokens: 0 automatic, -1 one 8-wave workgroup per (kv head, sequence), > 0 the
# stream split with partition_tokens / 16 stream slots per wave (16 tokens each; every
# sequence starts with one empty slot, so at 16 some waves hold no tile at all).
@pytest.mark.parametrize("part", [0, -1, 256])
@pytest.mark.parametrize("cfg", ["qwen2-0.5b-decode", "llama3-8b-decode"])
def test_decode_named_cases_vs_oracle(cfg, part):
    case = wl.config_case(cfg)
    got, _ = run_gpu(case, partition_tokens=part)
    want, pool = run_oracle(case)
    assert_close(got, want)
    s = case.shape
    ref64 = closed_form.decode_fp64(case.q, pool, case.block_table, case.context_lens, s.scale,
                                    s.num_heads, s.num_kv_heads)
    assert_close(got, ref64)


@pytest.mark.parametrize("part", [-1, 16, 64, 256, 512, 1024])
def test_partition_sizes_agree(part):
    case = wl.decode_case(wl.LLAMA3_8B, [0, 15, 16, 255, 256, 257, 1023, 3000], seed=201)
    got, _ = run_gpu(case, partition_tokens=part)
    want, _ = run_oracle(case)
    assert_close(got, want)


@pytest.mark.parametrize("shape", [
    wl.HeadShape(8, 8, 128), wl.HeadShape(16, 8, 128), wl.HeadShape(28, 4, 128),
    wl.HeadShape(64, 8, 128), wl.HeadShape(16, 1, 128), wl.HeadShape(4, 4, 64),
    wl.HeadShape(14, 2, 64), wl.HeadShape(12, 3, 64), wl.HeadShape(32, 2, 64)])
@pytest.mark.parametrize("part", [-1, 64])
def test_group_sizes_and_head_dims(shape, part):
    case = wl.decode_case(shape, [0, 1, 17, 100, 600], seed=202)
    got, _ = run_gpu(case, partition_tokens=part)
    want, _ = run_oracle(case)
    assert_close(got, want)


@pytest.mark.parametrize("part", [-1, 16])
def test_single_token_context_is_exact_value_row(part):
    case = wl.decode_case(wl.QWEN2_7B, [0, 0, 0, 0], seed=203)
    got, _ = run_gpu(case, partition_tokens=part)
    g = case.shape.group
    for h in range(case.shape.num_heads):
        assert torch.equal(got[:, h], case.v[:, h // g].float())


@pytest.mark.parametrize("part", [-1, 16])
def test_row_width_cap(part):
    # context 39 but two table columns: 32 tokens attended, like the reference slice
    # (every slot finite: no append runs here, so the attended slots are pre-filled)
    case = wl.decode_case(wl.LLAMA3_8B, [31, 20], seed=204, garbage=False)
    case.context_lens = torch.tensor([39, 20], dtype=torch.int32)
    case.ctx = [39, 20]
    s = case.shape
    g = case.to(DEV)
    out = ops.paged_decode(g.q, g.kv_cache, g.block_table, g.context_lens, s.scale,
                           s.num_heads, s.num_kv_heads, s.head_dim, partition_tokens=part)
    torch.cuda.synchronize()
    want = paged_ref.decode_pytorch(case.q, case.kv_cache, case.block_table, case.context_lens,
                                    s.scale, s.num_heads, s.num_kv_heads, s.head_dim)
    assert_close(out.float().cpu(), want.float())


def test_fragmented_long_context_sampled():
    # long-context style tables at reduced batch: allocator churn, contexts up to 32k
    ctx = [1024, 32768, 8192, 4097, 20000, 1500]
    case = wl.decode_case(wl.LLAMA3_8B, ctx, seed=205, table="allocator")
    got, _ = run_gpu(case)
    want, _ = run_oracle(case)
    assert_close(got, want)


def test_repeat_calls_are_deterministic():
    case = wl.config_case("qwen2-0.5b-decode")
    a, g = run_gpu(case)
    s = case.shape
    b = ops.paged_decode(g.q, g.kv_cache, g.block_table, g.context_lens, s.scale,
                         s.num_heads, s.num_kv_heads, s.head_dim).float().cpu()
    assert torch.equal(a, b)


@pytest.mark.parametrize("part", [-1, 16, 256])
def test_empty_contexts_give_zeros_between_live_ones(part):
    # context_lens + 1 <= 0: nothing to attend (the reference's empty softmax gives zeros);
    # the neighbours' tiles share the waves those sequences would sit between
    case = wl.decode_case(wl.LLAMA3_8B, [40, 3, 700, 0, 90], seed=206, garbage=False)
    case.context_lens = torch.tensor([40, -1, 700, -5, 90], dtype=torch.int32)
    case.ctx = [40, -1, 700, -5, 90]
    s = case.shape
    g = case.to(DEV)
    out = ops.paged_decode(g.q, g.kv_cache, g.block_table, g.context_lens, s.scale,
                           s.num_heads, s.num_kv_heads, s.head_dim, partition_tokens=part)
    torch.cuda.synchronize()
    got = out.float().cpu()
    assert torch.equal(got[1], torch.zeros_like(got[1]))
    assert torch.equal(got[3], torch.zeros_like(got[3]))
    live = [0, 2, 4]
    want = paged_ref.decode_pytorch(case.q[live], case.kv_cache, case.block_table[live],
                                    case.context_lens[live], s.scale, s.num_heads,
                                    s.num_kv_heads, s.head_dim)
    assert_close(got[live], want.float())


@pytest.mark.parametrize("part", [-1, 64])
def test_invalid_block_ids_are_skipped(part):
    """A block id outside [0, num_blocks) is never dereferenced: its keys are dropped."""
    shape = wl.LLAMA3_8B
    case = wl.decode_case(shape, [100, 300], seed=207, garbage=False)
    nb = case.kv_cache.shape[1]
    bt = case.block_table.clone()
    bt[0, 2] = -4          # tokens 32..47 of sequence 0
    bt[1, 5] = nb + 3      # tokens 80..95 of sequence 1
    case.block_table = bt
    s = case.shape
    g = case.to(DEV)
    out = ops.paged_decode(g.q, g.kv_cache, g.block_table, g.context_lens, s.scale,
                           s.num_heads, s.num_kv_heads, s.head_dim, partition_tokens=part)
    torch.cuda.synchronize()
    kvn = case.kv_cache.double().numpy()
    qn = case.q.double().numpy()
    btl = bt.tolist()
    want = np.zeros(out.shape)
    for i, ctx in enumerate(case.ctx):
        keys = [p for p in range(ctx + 1) if 0 <= btl[i][p // 16] < nb]
        for h in range(s.num_heads):
            kvh = h // s.group
            kr = np.stack([kvn[0, btl[i][p // 16], kvh, p % 16] for p in keys])
            vr = np.stack([kvn[1, btl[i][p // 16], kvh, p % 16] for p in keys])
            sc = kr @ qn[i, h] * s.scale
            pr = np.exp(sc - sc.max())
            want[i, h] = pr @ vr / pr.sum()
    assert_close(out.float().cpu(), want)


def test_one_workspace_across_calls_and_batch_sizes():
    """Sequences split over several waves leave partials in the workspace for the merge.
    One workspace serves a small batch, then a larger one, then both again, and a foreign
    workspace full of other bytes: every output equals that of a call with a fresh
    workspace."""
    s = wl.LLAMA3_8B
    small = wl.decode_case(s, [5000, 7000, 3000], seed=208).to(DEV)
    large = wl.decode_case(s, [300, 4100, 17, 2500, 9000, 64, 1200, 6000, 0, 800], seed=209)
    want_large, _ = run_oracle(large)
    large = large.to(DEV)
    for c in (small, large):
        ops.kv_append(c.k, c.v, c.kv_cache, c.block_table, c.context_lens)

    def call(c, ws=None):
        out = ops.paged_decode(c.q, c.kv_cache, c.block_table, c.context_lens, s.scale,
                               s.num_heads, s.num_kv_heads, s.head_dim, workspace=ws)
        return out.float().cpu()

    ref_small, ref_large = call(small), call(large)
    assert_close(ref_large, want_large)
    need = max(ops.decode_workspace_bytes(c.q.shape[0], s.num_heads, s.num_kv_heads,
                                          s.head_dim, c.block_table.shape[1])
               for c in (small, large))
    ws = ops.decode_workspace(need, DEV)
    for c, ref in ((small, ref_small), (large, ref_large), (small, ref_small),
                   (large, ref_large), (large, ref_large)):
        assert torch.equal(call(c, ws), ref)
    foreign = torch.full((need,), 0x5A, dtype=torch.uint8, device=DEV)
    assert torch.equal(call(large, foreign), ref_large)
    assert torch.equal(call(small, foreign), ref_small)


def test_graph_replays_of_two_batch_sizes_share_a_workspace():
    """Captured decodes of 10, 3 and 4 sequences (largest first, as the runner captures
    its buckets; the last one short enough for the per-sequence workgroups) on one
    workspace, replayed in mixed order with eager calls on the same workspace in between:
    every replay equals the eager output."""
    s = wl.LLAMA3_8B
    large = wl.decode_case(s, [300, 4100, 17, 2500, 9000, 64, 1200, 6000, 0, 800],
                           seed=210).to(DEV)
    small = wl.decode_case(s, [5000, 7000, 3000], seed=211).to(DEV)
    tiny = wl.decode_case(s, [100, 40, 300, 1], seed=212).to(DEV)
    cases = (large, small, tiny)
    for c in cases:
        ops.kv_append(c.k, c.v, c.kv_cache, c.block_table, c.context_lens)

    def call(c, ws=None):
        return ops.paged_decode(c.q, c.kv_cache, c.block_table, c.context_lens, s.scale,
                                s.num_heads, s.num_kv_heads, s.head_dim, workspace=ws)

    refs = {id(c): call(c).float().cpu() for c in cases}
    need = max(ops.decode_workspace_bytes(c.q.shape[0], s.num_heads, s.num_kv_heads,
                                          s.head_dim, c.block_table.shape[1]) for c in cases)
    ws = ops.decode_workspace(need, DEV)
    graphs = {}
    for c in cases:
        call(c, ws)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            out = call(c, ws)
        graphs[id(c)] = (g, out)
    torch.cuda.synchronize()
    order = (small, large, tiny, small, large, large, tiny, small)
    for n, c in enumerate(order):
        g, out = graphs[id(c)]
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.float().cpu(), refs[id(c)])
        other = order[(n + 1) % len(order)]
        assert torch.equal(call(other, ws).float().cpu(), refs[id(other)])


@pytest.mark.parametrize("part", [0, 64])
@pytest.mark.parametrize("nseq", [63, 64, 65, 130])
def test_batch_sizes_around_one_wave_of_sequences(nseq, part):
    """The stream split reads the context lengths with one load up to 64 sequences and
    scans them 64 at a time beyond; both sides of that boundary, with empty sequences at
    the edges of the 64-sequence chunks, against the oracle (the merge walks the same
    lengths)."""
    rng = np.random.default_rng(300 + nseq)
    ctx = rng.integers(0, 600, size=nseq).tolist()
    case = wl.decode_case(wl.LLAMA3_8B, ctx, seed=310 + nseq, garbage=False)
    for i in (0, 63, 64, nseq - 1):
        if i < nseq:
            ctx[i] = -1
    case.context_lens = torch.tensor(ctx, dtype=torch.int32)
    case.ctx = list(ctx)
    s = case.shape
    g = case.to(DEV)
    out = ops.paged_decode(g.q, g.kv_cache, g.block_table, g.context_lens, s.scale,
                           s.num_heads, s.num_kv_heads, s.head_dim, partition_tokens=part)
    torch.cuda.synchronize()
    got = out.float().cpu()
    empty = [i for i in range(nseq) if ctx[i] < 0]
    live = [i for i in range(nseq) if ctx[i] >= 0]
    for i in empty:
        assert torch.equal(got[i], torch.zeros_like(got[i]))
    want = paged_ref.decode_pytorch(case.q[live], case.kv_cache, case.block_table[live],
                                    case.context_lens[live], s.scale, s.num_heads,
                                    s.num_kv_heads, s.head_dim)
    assert_close(got[live], want.float())


@pytest.mark.parametrize("part", [0, -1])
def test_llama_decode_tp8_share(part):
    # One GPU's share of the Llama-3-8B decode under 8-way tensor parallelism (kv heads split
    # across GPUs, attention.py:45-46): 4 query heads over 1 kv head, the configuration's 64
    # sequences and context lengths, fused append.
    shape = wl.HeadShape(4, 1, 128)
    case = wl.decode_case(shape, wl.llama8b_decode_ctx(), seed=1002)
    g = case.to(DEV)
    s = case.shape
    got = ops.paged_decode(g.q, g.kv_cache, g.block_table, g.context_lens, s.scale,
                           s.num_heads, s.num_kv_heads, s.head_dim, partition_tokens=part,
                           new_k=g.k, new_v=g.v)
    torch.cuda.synchronize()
    want, pool = run_oracle(case)
    assert torch.equal(g.kv_cache.cpu().view(torch.int16), pool.view(torch.int16))
    assert_close(got.float().cpu(), want)
