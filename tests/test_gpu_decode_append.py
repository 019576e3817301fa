"""GPU parity of ndl_paged_decode_append: the decode append and the paged attention of
Attention._decode (attention.py:141-159) in one launch.

The fused call must leave the same cache bytes and return the same output, bit for bit,
as ndl_kv_append followed by ndl_paged_decode on the same inputs (the new row is attended
from the registers it was stored from, with the values the separate append writes), and
therefore the same tolerance parity against the oracle as the separate pair.
"""
import pytest
import torch

from oracle import paged_ref
from needle_amd import ops, workloads as wl

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def both(case, part=0):
    """(separate out, separate pool, fused out, fused pool) on copies of the same inputs."""
    s = case.shape
    a = case.to(DEV)
    ops.kv_append(a.k, a.v, a.kv_cache, a.block_table, a.context_lens)
    out_a = ops.paged_decode(a.q, a.kv_cache, a.block_table, a.context_lens, s.scale,
                             s.num_heads, s.num_kv_heads, s.head_dim, partition_tokens=part)
    b = case.to(DEV)
    out_b = ops.paged_decode(b.q, b.kv_cache, b.block_table, b.context_lens, s.scale,
                             s.num_heads, s.num_kv_heads, s.head_dim, partition_tokens=part,
                             new_k=b.k, new_v=b.v)
    torch.cuda.synchronize()
    return out_a.cpu(), a.kv_cache.cpu(), out_b.cpu(), b.kv_cache.cpu()


def assert_same(case, part=0):
    out_a, pool_a, out_b, pool_b = both(case, part)
    assert torch.equal(pool_a.view(torch.int16), pool_b.view(torch.int16)), "cache bytes differ"
    assert torch.equal(out_a.view(torch.int16), out_b.view(torch.int16)), "outputs differ"
    return out_b, pool_b


@pytest.mark.parametrize("part", [0, -1, 256])
@pytest.mark.parametrize("cfg", ["qwen2-0.5b-decode", "llama3-8b-decode"])
def test_fused_equals_append_then_decode(cfg, part):
    case = wl.config_case(cfg)
    out, pool = assert_same(case, part)
    s = case.shape
    want_pool = case.kv_cache.clone()
    want = paged_ref.decode(case.q, case.k, case.v, want_pool, case.block_table,
                            case.context_lens, s.scale, s.num_heads, s.num_kv_heads, s.head_dim)
    assert torch.equal(pool.view(torch.int16), want_pool.view(torch.int16))
    diff = (out.float() - want.float()).abs()
    assert (diff <= 2e-2 + 1e-2 * want.float().abs()).all()


@pytest.mark.parametrize("part", [-1, 16, 64, 1024])
def test_every_row_and_tile_boundary(part):
    """New token at rows 0, 15, 0 of a fresh block, 15, 0, 1, 15 ... and at position 0."""
    case = wl.decode_case(wl.LLAMA3_8B, [0, 15, 16, 255, 256, 257, 1023, 3000], seed=401)
    assert_same(case, part)


@pytest.mark.parametrize("shape", [wl.HeadShape(8, 8, 128), wl.HeadShape(28, 4, 128),
                                   wl.HeadShape(16, 1, 128), wl.HeadShape(14, 2, 64),
                                   wl.HeadShape(12, 3, 64)])
@pytest.mark.parametrize("part", [-1, 64])
def test_group_sizes_and_head_dims(shape, part):
    case = wl.decode_case(shape, [0, 1, 17, 100, 600], seed=402)
    assert_same(case, part)


@pytest.mark.parametrize("part", [-1, 16])
def test_table_row_clamp(part):
    """context 39 with two table columns: the append lands in column 1 (clamped) at row
    39 % 16, which the 32 attended tokens include."""
    case = wl.decode_case(wl.LLAMA3_8B, [31, 20], seed=403, garbage=False)
    case.context_lens = torch.tensor([39, 20], dtype=torch.int32)
    case.ctx = [39, 20]
    assert_same(case, part)


@pytest.mark.parametrize("part", [-1, 16, 256])
def test_empty_contexts_and_invalid_last_blocks(part):
    """Negative contexts append nothing and give zeros; an invalid id in a sequence's last
    column skips its append and drops those keys, as the separate calls do."""
    case = wl.decode_case(wl.LLAMA3_8B, [40, 3, 700, 0, 90, 130], seed=404, garbage=False)
    case.context_lens = torch.tensor([40, -1, 700, -5, 90, 130], dtype=torch.int32)
    case.ctx = [40, -1, 700, -5, 90, 130]
    nb = case.kv_cache.shape[1]
    bt = case.block_table.clone()
    bt[4, 90 // 16] = -2
    bt[5, 130 // 16] = nb + 5
    case.block_table = bt
    out, _ = assert_same(case, part)
    assert torch.equal(out[1], torch.zeros_like(out[1]))
    assert torch.equal(out[3], torch.zeros_like(out[3]))


def test_long_fragmented_contexts():
    ctx = [1024, 32768, 8192, 4097, 20000, 1500]
    case = wl.decode_case(wl.LLAMA3_8B, ctx, seed=405, table="allocator")
    assert_same(case)


def test_graph_replays_match_eager():
    """Captured once and replayed three times over a fresh cache each time."""
    case = wl.config_case("llama3-8b-decode")
    s = case.shape
    g = case.to(DEV)
    pristine = g.kv_cache.clone()
    out = torch.empty_like(g.q)
    ws = ops.decode_workspace(ops.decode_workspace_bytes(
        case.num_seqs, s.num_heads, s.num_kv_heads, s.head_dim, g.block_table.shape[1],
        s.block_size, 0), g.q.device)

    def call():
        ops.paged_decode(g.q, g.kv_cache, g.block_table, g.context_lens, s.scale, s.num_heads,
                         s.num_kv_heads, s.head_dim, out=out, workspace=ws,
                         new_k=g.k, new_v=g.v)
    call()
    torch.cuda.synchronize()
    want_out, want_pool = out.clone(), g.kv_cache.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        g.kv_cache.copy_(pristine)
        call()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    for _ in range(3):
        g.kv_cache.copy_(pristine)
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want_out.view(torch.int16))
        # bitwise: unused slots hold NaN patterns
        assert torch.equal(g.kv_cache.view(torch.int16), want_pool.view(torch.int16))
