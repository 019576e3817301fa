"""GPU parity of ndl_paged_decode_append_noalloc against ndl_paged_decode_append.

The allocation-free entry point runs the same kernels with its split-K partials in a
static device array instead of a caller workspace, so its output and the cache bytes it
leaves must equal the workspace entry point's bit for bit.  Two calls in a row share the
array: the second, smaller call must not see anything the first one left there.  Both
entry points are called through the C ABI (ctypes), with torch only holding the device
memory.
"""
import ctypes

import pytest
import torch

from needle_amd import _lib, ops, workloads as wl

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _call(lib, case, use_static, part=0):
    """(out, pool) after one decode step (append + attention) of `case` on the GPU."""
    s = case.shape
    g = case.to(DEV)
    b, w = g.num_seqs, g.block_table.shape[1]
    out = torch.empty((b, s.num_heads, s.head_dim), dtype=torch.bfloat16, device=DEV)
    stream = torch.cuda.current_stream().cuda_stream
    common_head = (out.data_ptr(), g.q.data_ptr(), s.num_heads * s.head_dim,
                   g.k.data_ptr(), s.num_kv_heads * s.head_dim,
                   g.v.data_ptr(), s.num_kv_heads * s.head_dim,
                   g.kv_cache.data_ptr(), g.num_blocks,
                   g.block_table.data_ptr(), g.block_table.stride(0), w,
                   g.context_lens.data_ptr(), b, s.num_heads, s.num_kv_heads, s.head_dim,
                   s.block_size, _lib.NDL_DTYPE_BF16, ctypes.c_float(s.scale), part)
    if use_static:
        rc = lib.ndl_paged_decode_append_noalloc(*common_head, stream)
        _lib.check(rc, "ndl_paged_decode_append_noalloc")
    else:
        need = int(lib.ndl_paged_decode_workspace_bytes(b, s.num_heads, s.num_kv_heads,
                                                        s.head_dim, w, s.block_size, part))
        assert 0 < need <= _lib.NDL_DECODE_STATIC_SCRATCH_BYTES
        ws = ops.decode_workspace(need, DEV)
        rc = lib.ndl_paged_decode_append(*common_head, ws.data_ptr(), need, stream)
        _lib.check(rc, "ndl_paged_decode_append")
    torch.cuda.synchronize()
    return out.cpu(), g.kv_cache.cpu()


def _same(a, b):
    return torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("part", [0, 1024])
def test_noalloc_equals_workspace_entry_point_twice(part):
    lib = _lib.load()
    big = wl.config_case("llama3-8b-decode")                  # 64 sequences, stream split
    # a smaller second call: 20 sequences whose tables are too wide for the per-sequence
    # workgroups, so the stream split writes partials into the same static array again
    small = wl.decode_case(wl.LLAMA3_8B, list(range(2100, 3000, 45)), seed=77)
    for case in (big, small):
        out_ws, pool_ws = _call(lib, case, use_static=False, part=part)
        out_st, pool_st = _call(lib, case, use_static=True, part=part)
        assert _same(out_ws, out_st), "outputs differ from ndl_paged_decode_append"
        assert _same(pool_ws, pool_st), "cache bytes differ from ndl_paged_decode_append"


def test_noalloc_per_sequence_workgroups():
    """The Qwen2-0.5B decode shape takes the per-sequence workgroups (no partials)."""
    lib = _lib.load()
    case = wl.config_case("qwen2-0.5b-decode")
    out_ws, pool_ws = _call(lib, case, use_static=False)
    out_st, pool_st = _call(lib, case, use_static=True)
    assert _same(out_ws, out_st) and _same(pool_ws, pool_st)


def _args(case, out, part=0):
    s = case.shape
    return (out.data_ptr(), case.q.data_ptr(), s.num_heads * s.head_dim,
            case.k.data_ptr(), s.num_kv_heads * s.head_dim,
            case.v.data_ptr(), s.num_kv_heads * s.head_dim,
            case.kv_cache.data_ptr(), case.num_blocks,
            case.block_table.data_ptr(), case.block_table.stride(0), case.block_table.shape[1],
            case.context_lens.data_ptr(), case.num_seqs, s.num_heads, s.num_kv_heads,
            s.head_dim, s.block_size, _lib.NDL_DTYPE_BF16, ctypes.c_float(s.scale), part)


def test_noalloc_replayed_from_a_graph():
    """The callers this entry point is for capture it.  After one call outside capture (the
    first on the device looks the array up), a captured call is replayed three times, with
    eager work between the replays, and must equal the eager call every time."""
    lib = _lib.load()
    g = wl.config_case("llama3-8b-decode").to(DEV)
    s = g.shape
    out = torch.empty((g.num_seqs, s.num_heads, s.head_dim), dtype=torch.bfloat16, device=DEV)
    _lib.check(lib.ndl_paged_decode_append_noalloc(
        *_args(g, out), torch.cuda.current_stream().cuda_stream), "eager call")
    torch.cuda.synchronize()
    want_out, want_pool = out.clone(), g.kv_cache.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = lib.ndl_paged_decode_append_noalloc(*_args(g, out),
                                                 torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "captured call")
    x = torch.randn(1024, 1024, device=DEV)
    for _ in range(3):
        out.zero_()
        y = x @ x
        graph.replay()
        torch.cuda.synchronize()
        assert _same(out, want_out) and _same(g.kv_cache, want_pool)
        del y
