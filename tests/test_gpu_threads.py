"""The entry points called from several host threads at once, each thread on its own stream.

The C ABI keeps no per-call state (the decode workspace comes from the caller; the occupancy
answers behind the automatic launch shapes are cached per device under a lock), and the
ctypes calls release the GIL, so calls that overlap on distinct streams must leave the same
bytes as the same calls made one after another.
"""
import threading

import pytest
import torch

from needle_amd import ops, workloads as wl

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
REPS = 6


def run(kind, g, pristine):
    """One call of `kind` on the current stream over a fresh copy of the pool."""
    s = g.shape
    g.kv_cache.copy_(pristine)
    if kind == "prefill":
        ops.write_kv(g.k, g.v, g.kv_cache, g.block_table, g.cu_seqlens, g.context_lens)
        return ops.varlen_prefill(g.q, g.kv_cache, g.block_table, g.cu_seqlens, g.context_lens,
                                  g.max_seqlen, s.scale, s.num_heads, s.num_kv_heads,
                                  s.head_dim)
    part = {"decode_fused": 0, "decode_split": 64, "decode_groups": -1}[kind]
    return ops.paged_decode(g.q, g.kv_cache, g.block_table, g.context_lens, s.scale,
                            s.num_heads, s.num_kv_heads, s.head_dim, partition_tokens=part,
                            new_k=g.k, new_v=g.v)


def jobs():
    out = []
    for i, kind in enumerate(["decode_fused", "decode_split", "decode_groups"] * 2):
        ctx = [37 * i + 5, 900 + 13 * i, 17, 2000, 300 + i]
        shape = wl.LLAMA3_8B if i % 2 == 0 else wl.HeadShape(14, 2, 64)
        out.append((kind, wl.decode_case(shape, ctx, seed=700 + i)))
    for i in range(2):
        out.append(("prefill", wl.prefill_case(wl.HeadShape(28, 4, 128), [300 + 50 * i, 77, 1000],
                                               seed=720 + i)))
    return out


def test_concurrent_threads_match_serial():
    work = []
    for kind, case in jobs():
        g = case.to(DEV)
        pristine = g.kv_cache.clone()
        want = run(kind, g, pristine)
        torch.cuda.synchronize()
        work.append((kind, g, pristine, want.cpu(), g.kv_cache.cpu()))

    results = [None] * len(work)
    errors = []
    start = threading.Barrier(len(work))

    def worker(idx):
        kind, g, pristine, _, _ = work[idx]
        try:
            stream = torch.cuda.Stream()
            start.wait()
            with torch.cuda.stream(stream):
                outs = [run(kind, g, pristine) for _ in range(REPS)]
            stream.synchronize()
            results[idx] = ([o.cpu() for o in outs], g.kv_cache.cpu())
        except Exception as exc:   # reported by the main thread
            errors.append((idx, kind, repr(exc)))

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(len(work))]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=60)
    assert not any(t.is_alive() for t in threads), "a worker did not finish"
    assert not errors, errors
    for (kind, _, _, want, want_pool), (outs, pool) in zip(work, results):
        assert torch.equal(pool.view(torch.int16), want_pool.view(torch.int16)), kind
        for o in outs:
            assert torch.equal(o.view(torch.int16), want.view(torch.int16)), kind


def test_launch_stream_is_torchs_current_stream():
    """Every entry point launches on the handle ops._stream gives: torch's current stream of
    the calling thread, also inside a `with torch.cuda.stream(...)` block and on a thread of
    its own."""
    dev = torch.device(DEV)
    assert ops._stream(dev) == torch.cuda.current_stream(dev).cuda_stream
    assert ops._stream(torch.device("cuda")) == torch.cuda.current_stream().cuda_stream
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        assert ops._stream(dev) == side.cuda_stream
    assert ops._stream(dev) == torch.cuda.current_stream(dev).cuda_stream
    seen = []

    def worker():
        own = torch.cuda.Stream()
        with torch.cuda.stream(own):
            seen.append(ops._stream(dev) == own.cuda_stream)

    t = threading.Thread(target=worker)
    t.start()
    t.join(timeout=60)
    assert seen == [True]
