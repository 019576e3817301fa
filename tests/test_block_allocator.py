"""BlockAllocator: the block-id contract the kernels consume (block_allocator.py:10-124).

Semantics pinned here:
  * ids come out of a FIFO free list: a fresh pool hands out 0, 1, 2, ... and a freed id
    goes to the back of the line;
  * a block leaves the free list with ref_count 1 and returns when it drops to 0;
  * an empty pool raises MemoryError (single and multi-block requests; a multi-block
    request that cannot be met takes nothing);
  * freeing a block that is already free raises AssertionError;
  * swap_out / swap_in move blocks between the pools and return source -> destination maps;
plus the allocator-churned table generator used for the long-context workload.
"""
import random

import pytest

from needle_amd.backend.block_allocator import BlockAllocator
from needle_amd import workloads as wl


def test_fresh_pool_hands_out_ids_in_order():
    a = BlockAllocator(num_gpu_blocks=6, num_cpu_blocks=0, block_size=16)
    assert [a.allocate_gpu() for _ in range(3)] == [0, 1, 2]
    assert a.allocate_gpu_blocks(3) == [3, 4, 5]
    assert a.num_free_gpu_blocks == 0 and not a.can_allocate_gpu(1)


def test_freed_ids_queue_behind_the_never_used_ones():
    a = BlockAllocator(5, 0, 16)
    first = a.allocate_gpu_blocks(3)             # 0 1 2 ; free list: 3 4
    a.free_gpu(first[1])                         # free list: 3 4 1
    a.free_gpu(first[0])                         # free list: 3 4 1 0
    assert a.allocate_gpu_blocks(4) == [3, 4, 1, 0]


def test_churn_matches_a_model_deque():
    """Random alloc/free against a plain FIFO model of the same operations."""
    rng = random.Random(11)
    n = 40
    a = BlockAllocator(n, 0, 16)
    free = list(range(n))
    held = []
    for _ in range(2000):
        if held and (rng.random() < 0.45 or not free):
            bid = held.pop(rng.randrange(len(held)))
            a.free_gpu(bid)
            free.append(bid)
        else:
            k = rng.randint(1, 4)
            if len(free) < k:
                with pytest.raises(MemoryError):
                    a.allocate_gpu_blocks(k)
                continue
            got = a.allocate_gpu_blocks(k)
            assert got == free[:k]
            del free[:k]
            held += got
        assert a.num_free_gpu_blocks == len(free)


def test_ref_counts():
    a = BlockAllocator(3, 0, 16)
    bid = a.allocate_gpu()
    assert a.get_block(bid).ref_count == 1
    a.get_block(bid).ref_count += 1              # a second holder
    a.free_gpu(bid)
    assert a.num_free_gpu_blocks == 2            # still held once
    a.free_gpu(bid)
    assert a.num_free_gpu_blocks == 3 and a.get_block(bid).ref_count == 0


def test_exhaustion_raises_and_takes_nothing():
    a = BlockAllocator(4, 2, 16)
    a.allocate_gpu_blocks(3)
    with pytest.raises(MemoryError):
        a.allocate_gpu_blocks(2)
    assert a.num_free_gpu_blocks == 1            # the failed request took no block
    a.allocate_gpu()
    with pytest.raises(MemoryError):
        a.allocate_gpu()
    a.allocate_cpu()
    a.allocate_cpu()
    with pytest.raises(MemoryError):
        a.allocate_cpu()


@pytest.mark.parametrize("pool", ["gpu", "cpu"])
def test_double_free_is_an_assertion(pool):
    a = BlockAllocator(2, 2, 16)
    alloc, free = ((a.allocate_gpu, a.free_gpu) if pool == "gpu"
                   else (a.allocate_cpu, a.free_cpu))
    bid = alloc()
    free(bid)
    with pytest.raises(AssertionError):
        free(bid)


def test_swap_round_trip_maps_and_counts():
    a = BlockAllocator(6, 4, 16)
    gpu = a.allocate_gpu_blocks(3)
    out = a.swap_out(gpu)
    assert list(out) == gpu and sorted(out.values()) == [0, 1, 2]
    assert a.num_free_gpu_blocks == 6 and a.num_free_cpu_blocks == 1
    back = a.swap_in([out[g] for g in gpu])
    assert list(back) == [out[g] for g in gpu]
    assert a.num_free_cpu_blocks == 4 and a.num_free_gpu_blocks == 3
    # the GPU ids come back from the FIFO list: the never-used 3, 4, 5 first
    assert list(back.values()) == [3, 4, 5]


def test_swap_out_beyond_the_cpu_pool_raises():
    a = BlockAllocator(6, 2, 16)
    with pytest.raises(MemoryError):
        a.swap_out(a.allocate_gpu_blocks(3))


def test_allocator_tables_are_disjoint_and_scattered():
    blocks = [5, 40, 1, 17, 64]
    tables = wl.tables_by_allocator(blocks, num_blocks=400, seed=3, cycles=500)
    assert [len(t) for t in tables] == blocks
    flat = [b for t in tables for b in t]
    assert len(set(flat)) == len(flat) and all(0 <= b < 400 for b in flat)
    # churn leaves the free list out of order: some sequence holds non-consecutive ids
    assert any(t != list(range(t[0], t[0] + len(t))) for t in tables if len(t) > 1)
    assert tables == wl.tables_by_allocator(blocks, num_blocks=400, seed=3, cycles=500)
