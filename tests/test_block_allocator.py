"""BlockAllocator semantics: the reference's own assertions
(tests/unit/test_block_allocator.py:11-87, with the import pointed at this
package) plus the FIFO order and the fragmented-table generator."""
import pytest

from needle_amd.backend.block_allocator import BlockAllocator
from needle_amd import workloads as wl


@pytest.fixture
def allocator():
    return BlockAllocator(num_gpu_blocks=8, num_cpu_blocks=4, block_size=16)


class TestAllocateFree:
    def test_allocate_single(self, allocator):
        bid = allocator.allocate_gpu()
        assert 0 <= bid < 8
        assert allocator.num_free_gpu_blocks == 7

    def test_allocate_multiple(self, allocator):
        blocks = allocator.allocate_gpu_blocks(4)
        assert len(blocks) == 4 and len(set(blocks)) == 4
        assert allocator.num_free_gpu_blocks == 4

    def test_free_returns_to_pool(self, allocator):
        bid = allocator.allocate_gpu()
        allocator.free_gpu(bid)
        assert allocator.num_free_gpu_blocks == 8

    def test_free_double_raises(self, allocator):
        bid = allocator.allocate_gpu()
        allocator.free_gpu(bid)
        with pytest.raises(AssertionError):
            allocator.free_gpu(bid)

    def test_oom_raises(self, allocator):
        allocator.allocate_gpu_blocks(8)
        with pytest.raises(MemoryError):
            allocator.allocate_gpu()
        with pytest.raises(MemoryError):
            allocator.allocate_gpu_blocks(1)

    def test_can_allocate_check(self, allocator):
        assert allocator.can_allocate_gpu(8)
        assert not allocator.can_allocate_gpu(9)


class TestSwap:
    def test_swap_out_frees_gpu_allocates_cpu(self, allocator):
        gpu_blocks = allocator.allocate_gpu_blocks(3)
        mapping = allocator.swap_out(gpu_blocks)
        assert allocator.num_free_gpu_blocks == 8
        assert allocator.num_free_cpu_blocks == 1
        assert set(mapping.keys()) == set(gpu_blocks)
        assert all(0 <= v < 4 for v in mapping.values())

    def test_swap_in_frees_cpu_allocates_gpu(self, allocator):
        out_map = allocator.swap_out(allocator.allocate_gpu_blocks(3))
        allocator.swap_in(list(out_map.values()))
        assert allocator.num_free_cpu_blocks == 4
        assert allocator.num_free_gpu_blocks == 5

    def test_round_trip_mapping(self, allocator):
        out_map = allocator.swap_out(allocator.allocate_gpu_blocks(2))
        cpu = list(out_map.values())
        in_map = allocator.swap_in(cpu)
        new_gpu = [in_map[c] for c in cpu]
        assert len(new_gpu) == 2 and all(0 <= g < 8 for g in new_gpu)


class TestRefCount:
    def test_ref_count_increments(self, allocator):
        bid = allocator.allocate_gpu()
        assert allocator.get_block(bid, "gpu").ref_count == 1

    def test_partial_free(self, allocator):
        bid = allocator.allocate_gpu()
        block = allocator.get_block(bid)
        block.ref_count += 1
        allocator.free_gpu(bid)
        assert block.ref_count == 1 and allocator.num_free_gpu_blocks == 7
        allocator.free_gpu(bid)
        assert allocator.num_free_gpu_blocks == 8


def test_fifo_order():
    # block_allocator.py:40 popleft / :56 append: a freed id goes to the back.
    a = BlockAllocator(4, 0, 16)
    assert a.allocate_gpu_blocks(2) == [0, 1]
    a.free_gpu(0)
    assert a.allocate_gpu_blocks(3) == [2, 3, 0]


def test_fragmented_tables_are_disjoint_and_scattered():
    blocks = [40, 7, 130, 1, 64]
    tables = wl.tables_by_allocator(blocks, num_blocks=600, seed=5, cycles=2000)
    flat = [b for t in tables for b in t]
    assert [len(t) for t in tables] == blocks
    assert len(set(flat)) == len(flat)
    assert all(0 <= b < 600 for b in flat)
    # scattered: most consecutive logical blocks are not physically adjacent
    steps = sum(1 for t in tables for x, y in zip(t, t[1:]) if y != x + 1)
    assert steps > 0.5 * sum(len(t) - 1 for t in tables)
    again = wl.tables_by_allocator(blocks, num_blocks=600, seed=5, cycles=2000)
    assert again == tables
