"""KV block allocator with the reference's block-id contract.

Semantics follow needle/backend/block_allocator.py:10-124 of the reference:
  * free lists are FIFO: allocation pops the oldest free id, freeing appends
    (so alloc/free churn scatters ids across the pool);
  * a block starts with ref_count 1; freeing decrements and returns the id to
    the free list when the count reaches 0;
  * exhausting a pool raises MemoryError; freeing a free block raises
    AssertionError;
  * swap_out / swap_in move a list of blocks between the GPU and CPU pools and
    return the id mapping.
The ids it hands out are the entries of block_table consumed by the kernels.
"""
from __future__ import annotations

from collections import deque
from dataclasses import dataclass
from typing import Dict, List


@dataclass
class PhysicalBlock:
    """needle/backend/sequence.py:83-87."""
    block_id: int
    ref_count: int = 0
    device: str = "gpu"


class _Pool:
    def __init__(self, n: int, device: str):
        self.free: deque = deque(range(n))
        self.blocks: Dict[int, PhysicalBlock] = {
            i: PhysicalBlock(block_id=i, device=device) for i in range(n)}
        self.device = device

    def alloc(self) -> int:
        if not self.free:
            raise MemoryError(f"No free {self.device.upper()} blocks available")
        bid = self.free.popleft()
        self.blocks[bid].ref_count = 1
        return bid

    def release(self, bid: int) -> None:
        blk = self.blocks[bid]
        assert blk.ref_count > 0, f"Block {bid} already free"
        blk.ref_count -= 1
        if blk.ref_count == 0:
            self.free.append(bid)


class BlockAllocator:
    """block_allocator.py:10 -- GPU pool plus a CPU swap pool."""

    def __init__(self, num_gpu_blocks: int, num_cpu_blocks: int, block_size: int):
        self.block_size = block_size
        self._gpu = _Pool(num_gpu_blocks, "gpu")
        self._cpu = _Pool(num_cpu_blocks, "cpu")

    # GPU pool (block_allocator.py:37-60)
    def allocate_gpu(self) -> int:
        return self._gpu.alloc()

    def allocate_gpu_blocks(self, num: int) -> List[int]:
        if len(self._gpu.free) < num:
            raise MemoryError(
                f"Requested {num} GPU blocks but only {len(self._gpu.free)} available")
        return [self._gpu.alloc() for _ in range(num)]

    def free_gpu(self, block_id: int) -> None:
        self._gpu.release(block_id)

    def free_gpu_blocks(self, block_ids: List[int]) -> None:
        for bid in block_ids:
            self._gpu.release(bid)

    # CPU pool (block_allocator.py:66-82)
    def allocate_cpu(self) -> int:
        return self._cpu.alloc()

    def free_cpu(self, block_id: int) -> None:
        self._cpu.release(block_id)

    def free_cpu_blocks(self, block_ids: List[int]) -> None:
        for bid in block_ids:
            self._cpu.release(bid)

    # swap (block_allocator.py:88-104)
    def swap_out(self, gpu_block_ids: List[int]) -> Dict[int, int]:
        """Allocate a CPU block per GPU block, free the GPU block; gpu id -> cpu id."""
        mapping: Dict[int, int] = {}
        for gid in gpu_block_ids:
            mapping[gid] = self._cpu.alloc()
            self._gpu.release(gid)
        return mapping

    def swap_in(self, cpu_block_ids: List[int]) -> Dict[int, int]:
        """Allocate a GPU block per CPU block, free the CPU block; cpu id -> gpu id."""
        mapping: Dict[int, int] = {}
        for cid in cpu_block_ids:
            mapping[cid] = self._gpu.alloc()
            self._cpu.release(cid)
        return mapping

    # queries (block_allocator.py:110-124)
    @property
    def num_free_gpu_blocks(self) -> int:
        return len(self._gpu.free)

    @property
    def num_free_cpu_blocks(self) -> int:
        return len(self._cpu.free)

    def can_allocate_gpu(self, num: int = 1) -> bool:
        return len(self._gpu.free) >= num

    def get_block(self, block_id: int, device: str = "gpu") -> PhysicalBlock:
        return (self._gpu if device == "gpu" else self._cpu).blocks[block_id]
