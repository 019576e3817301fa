"""Continuous-batching scheduler (reference needle/backend/scheduler.py:22-154).

Same policy and defaults, step for step:
  1. swap SWAPPED sequences back in when their blocks fit (:54-67);
  2. admit WAITING sequences in FIFO order while the running count stays under
     max_num_seqs, the summed length of running sequences stays within
     max_num_batched_tokens and their blocks fit (:69-88);
  3. while no GPU block is free, preempt the newest running sequence: swap it
     out if the CPU pool can hold it, else free its blocks for recompute
     (:90-109);
  4. give every decoding sequence one more block when its length needs it (:111-118);
  5. split running sequences into prefill and decode (:120-134).
The only change: prefill/decode is decided by Sequence.prefilled (see
sequence.py), so a recompute-preempted sequence is prefilled again.
"""
from __future__ import annotations

from collections import deque
from typing import Dict, List

from .block_allocator import BlockAllocator
from .sequence import SchedulerOutput, Sequence, SequenceStatus


class Scheduler:
    def __init__(self, block_allocator: BlockAllocator, max_num_seqs: int = 256,
                 max_num_batched_tokens: int = 8192):
        self.allocator = block_allocator
        self.max_num_seqs = max_num_seqs
        self.max_num_batched_tokens = max_num_batched_tokens
        self.waiting: deque = deque()
        self.running: List[Sequence] = []
        self.swapped: List[Sequence] = []
        self._block_tables: Dict[int, List[int]] = {}
        self._cpu_block_tables: Dict[int, List[int]] = {}

    def add_sequence(self, seq: Sequence) -> None:
        self.waiting.append(seq)

    def schedule(self) -> SchedulerOutput:
        swap_in_map: Dict[int, int] = {}
        swap_out_map: Dict[int, int] = {}
        blocks_to_free: List[int] = []

        still_swapped: List[Sequence] = []
        for seq in self.swapped:
            cpu_blocks = self._cpu_block_tables[seq.seq_id]
            if self.allocator.can_allocate_gpu(len(cpu_blocks)):
                mapping = self.allocator.swap_in(cpu_blocks)
                swap_in_map.update(mapping)
                self._block_tables[seq.seq_id] = [mapping[c] for c in cpu_blocks]
                del self._cpu_block_tables[seq.seq_id]
                seq.status = SequenceStatus.RUNNING
                self.running.append(seq)
            else:
                still_swapped.append(seq)
        self.swapped = still_swapped

        batched = sum(s.length for s in self.running)
        while self.waiting:
            seq = self.waiting[0]
            need_blocks = seq.num_logical_blocks
            if (len(self.running) >= self.max_num_seqs
                    or batched + seq.length > self.max_num_batched_tokens
                    or not self.allocator.can_allocate_gpu(need_blocks)):
                break
            self.waiting.popleft()
            self._block_tables[seq.seq_id] = self.allocator.allocate_gpu_blocks(need_blocks)
            seq.status = SequenceStatus.RUNNING
            self.running.append(seq)
            batched += seq.length

        while self.running and not self.allocator.can_allocate_gpu(1):
            victim = self.running.pop()
            gpu_blocks = self._block_tables.pop(victim.seq_id)
            if self.allocator.num_free_cpu_blocks >= len(gpu_blocks):
                mapping = self.allocator.swap_out(gpu_blocks)
                swap_out_map.update(mapping)
                self._cpu_block_tables[victim.seq_id] = [mapping[g] for g in gpu_blocks]
                victim.status = SequenceStatus.SWAPPED
                self.swapped.append(victim)
            else:
                self.allocator.free_gpu_blocks(gpu_blocks)
                blocks_to_free.extend(gpu_blocks)
                victim.status = SequenceStatus.WAITING
                victim.prefilled = False            # its KV is gone: prefill again
                self.waiting.appendleft(victim)

        for seq in self.running:
            if seq.prefilled:
                table = self._block_tables[seq.seq_id]
                if seq.num_logical_blocks > len(table):
                    table.append(self.allocator.allocate_gpu())

        prefill = [s for s in self.running if not s.prefilled]
        decode = [s for s in self.running if s.prefilled]
        return SchedulerOutput(prefill_seqs=prefill, decode_seqs=decode,
                               block_tables={k: list(v) for k, v in self._block_tables.items()},
                               swap_in_map=swap_in_map, swap_out_map=swap_out_map,
                               blocks_to_free=blocks_to_free)

    def free_sequence(self, seq: Sequence) -> None:
        if seq.seq_id in self._block_tables:
            self.allocator.free_gpu_blocks(self._block_tables.pop(seq.seq_id))
        if seq.seq_id in self._cpu_block_tables:
            self.allocator.free_cpu_blocks(self._cpu_block_tables.pop(seq.seq_id))
        seq.finish()
        try:
            self.running.remove(seq)
        except ValueError:
            pass

    def has_unfinished_seqs(self) -> bool:
        return bool(self.waiting or self.running or self.swapped)
