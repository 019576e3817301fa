"""Continuous-batching scheduler producing the block tables the paged kernels read.

The policy is the reference's (needle/backend/scheduler.py:49-134), because it decides
which block ids reach block_table; each step, in this order:

  resume    swapped sequences, oldest first, each as soon as its whole block list fits
            on the GPU (every swapped sequence is tried, not only the first);
  admit     queued sequences in arrival order while the active count stays below
            max_num_seqs, the summed length of the active sequences plus the newcomer
            stays within max_num_batched_tokens, and its blocks fit;
  evict     while the GPU pool has no free block, the most recently activated sequence
            leaves: to the CPU pool when that can hold all its blocks, otherwise its
            blocks are released and it goes back to the head of the queue;
  extend    every sequence with ready K/V gets one more block when its length needs it
            (when several need one and the pool runs dry, the newest sequences are evicted
            by the rule above; the reference raises MemoryError there);
  split     active sequences without ready K/V are prefilled, the others decode.

So every table covers position length-1 (the slot a decode step appends to) and no
block is shared between sequences.  A sequence evicted without a CPU copy is prefilled
again when readmitted (see request.py).
"""
from __future__ import annotations

from collections import deque
from dataclasses import dataclass, field
from typing import Deque, Dict, List

from .block_allocator import BlockAllocator
from .request import Phase, SeqState


@dataclass
class StepPlan:
    """One step's work: the two forward groups and the block copies that precede them."""
    prefill: List[SeqState] = field(default_factory=list)
    decode: List[SeqState] = field(default_factory=list)
    swap_in: Dict[int, int] = field(default_factory=dict)    # CPU id -> GPU id
    swap_out: Dict[int, int] = field(default_factory=dict)   # GPU id -> CPU id
    released: List[int] = field(default_factory=list)        # GPU ids of evicted K/V

    @property
    def seqs(self) -> List[SeqState]:
        return self.prefill + self.decode

    @property
    def empty(self) -> bool:
        return not self.prefill and not self.decode


class Scheduler:
    def __init__(self, allocator: BlockAllocator, max_num_seqs: int = 256,
                 max_num_batched_tokens: int = 8192):
        self.allocator = allocator
        self.block_size = allocator.block_size
        self.max_num_seqs = max_num_seqs
        self.max_num_batched_tokens = max_num_batched_tokens
        self.queue: Deque[SeqState] = deque()
        self.active: List[SeqState] = []
        self.swapped: List[SeqState] = []

    def add(self, seq: SeqState) -> None:
        seq.phase = Phase.QUEUED
        self.queue.append(seq)

    def pending(self) -> bool:
        return bool(self.queue or self.active or self.swapped)

    def schedule(self) -> StepPlan:
        plan = StepPlan()
        self._resume(plan)
        self._admit()
        self._evict(plan)
        self._extend(plan)
        for s in self.active:
            (plan.decode if s.kv_ready else plan.prefill).append(s)
        return plan

    def finish(self, seq: SeqState) -> None:
        """Return a finished sequence's blocks; calling it twice is harmless."""
        if seq.phase is Phase.ACTIVE and seq.blocks:
            self.allocator.free_gpu_blocks(seq.blocks)
        elif seq.phase is Phase.SWAPPED and seq.blocks:
            self.allocator.free_cpu_blocks(seq.blocks)
        seq.blocks = []
        for pool in (self.active, self.swapped):
            if seq in pool:
                pool.remove(seq)
        if seq in self.queue:
            self.queue.remove(seq)
        seq.phase = Phase.DONE

    # ---------------------------------------------------------------- policy steps

    def _activate(self, seq: SeqState, blocks: List[int]) -> None:
        seq.blocks = blocks
        seq.phase = Phase.ACTIVE
        self.active.append(seq)

    def _resume(self, plan: StepPlan) -> None:
        waiting_for_room = []
        for seq in self.swapped:
            if not self.allocator.can_allocate_gpu(len(seq.blocks)):
                waiting_for_room.append(seq)
                continue
            moved = self.allocator.swap_in(seq.blocks)
            plan.swap_in.update(moved)
            self._activate(seq, [moved[c] for c in seq.blocks])
        self.swapped = waiting_for_room

    def _admit(self) -> None:
        in_flight = sum(s.length for s in self.active)
        while self.queue and len(self.active) < self.max_num_seqs:
            head = self.queue[0]
            need = head.blocks_needed(self.block_size)
            if in_flight + head.length > self.max_num_batched_tokens:
                break
            if not self.allocator.can_allocate_gpu(need):
                break
            self.queue.popleft()
            self._activate(head, self.allocator.allocate_gpu_blocks(need))
            in_flight += head.length

    def _evict(self, plan: StepPlan) -> None:
        while self.active and not self.allocator.can_allocate_gpu(1):
            self._evict_newest(plan)

    def _evict_newest(self, plan: StepPlan) -> None:
        seq = self.active.pop()
        if self.allocator.num_free_cpu_blocks >= len(seq.blocks):
            moved = self.allocator.swap_out(seq.blocks)
            plan.swap_out.update(moved)
            seq.blocks = [moved[g] for g in seq.blocks]
            seq.phase = Phase.SWAPPED
            self.swapped.append(seq)
        else:
            self.allocator.free_gpu_blocks(seq.blocks)
            plan.released.extend(seq.blocks)
            seq.blocks = []
            seq.kv_ready = False
            seq.phase = Phase.QUEUED
            self.queue.appendleft(seq)

    def _extend(self, plan: StepPlan) -> None:
        for seq in list(self.active):
            if seq.phase is not Phase.ACTIVE:        # evicted below for an earlier one
                continue
            if not (seq.kv_ready and seq.blocks_needed(self.block_size) > len(seq.blocks)):
                continue
            # Several sequences can cross a block edge in one step while the eviction step
            # left one free block; the reference then raises MemoryError.  Here the newest
            # sequences are evicted, by the same rule, until the block fits.
            while self.active and not self.allocator.can_allocate_gpu(1):
                self._evict_newest(plan)
            if seq.phase is Phase.ACTIVE:
                seq.blocks.append(self.allocator.allocate_gpu())
