"""Scheduler policy (scheduler.py:49-134 of the reference) on the CPU.

Each test drives the scheduler the way the engine does: schedule, mark the prefilled
sequences' K/V ready, append one token to every scheduled sequence, finish the ones that
are done.  A randomized run checks the invariants the kernels rely on after every step.
"""
import random

import pytest

from needle_amd.backend.block_allocator import BlockAllocator
from needle_amd.backend.request import Phase, SamplingParams, SeqState
from needle_amd.backend.scheduler import Scheduler

BS = 16


def seq(i, n=8, max_new=32):
    return SeqState(i, f"r{i}", list(range(100, 100 + n)), SamplingParams(max_new_tokens=max_new))


def advance(sched, plan, token=7):
    """What runner + engine do after the step's forwards."""
    for s in plan.prefill:
        s.kv_ready = True
    done = []
    for s in plan.seqs:
        if s.push(token):
            done.append(s)
    for s in done:
        sched.finish(s)


def test_admission_is_fifo_and_capped_by_count():
    sched = Scheduler(BlockAllocator(64, 0, BS), max_num_seqs=3, max_num_batched_tokens=10_000)
    seqs = [seq(i) for i in range(5)]
    for s in seqs:
        sched.add(s)
    plan = sched.schedule()
    assert plan.prefill == seqs[:3] and not plan.decode
    assert list(sched.queue) == seqs[3:]
    assert all(s.phase is Phase.ACTIVE for s in seqs[:3])


def test_token_budget_counts_whole_running_lengths():
    # 40 + 40 fit in 100; the third would make 120.  After a step the two running
    # sequences count 41 each, so a 19-token newcomer still fits (101 > 100 does not).
    sched = Scheduler(BlockAllocator(64, 0, BS), max_num_seqs=8, max_num_batched_tokens=100)
    a, b, c = seq(1, 40), seq(2, 40), seq(3, 40)
    for s in (a, b, c):
        sched.add(s)
    plan = sched.schedule()
    assert plan.prefill == [a, b]
    advance(sched, plan)
    d = seq(4, 18)
    sched.queue.appendleft(d)
    plan = sched.schedule()
    assert plan.prefill == [d] and plan.decode == [a, b] and list(sched.queue) == [c]


def test_admission_stops_at_the_first_that_does_not_fit():
    # head needs 3 blocks, only 2 free: nothing behind it is admitted either
    sched = Scheduler(BlockAllocator(4, 0, BS), max_num_seqs=8, max_num_batched_tokens=10_000)
    sched.add(seq(1, 30))                        # 2 blocks
    sched.schedule()
    sched.add(seq(2, 40))                        # 3 blocks
    sched.add(seq(3, 4))                         # 1 block
    plan = sched.schedule()
    assert [s.seq_id for s in sched.queue] == [2, 3] and len(plan.seqs) == 1


def test_prefill_then_decode_and_table_growth_at_block_edges():
    sched = Scheduler(BlockAllocator(8, 0, BS), max_num_seqs=4, max_num_batched_tokens=512)
    s = seq(1, n=15, max_new=40)
    sched.add(s)
    plan = sched.schedule()
    assert plan.prefill == [s] and len(s.blocks) == 1
    lengths = []
    for _ in range(20):
        advance(sched, plan)
        plan = sched.schedule()
        assert plan.decode == [s]
        lengths.append((s.length, len(s.blocks)))
    # the table always covers position length-1 and never more than needed
    assert all(nb == (n + BS - 1) // BS for n, nb in lengths)
    assert (16, 1) in lengths and (17, 2) in lengths and (33, 3) in lengths


def test_finish_returns_blocks_and_is_idempotent():
    alloc = BlockAllocator(8, 0, BS)
    sched = Scheduler(alloc, 4, 512)
    s = seq(1, n=40)
    sched.add(s)
    sched.schedule()
    assert alloc.num_free_gpu_blocks == 5
    sched.finish(s)
    sched.finish(s)
    assert alloc.num_free_gpu_blocks == 8 and s.phase is Phase.DONE
    assert not sched.pending()


def test_full_pool_evicts_the_newest_to_cpu_then_resumes_it():
    alloc = BlockAllocator(3, 4, BS)
    sched = Scheduler(alloc, 4, 512)
    a, b = seq(1, 20), seq(2, 10)                # 2 + 1 blocks: the pool is then full
    sched.add(a)
    sched.add(b)
    plan = sched.schedule()
    assert plan.prefill == [a] and b.phase is Phase.SWAPPED
    assert list(plan.swap_out) == [2] and b.blocks == [plan.swap_out[2]]
    sched.finish(a)                              # room again
    plan = sched.schedule()
    assert plan.swap_in == {0: b.blocks[0]} and b.phase is Phase.ACTIVE
    # b never ran, so it is prefilled from its swapped-in (stale) block
    assert plan.prefill == [b]


def test_swapped_decoder_keeps_decoding_after_resume():
    alloc = BlockAllocator(4, 4, BS)
    sched = Scheduler(alloc, 4, 512)
    a, b = seq(1, 16), seq(2, 30)                # 1 + 2 blocks, one left
    sched.add(a)
    sched.add(b)
    advance(sched, sched.schedule())             # both prefilled: lengths 17 and 31
    plan = sched.schedule()                      # a grows into the last free block
    assert plan.decode == [a, b] and alloc.num_free_gpu_blocks == 0 and not plan.swap_out
    advance(sched, plan)
    plan = sched.schedule()                      # no free block: the newest, b, leaves
    assert b.phase is Phase.SWAPPED and plan.decode == [a] and len(plan.swap_out) == 2
    assert sorted(plan.swap_out.values()) == sorted(b.blocks)
    sched.finish(a)
    plan = sched.schedule()
    assert b.phase is Phase.ACTIVE and plan.decode == [b] and b.kv_ready
    assert len(plan.swap_in) == 2 and sorted(plan.swap_in.values()) == sorted(b.blocks)


def test_every_swapped_sequence_is_tried_for_resume():
    # the first swapped sequence is too big to come back, the second fits
    alloc = BlockAllocator(4, 8, BS)
    sched = Scheduler(alloc, 4, 10_000)
    big, small = seq(1, 60), seq(2, 10)          # 4 blocks, 1 block
    big.phase = small.phase = Phase.SWAPPED
    big.blocks = [alloc.allocate_cpu() for _ in range(4)]
    small.blocks = [alloc.allocate_cpu()]
    big.kv_ready = small.kv_ready = True
    sched.swapped = [big, small]
    hog = alloc.allocate_gpu_blocks(2)
    plan = sched.schedule()
    assert sched.swapped == [big] and small.phase is Phase.ACTIVE and plan.decode == [small]
    assert hog and len(plan.swap_in) == 1


def test_eviction_without_cpu_room_requeues_for_a_new_prefill():
    alloc = BlockAllocator(2, 0, BS)
    sched = Scheduler(alloc, 4, 512)
    a, b = seq(1), seq(2)
    sched.add(a)
    sched.add(b)
    plan = sched.schedule()
    assert plan.prefill == [a] and b.phase is Phase.QUEUED and plan.released
    assert sched.queue[0] is b and not b.kv_ready and b.blocks == []
    advance(sched, plan)
    sched.finish(a)
    plan = sched.schedule()
    assert plan.prefill == [b]


def test_empty_schedule():
    sched = Scheduler(BlockAllocator(4, 0, BS))
    plan = sched.schedule()
    assert plan.empty and not sched.pending()


@pytest.mark.parametrize("cpu_blocks", [0, 12])
def test_random_run_keeps_the_table_invariants(cpu_blocks):
    rng = random.Random(cpu_blocks + 5)
    n_gpu = 24
    alloc = BlockAllocator(n_gpu, cpu_blocks, BS)
    sched = Scheduler(alloc, max_num_seqs=6, max_num_batched_tokens=300)
    for i in range(30):
        sched.add(seq(i, rng.randint(1, 60), rng.randint(1, 40)))
    steps = 0
    while sched.pending() and steps < 3000:
        plan = sched.schedule()
        held = [b for s in sched.active for b in s.blocks]
        assert len(held) == len(set(held)) and all(0 <= b < n_gpu for b in held)
        assert alloc.num_free_gpu_blocks + len(held) == n_gpu
        cpu_held = [b for s in sched.swapped for b in s.blocks]
        assert alloc.num_free_cpu_blocks + len(cpu_held) == cpu_blocks
        assert len(sched.active) <= 6
        for s in plan.decode:
            assert s.kv_ready and len(s.blocks) == (s.length + BS - 1) // BS
        for s in plan.prefill:
            assert len(s.blocks) == (s.length + BS - 1) // BS
        advance(sched, plan, token=rng.randint(0, 99))
        steps += 1
    assert not sched.pending() and alloc.num_free_gpu_blocks == n_gpu


def test_two_block_edges_in_one_step_evict_instead_of_raising():
    # a, b and c all cross a block edge in the same step with one free block: a takes it,
    # the newest (c) is evicted so that b gets one (the reference raises MemoryError here)
    alloc = BlockAllocator(5, 0, BS)
    sched = Scheduler(alloc, 4, 512)
    a, b, c = seq(1, 16), seq(2, 16), seq(3, 32)
    for s in (a, b, c):
        sched.add(s)
    advance(sched, sched.schedule())             # lengths 17, 17, 33
    plan = sched.schedule()
    assert plan.decode == [a, b] and len(a.blocks) == 2 and len(b.blocks) == 2
    assert c.phase is Phase.QUEUED and sched.queue[0] is c and len(plan.released) == 2
