"""Scheduler semantics: the reference's own tests (tests/unit/test_scheduler.py:22-108,
imports pointed at this package) plus preemption paths, on the CPU."""
import pytest

from needle_amd.backend.block_allocator import BlockAllocator
from needle_amd.backend.scheduler import Scheduler
from needle_amd.backend.sequence import Request, SamplingParams, Sequence, SequenceStatus


def make_seq(seq_id, prompt_len=8, block_size=16):
    prompt = list(range(prompt_len))
    req = Request(f"req-{seq_id}", prompt, SamplingParams(max_new_tokens=32))
    n = (prompt_len + block_size - 1) // block_size
    return Sequence(seq_id=seq_id, request=req, token_ids=list(prompt),
                    logical_blocks=list(range(n)), block_size=block_size)


def run_step(sched, out, token=100):
    # what the runner + engine do after a forward: mark prefills, append one token
    for s in out.prefill_seqs:
        s.prefilled = True
    for s in out.prefill_seqs + out.decode_seqs:
        s.append_token(token)


@pytest.fixture
def scheduler():
    return Scheduler(BlockAllocator(16, 8, 16), max_num_seqs=4, max_num_batched_tokens=512)


def test_waiting_to_running(scheduler):
    seq = make_seq(1)
    scheduler.add_sequence(seq)
    out = scheduler.schedule()
    assert seq in out.prefill_seqs and seq.status == SequenceStatus.RUNNING


def test_prefill_then_decode(scheduler):
    seq = make_seq(1)
    scheduler.add_sequence(seq)
    out = scheduler.schedule()
    assert seq in out.prefill_seqs
    run_step(scheduler, out)
    assert seq in scheduler.schedule().decode_seqs


def test_max_seqs_limit(scheduler):
    for i in range(6):
        scheduler.add_sequence(make_seq(i))
    out = scheduler.schedule()
    assert len(out.prefill_seqs + out.decode_seqs) <= 4


def test_token_budget_counts_running_lengths():
    # scheduler.py:70-81: admission stops when running lengths + the next prompt > budget
    sched = Scheduler(BlockAllocator(64, 0, 16), max_num_seqs=8, max_num_batched_tokens=100)
    for i in range(4):
        sched.add_sequence(make_seq(i, prompt_len=40))
    out = sched.schedule()
    assert len(out.prefill_seqs) == 2 and len(sched.waiting) == 2


def test_block_table_populated_and_grows(scheduler):
    seq = make_seq(1, prompt_len=16)
    scheduler.add_sequence(seq)
    out = scheduler.schedule()
    assert len(out.block_tables[seq.seq_id]) == 1
    run_step(scheduler, out)                      # length 17 -> needs a second block
    out2 = scheduler.schedule()
    assert len(out2.block_tables[seq.seq_id]) == 2
    assert len(set(out2.block_tables[seq.seq_id])) == 2


def test_free_sequence(scheduler):
    seq = make_seq(1)
    scheduler.add_sequence(seq)
    scheduler.schedule()
    scheduler.free_sequence(seq)
    scheduler.free_sequence(seq)                  # double free tolerated (scheduler.py:136-151)
    assert seq.status == SequenceStatus.FINISHED and not scheduler.has_unfinished_seqs()
    assert scheduler.allocator.num_free_gpu_blocks == 16


def test_swap_out_when_pool_runs_dry():
    # Two blocks, two one-block prompts: admitting both leaves no free block, so step 3
    # of the policy preempts the newest one into the CPU pool right away
    # (scheduler.py:90-102).  The reference's test expects 2 running here, which its own
    # scheduler does not produce.
    sched = Scheduler(BlockAllocator(2, 4, 16), max_num_seqs=4, max_num_batched_tokens=512)
    s1, s2 = make_seq(1), make_seq(2)
    sched.add_sequence(s1)
    sched.add_sequence(s2)
    out = sched.schedule()
    assert out.prefill_seqs == [s1] and s2.status == SequenceStatus.SWAPPED
    assert len(out.swap_out_map) == 1
    sched.add_sequence(make_seq(3))
    out2 = sched.schedule()
    assert len(out2.prefill_seqs) + len(out2.decode_seqs) <= 2


def test_recompute_preemption_prefills_again():
    # no CPU pool: the victim's blocks are freed and it must be prefilled again
    sched = Scheduler(BlockAllocator(2, 0, 16), max_num_seqs=4, max_num_batched_tokens=512)
    s1, s2 = make_seq(1), make_seq(2)
    sched.add_sequence(s1)
    sched.add_sequence(s2)
    out = sched.schedule()
    assert out.prefill_seqs == [s1] and s2.status == SequenceStatus.WAITING
    assert out.blocks_to_free and not s2.prefilled
    run_step(sched, out)
    sched.free_sequence(s1)
    out2 = sched.schedule()
    assert s2 in out2.prefill_seqs                # re-admitted as a prefill, not a decode


def test_empty_schedule(scheduler):
    assert scheduler.schedule().is_empty and not scheduler.has_unfinished_seqs()
