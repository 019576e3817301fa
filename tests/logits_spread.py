"""How far two valid arithmetics of the reference path move the real Qwen2-0.5B's logits.

The end-to-end model's logits carry the bf16 rounding of 24 layers of GEMMs and attention,
so a GPU-vs-oracle logits bound cannot be the attention tolerance.  This module measures
the spread the oracle itself shows when only its attention arithmetic changes: the same CPU
model and schedule with the oracle's attention seams (reference needle/layers/attention.py
:102-107, :140-159, in bf16 op for op) against the same seams computed in fp32 (q, k, v and
the pool upcast, the output rounded to bf16 once).  Both runners see the same
scheduler-built batches (reference needle/model/runner.py:194-249), teacher-forced with the
bf16 runner's greedy tokens.  The logits bounds of the GPU engine test are derived from
this spread (BOUND_FACTOR times it); tests/test_logits_spread.py recomputes it on the CPU.
"""
from __future__ import annotations

import types

import torch

from needle_amd import e2e
from needle_amd.backend.block_allocator import BlockAllocator
from needle_amd.backend.request import SamplingParams, SeqState
from needle_amd.backend.scheduler import Scheduler
from needle_amd.model.config import QWEN2_0_5B, ModelConfig
from needle_amd.model.qwen2 import build_model, random_init_
from needle_amd.model.runner import ModelRunner
from oracle import paged_ref

# The GPU engine's logits may differ from the bf16 oracle's by this multiple of the spread.
BOUND_FACTOR = 2.0

# Measured by logits_spread() (tests/test_logits_spread.py keeps these in step with it):
# max |fp32-attention logits - bf16-attention logits|, and max over forwards of
# ||diff||_2 / ||bf16 logits||_2.
SPREAD_MAX_DIFF = 0.06885
SPREAD_REL_L2 = 0.02207


def _prefill(dtype):
    def seam(self, q, k, v, kv_cache, block_table, cu_seqlens, context_lens, max_seqlen):
        if dtype is None:
            return paged_ref.prefill(q, k, v, kv_cache, block_table, cu_seqlens, context_lens,
                                     self.num_heads, self.num_kv_heads)
        pool = kv_cache.to(dtype)
        out = paged_ref.prefill(q.to(dtype), k.to(dtype), v.to(dtype), pool, block_table,
                                cu_seqlens, context_lens, self.num_heads, self.num_kv_heads)
        kv_cache.copy_(pool)
        return out.to(q.dtype)
    return seam


def _decode(dtype):
    def seam(self, q, k, v, kv_cache, block_table, context_lens):
        if dtype is None:
            return paged_ref.decode(q, k, v, kv_cache, block_table, context_lens, self.scale,
                                    self.num_heads, self.num_kv_heads, self.head_dim)
        pool = kv_cache.to(dtype)
        out = paged_ref.decode(q.to(dtype), k.to(dtype), v.to(dtype), pool, block_table,
                               context_lens, self.scale, self.num_heads, self.num_kv_heads,
                               self.head_dim)
        kv_cache.copy_(pool)
        return out.to(q.dtype)
    return seam


def oracle_runner(cfg: ModelConfig, model, attention_dtype=None,
                  block_size: int = 16) -> ModelRunner:
    """A CPU runner whose attention seams are the oracle: RoPE as the reference's torch ops,
    then write_kv + per-sequence SDPA (prefill) or the decode append + _decode_pytorch, in
    the model dtype (attention_dtype None) or computed in attention_dtype."""
    r = ModelRunner(cfg, block_size, device="cpu", model=model)
    for layer in r.model.model.layers:
        att = layer.self_attn
        att.fuse_rope = False
        att._prefill = types.MethodType(_prefill(attention_dtype), att)
        att._decode = types.MethodType(_decode(attention_dtype), att)
    return r


def add_requests(sched: Scheduler, n: int = 8) -> None:
    """The first n benchmark requests; the first two stop after 3 tokens, the rest after 7,
    so the two that wait are admitted next to decoding sequences (a mixed step)."""
    for i, (rid, prompt, _olen) in enumerate(e2e.requests(n)):
        sched.add(SeqState(i + 1, rid, prompt,
                           SamplingParams(temperature=0.0, max_new_tokens=3 if i < 2 else 7)))


def scheduler(nb: int = 800) -> Scheduler:
    return Scheduler(BlockAllocator(nb, 0, 16), max_num_seqs=6, max_num_batched_tokens=8192)


@torch.no_grad()
def logits_spread(nb: int = 800):
    """(max |diff|, max relative L2, forwards) between the bf16 and fp32-attention oracle
    runners over the schedule of add_requests()."""
    cfg = ModelConfig(**QWEN2_0_5B)
    a = oracle_runner(cfg, random_init_(build_model(cfg), e2e.E2E_SEED))
    b = oracle_runner(cfg, random_init_(build_model(cfg), e2e.E2E_SEED), torch.float32)
    a.init_kv_cache(nb)
    b.init_kv_cache(nb)
    sched = scheduler(nb)
    add_requests(sched)
    worst = worst_rel = 0.0
    forwards = 0
    while sched.pending():
        plan = sched.schedule()
        picks = []
        for group, pre in ((plan.prefill, True), (plan.decode, False)):
            if not group:
                continue
            la = a.forward(a.prepare_inputs(group, pre)).float()
            lb = b.forward(b.prepare_inputs(group, pre)).float()
            d = (la - lb).abs()
            worst = max(worst, float(d.max()))
            worst_rel = max(worst_rel, float(d.norm() / la.norm()))
            picks += la.argmax(-1).tolist()
            forwards += 1
        for s in plan.prefill:
            s.kv_ready = True
        for s, t in zip(plan.seqs, picks):
            if s.push(t):
                sched.finish(s)
    return worst, worst_rel, forwards
