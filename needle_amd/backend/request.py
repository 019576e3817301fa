"""What the continuous-batching driver knows about each request.

SamplingParams is the argument of LLMEngine.add_request, so its field names, defaults
and accepted ranges are the reference's (needle/backend/sequence.py:13-25); a value out
of range raises ValueError here.

SeqState is this driver's record of one sequence.  Besides the tokens it holds the
physical ids of the blocks that store the sequence's K/V (`blocks`: GPU pool ids while
the sequence is ACTIVE, CPU pool ids while it is SWAPPED, empty otherwise) and whether
those blocks hold the K/V of every token but the newest (`kv_ready`).  A sequence
without ready K/V is prefilled; with it, it takes one decode step.  The reference
decides prefill against decode by "no token generated yet" (scheduler.py:120-134),
which sends a recompute-preempted sequence (blocks freed, scheduler.py:103-109) to a
decode step over blocks it no longer owns; here such a sequence is prefilled again.
"""
from __future__ import annotations

import time
from dataclasses import dataclass, field
from enum import Enum
from typing import List, Optional


@dataclass
class SamplingParams:
    temperature: float = 1.0
    top_p: float = 1.0
    top_k: int = -1
    max_new_tokens: int = 512
    stop_token_ids: List[int] = field(default_factory=list)
    stream: bool = False

    def __post_init__(self):
        bad = []
        if not self.temperature >= 0.0:
            bad.append(f"temperature {self.temperature} < 0")
        if not 0.0 < self.top_p <= 1.0:
            bad.append(f"top_p {self.top_p} outside (0, 1]")
        if self.max_new_tokens <= 0:
            bad.append(f"max_new_tokens {self.max_new_tokens} <= 0")
        if bad:
            raise ValueError("invalid sampling parameters: " + ", ".join(bad))

    @property
    def greedy(self) -> bool:
        return self.temperature == 0.0


class Phase(Enum):
    QUEUED = "queued"        # waiting for admission; owns no blocks
    ACTIVE = "active"        # owns GPU blocks; takes part in every step
    SWAPPED = "swapped"      # its K/V sits in CPU pool blocks
    DONE = "done"


class SeqState:
    """One sequence of the driver: tokens so far, where its K/V lives, its phase."""

    __slots__ = ("seq_id", "request_id", "tokens", "prompt_len", "params", "phase",
                 "kv_ready", "blocks", "arrival")

    def __init__(self, seq_id: int, request_id: str, prompt: List[int],
                 params: Optional[SamplingParams] = None, arrival: Optional[float] = None):
        if not prompt:
            raise ValueError(f"request {request_id!r} has an empty prompt")
        self.seq_id = seq_id
        self.request_id = request_id
        self.tokens: List[int] = list(prompt)
        self.prompt_len = len(self.tokens)
        self.params = params if params is not None else SamplingParams()
        self.phase = Phase.QUEUED
        self.kv_ready = False
        self.blocks: List[int] = []
        self.arrival = time.time() if arrival is None else arrival

    @property
    def length(self) -> int:
        return len(self.tokens)

    @property
    def generated(self) -> int:
        return len(self.tokens) - self.prompt_len

    @property
    def last_token(self) -> int:
        return self.tokens[-1]

    def blocks_needed(self, block_size: int) -> int:
        """Blocks that hold positions 0..length-1 (the table must cover the newest)."""
        return -(-len(self.tokens) // block_size)

    def output(self) -> List[int]:
        return self.tokens[self.prompt_len:]

    def push(self, token: int) -> bool:
        """Append a sampled token; True when the request is complete (a stop token or
        max_new_tokens reached, as engine.py:124-130 decides)."""
        self.tokens.append(token)
        return token in self.params.stop_token_ids or self.generated >= self.params.max_new_tokens

    def __repr__(self) -> str:
        return (f"SeqState({self.seq_id}, {self.request_id!r}, len={self.length}, "
                f"{self.phase.value}, blocks={len(self.blocks)})")
