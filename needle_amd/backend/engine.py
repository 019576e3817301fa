"""LLMEngine: scheduler + runner step loop (reference needle/backend/engine.py:23-153).

add_request / step / has_unfinished_requests / generate keep the reference's
meaning: a request finishes when it emits a stop token or max_new_tokens
tokens; step() returns {request_id: generated token ids} for the requests that
finished in that step.  The model comes from a ModelConfig with synthetic
weights (no checkpoint loading) or is passed in.  decode_graphs=True replays
decode steps from HIP graphs captured per batch-size bucket (sequences longer than
max_model_len fall back to eager launches).
"""
from __future__ import annotations

import itertools
import time
from typing import Dict, List, Optional

import torch

from ..model.config import ModelConfig
from ..model.runner import ModelRunner
from .block_allocator import BlockAllocator
from .scheduler import Scheduler
from .sequence import Request, SamplingParams, Sequence


class LLMEngine:
    def __init__(self, model_config: ModelConfig, block_size: int = 16, max_num_seqs: int = 256,
                 max_num_batched_tokens: int = 8192, gpu_memory_utilization: float = 0.90,
                 max_gpu_blocks: int = 0, cpu_swap_bytes: int = 0, dtype: str = "bfloat16",
                 device: str = "cuda:0", seed: int = 0,
                 model: Optional[torch.nn.Module] = None, decode_graphs: bool = False,
                 max_model_len: int = 0):
        self.block_size = block_size
        self.model_config = model_config
        self.runner = ModelRunner(model_config, block_size, dtype, device, seed, model)
        n_gpu, n_cpu = self.runner.profile_memory(gpu_memory_utilization, max_gpu_blocks,
                                                  cpu_swap_bytes)
        # With decode graphs the last pool block is the runner's scratch block for padding
        # rows, so the allocator only sees the others.
        self.allocator = BlockAllocator(n_gpu - 1 if decode_graphs else n_gpu, n_cpu, block_size)
        self.scheduler = Scheduler(self.allocator, max_num_seqs, max_num_batched_tokens)
        self.runner.init_kv_cache(n_gpu, n_cpu)
        if decode_graphs:
            buckets = tuple(b for b in ModelRunner.DEFAULT_BUCKETS if b < max_num_seqs)
            buckets = buckets + (max_num_seqs,)
            self.runner.enable_decode_graphs(max_model_len or model_config.max_position_embeddings,
                                             buckets)
        self._ids = itertools.count(1)

    def add_request(self, request_id: str, prompt_token_ids: List[int],
                    sampling_params: SamplingParams) -> None:
        req = Request(request_id, list(prompt_token_ids), sampling_params, time.time())
        n = (len(prompt_token_ids) + self.block_size - 1) // self.block_size
        self.scheduler.add_sequence(Sequence(seq_id=next(self._ids), request=req,
                                             token_ids=list(prompt_token_ids),
                                             logical_blocks=list(range(n)),
                                             block_size=self.block_size))

    def step(self) -> Dict[str, List[int]]:
        sched = self.scheduler.schedule()
        if sched.is_empty:
            return {}
        out = self.runner.execute(sched)
        finished: Dict[str, List[int]] = {}
        for seq, tok in zip(sched.prefill_seqs + sched.decode_seqs, out.next_token_ids):
            seq.append_token(tok)
            p = seq.request.sampling_params
            if tok in p.stop_token_ids or seq.num_generated_tokens >= p.max_new_tokens:
                self.scheduler.free_sequence(seq)
                finished[seq.request.request_id] = seq.token_ids[seq.prompt_len:]
        return finished

    def has_unfinished_requests(self) -> bool:
        return self.scheduler.has_unfinished_seqs()

    def generate(self, prompt_token_ids: List[int],
                 sampling_params: Optional[SamplingParams] = None,
                 request_id: str = "sync-0") -> List[int]:
        self.add_request(request_id, prompt_token_ids, sampling_params or SamplingParams())
        while self.has_unfinished_requests():
            done = self.step()
            if request_id in done:
                return done[request_id]
        return []
