"""LLMEngine: the scheduler + runner step loop (the API of reference needle/backend/engine.py:86-153).

add_request / step / has_unfinished_requests / generate keep the reference's meaning: a
request finishes when it emits a stop token or max_new_tokens tokens, and step() returns
{request_id: generated token ids} for the requests that finished in that step.  Sampling
is greedy only: a request with temperature > 0 is refused when it is added.  The model
comes from a ModelConfig with synthetic weights (no checkpoint loading) or is passed in.
decode_graphs=True replays decode steps from HIP graphs captured per batch-size bucket;
their metadata stays on the device between steps (sequences longer than max_model_len, or
batches beyond the largest bucket, run eagerly).  cpu_swap_bytes sizes a pinned CPU pool
that preemption swaps blocks into (0: evicted sequences are recomputed).
"""
from __future__ import annotations

import itertools
from typing import Dict, List, Optional

import torch

from ..model.config import ModelConfig
from ..model.runner import ModelRunner
from ..model.sampler import check_greedy
from .block_allocator import BlockAllocator
from .request import SamplingParams, SeqState
from .scheduler import Scheduler


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
        # With decode graphs the last pool block is the padding rows' scratch block, so the
        # allocator only hands out the others.
        self.allocator = BlockAllocator(n_gpu - 1 if decode_graphs else n_gpu, n_cpu, block_size)
        self.scheduler = Scheduler(self.allocator, max_num_seqs, max_num_batched_tokens)
        self.runner.init_kv_cache(n_gpu, n_cpu)
        if decode_graphs:
            buckets = tuple(b for b in ModelRunner.DEFAULT_BUCKETS if b < max_num_seqs)
            self.runner.enable_decode_graphs(max_model_len or model_config.max_position_embeddings,
                                             buckets + (max_num_seqs,))
        self._ids = itertools.count(1)

    def add_request(self, request_id: str, prompt_token_ids: List[int],
                    sampling_params: SamplingParams) -> None:
        check_greedy(sampling_params)
        self.scheduler.add(SeqState(next(self._ids), request_id, list(prompt_token_ids),
                                    sampling_params))

    def step(self) -> Dict[str, List[int]]:
        plan = self.scheduler.schedule()
        if plan.empty:
            return {}
        tokens = self.runner.execute(plan)
        finished: Dict[str, List[int]] = {}
        for seq, tok in zip(plan.seqs, tokens):
            if seq.push(tok):
                self.scheduler.finish(seq)
                finished[seq.request_id] = seq.output()
        return finished

    def has_unfinished_requests(self) -> bool:
        return self.scheduler.pending()

    def generate(self, prompt_token_ids: List[int],
                 sampling_params: Optional[SamplingParams] = None,
                 request_id: str = "sync-0") -> List[int]:
        self.add_request(request_id, prompt_token_ids,
                         sampling_params or SamplingParams(temperature=0.0))
        while self.has_unfinished_requests():
            done = self.step()
            if request_id in done:
                return done[request_id]
        return []
