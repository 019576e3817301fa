"""End-to-end continuous-batching workload: random-init Qwen2-0.5B, synthetic requests.

Qwen2-0.5B shape (24 layers, hidden 896, 14/2 heads, head_dim 64, FFN 4864, vocab
151936), bf16 weights ~N(0, 0.02) with unit norms; 256 requests with prompt ids
uniform over the vocabulary, prompt length U{64..1024}, greedy output length
U{128..512}, no stop tokens, scheduler limits 256 sequences / 8192 batched tokens.
Output tok/s = generated tokens / wall time of the step loop after every request
is submitted (the reference's definition, benchmarks/bench_throughput.py:66-92).
"""
from __future__ import annotations

import time
from typing import Optional

import numpy as np

from .backend.engine import LLMEngine
from .backend.request import SamplingParams
from .model.config import QWEN2_0_5B, ModelConfig

E2E_SEED = 1004


def requests(n: int = 256, seed: int = E2E_SEED, prompt=(64, 1024), output=(128, 512),
             vocab: int = 151936):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        plen = int(rng.integers(prompt[0], prompt[1], endpoint=True))
        olen = int(rng.integers(output[0], output[1], endpoint=True))
        out.append((f"req-{i}", rng.integers(0, vocab, plen).tolist(), olen))
    return out


def build_engine(device: str = "cuda:0", max_gpu_blocks: int = 40000, seed: int = E2E_SEED,
                 model=None, max_num_seqs: int = 256, max_num_batched_tokens: int = 8192,
                 decode_graphs: bool = True, max_model_len: int = 1536):
    return LLMEngine(ModelConfig(**QWEN2_0_5B), max_num_seqs=max_num_seqs,
                     max_num_batched_tokens=max_num_batched_tokens,
                     max_gpu_blocks=max_gpu_blocks, device=device, seed=seed, model=model,
                     decode_graphs=decode_graphs, max_model_len=max_model_len)


def run(engine: LLMEngine, reqs, sync=None, time_limit_s: Optional[float] = None):
    """Submit every request, then step until done; returns (output tokens, seconds, finished)."""
    for rid, prompt, olen in reqs:
        engine.add_request(rid, prompt, SamplingParams(temperature=0.0, max_new_tokens=olen))
    n_tok = 0
    finished = 0
    t0 = time.perf_counter()
    while engine.has_unfinished_requests():
        for _rid, toks in engine.step().items():
            n_tok += len(toks)
            finished += 1
        if time_limit_s is not None and time.perf_counter() - t0 > time_limit_s:
            break
    if sync is not None:
        sync()
    return n_tok, time.perf_counter() - t0, finished


def main(argv=None) -> None:
    """python -m needle_amd.e2e [--requests N]: the benchmark's first N requests on cuda:0,
    printing output tok/s (the command the kernel-trace profiles of this run use)."""
    import argparse

    import torch

    p = argparse.ArgumentParser(description=main.__doc__.splitlines()[0])
    p.add_argument("--requests", type=int, default=256)
    p.add_argument("--time-limit", type=float, default=None)
    args = p.parse_args(argv)
    engine = build_engine()
    reqs = requests(args.requests)
    torch.cuda.synchronize()
    n_tok, secs, finished = run(engine, reqs, sync=torch.cuda.synchronize,
                                time_limit_s=args.time_limit)
    print(f"e2e {len(reqs)} requests: {n_tok} tokens in {secs:.2f} s = {n_tok / secs:.1f} "
          f"tok/s, {finished} finished", flush=True)


if __name__ == "__main__":
    main()
