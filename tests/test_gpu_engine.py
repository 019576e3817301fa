"""Continuous batching through the HIP path against the reference torch path (oracle).

A small random-init Qwen2 (2 layers, 4/2 heads, head_dim 64) runs scheduler-driven
steps: prompts of different lengths, mixed prefill + decode batches, block-table
growth.  The GPU model (HIP kernels) and a CPU copy of the same weights whose
attention seams are the oracle (attention.py:_prefill/_decode restated) see the
same metadata every step; tokens are teacher-forced from the GPU side.  Logits
must agree to |gpu - ref| <= 2e-2 + 1e-2 |ref|.  Greedy ties on random weights can
flip, so the token streams themselves are not compared here.
"""
import types

import numpy as np
import pytest
import torch

from oracle import paged_ref
from needle_amd.backend.block_allocator import BlockAllocator
from needle_amd.backend.engine import LLMEngine
from needle_amd.backend.scheduler import Scheduler
from needle_amd.backend.sequence import Request, SamplingParams, Sequence
from needle_amd.model.config import ModelConfig
from needle_amd.model.runner import ModelRunner
from needle_amd.model.qwen2 import build_model, random_init_

pytestmark = pytest.mark.gpu

CFG = dict(model_type="qwen2", hidden_size=256, num_hidden_layers=2, num_attention_heads=4,
           num_key_value_heads=2, intermediate_size=512, vocab_size=1000,
           max_position_embeddings=2048, rms_norm_eps=1e-6, rope_theta=1e6)


def _oracle_prefill(self, q, k, v, kv_cache, block_table, cu_seqlens, context_lens, max_seqlen):
    return paged_ref.prefill(q, k, v, kv_cache, block_table, cu_seqlens, context_lens,
                             self.num_heads, self.num_kv_heads)


def _oracle_decode(self, q, k, v, kv_cache, block_table, context_lens):
    return paged_ref.decode(q, k, v, kv_cache, block_table, context_lens, self.scale,
                            self.num_heads, self.num_kv_heads, self.head_dim)


def oracle_runner(cfg, model_cpu):
    r = ModelRunner(cfg, device="cpu", model=model_cpu)
    for layer in r.model.model.layers:
        layer.self_attn.fuse_rope = False       # RoPE as torch ops, then the oracle seams
        layer.self_attn._prefill = types.MethodType(_oracle_prefill, layer.self_attn)
        layer.self_attn._decode = types.MethodType(_oracle_decode, layer.self_attn)
    return r


def _close(got, want):
    got = got.float().cpu().numpy().astype(np.float64)
    want = want.float().numpy().astype(np.float64)
    excess = np.abs(got - want) - (2e-2 + 1e-2 * np.abs(want))
    assert np.isfinite(got).all() and excess.max() <= 0, float(np.abs(got - want).max())


@torch.no_grad()
def test_continuous_batching_logits_match_reference_path():
    cfg = ModelConfig(**CFG)
    model = random_init_(build_model(cfg), seed=3)
    gpu = ModelRunner(cfg, device="cuda:0", model=build_model(cfg))
    gpu.model.load_state_dict(model.state_dict())
    gpu.model.to(torch.bfloat16)
    cpu = oracle_runner(cfg, model)
    nb = 64
    gpu.init_kv_cache(nb)
    cpu.init_kv_cache(nb)
    sched = Scheduler(BlockAllocator(nb, 0, 16), max_num_seqs=8, max_num_batched_tokens=600)
    rng = np.random.default_rng(0)
    lens = [5, 31, 16, 70, 1, 120]
    for i, n in enumerate(lens):
        req = Request(f"r{i}", rng.integers(0, cfg.vocab_size, n).tolist(),
                      SamplingParams(temperature=0.0, max_new_tokens=6 + i))
        sched.add_sequence(Sequence(i + 1, req, list(req.prompt_token_ids),
                                    list(range((n + 15) // 16)), 16))
    steps = agree = total = 0
    while sched.has_unfinished_seqs() and steps < 40:
        out = sched.schedule()
        seqs, logits = [], []
        for group in (out.prefill_seqs, out.decode_seqs):
            if not group:
                continue
            pre = not group[0].prefilled
            lg = gpu.forward(gpu.prepare_inputs(group, out.block_tables, pre))
            lc = cpu.forward(cpu.prepare_inputs(group, out.block_tables, pre))
            torch.cuda.synchronize()
            _close(lg, lc)
            seqs += group
            logits.append((lg.float().cpu(), lc.float()))
        for s in out.prefill_seqs:
            s.prefilled = True
        toks = torch.cat([g for g, _ in logits]).argmax(-1).tolist()
        ref = torch.cat([c for _, c in logits]).argmax(-1).tolist()
        agree += sum(a == b for a, b in zip(toks, ref))
        total += len(toks)
        for s, t in zip(seqs, toks):
            s.append_token(t)
            if s.num_generated_tokens >= s.request.sampling_params.max_new_tokens:
                sched.free_sequence(s)
        steps += 1
    assert not sched.has_unfinished_seqs()
    print(f"greedy agreement {agree}/{total}")


@torch.no_grad()
def test_engine_runs_requests_to_completion():
    cfg = ModelConfig(**CFG)
    eng = LLMEngine(cfg, max_gpu_blocks=256, seed=1)
    rng = np.random.default_rng(1)
    want = {}
    for i in range(12):
        n_out = int(rng.integers(1, 20))
        want[f"q{i}"] = n_out
        eng.add_request(f"q{i}", rng.integers(0, cfg.vocab_size, int(rng.integers(1, 200))).tolist(),
                        SamplingParams(temperature=0.0, max_new_tokens=n_out))
    got = {}
    while eng.has_unfinished_requests():
        got.update(eng.step())
    assert {k: len(v) for k, v in got.items()} == want
    assert eng.allocator.num_free_gpu_blocks == 256
    assert all(0 <= t < cfg.vocab_size for v in got.values() for t in v)
    # the same greedy request twice gives the same tokens (the cache is reused correctly)
    a = eng.generate([5, 6, 7] * 20, SamplingParams(temperature=0.0, max_new_tokens=8), "a")
    b = eng.generate([5, 6, 7] * 20, SamplingParams(temperature=0.0, max_new_tokens=8), "b")
    assert a == b and len(a) == 8
