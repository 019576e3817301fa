"""The KV swap on the GPU: ndl_kv_block_copy and the runner/engine paths that use it.

Reference: needle/model/runner.py:107-116,175-192 (the swap copies before the forward),
needle/backend/scheduler.py:54-67,90-109 (resume / evict), block_allocator.py:88-106.

  * kernel: random GPU pools and pinned CPU pools, several layers, scattered block pairs;
    every destination block equals its source byte for byte, nothing else changes, pairs
    with an out-of-range id are skipped;
  * runner: a sequence decodes, its blocks go to the CPU pool, the GPU copies are
    overwritten, it comes back into other GPU blocks and keeps decoding; its logits equal,
    bit for bit, those of a runner that never swapped it;
  * engine: a small GPU pool with a CPU pool; the scheduler evicts and resumes sequences
    while every request runs to completion with clean block accounting.
"""
import numpy as np
import pytest
import torch

from needle_amd import ops
from needle_amd.backend.engine import LLMEngine
from needle_amd.backend.request import SamplingParams, SeqState
from needle_amd.model.config import ModelConfig
from needle_amd.model.runner import ModelRunner
from needle_amd.model.qwen2 import build_model, random_init_

pytestmark = pytest.mark.gpu
DEV = "cuda:0"

CFG = dict(model_type="qwen2", hidden_size=256, num_hidden_layers=3, num_attention_heads=4,
           num_key_value_heads=2, intermediate_size=512, vocab_size=1000,
           max_position_embeddings=2048, rms_norm_eps=1e-6, rope_theta=1e6)


def _bits(t):
    return t.view(torch.int16)


@pytest.mark.parametrize("hkv,d", [(2, 64), (8, 128)])
def test_block_copy_both_directions(hkv, d):
    g = torch.Generator(device="cpu").manual_seed(hkv * d)
    layers, n_gpu, n_cpu = 5, 300, 120
    gpu = [torch.randn((2, n_gpu, hkv, 16, d), generator=g).to(torch.bfloat16).to(DEV)
           for _ in range(layers)]
    cpu = [torch.randn((2, n_cpu, hkv, 16, d), generator=g).to(torch.bfloat16).pin_memory()
           for _ in range(layers)]
    rng = np.random.default_rng(hkv)
    src = rng.choice(n_gpu, 90, replace=False).tolist()
    dst = rng.choice(n_cpu, 90, replace=False).tolist()
    # out: GPU -> pinned CPU; ids on the GPU
    want = [c.clone() for c in cpu]
    for w, gp in zip(want, gpu):
        w[:, dst] = gp[:, src].cpu()
    ops.kv_block_copy(cpu, gpu, torch.tensor(src, dtype=torch.int32, device=DEV),
                      torch.tensor(dst, dtype=torch.int32, device=DEV))
    torch.cuda.synchronize()
    for c, w in zip(cpu, want):
        assert torch.equal(_bits(c), _bits(w))
    # in: pinned CPU -> GPU, ids in pinned host memory, one pair out of range (skipped)
    src2 = rng.choice(n_cpu, 40, replace=False).tolist()
    dst2 = rng.choice(n_gpu, 40, replace=False).tolist()
    src2[7] = n_cpu + 3
    want = [gp.cpu() for gp in gpu]
    for w, c in zip(want, cpu):
        keep = [i for i in range(40) if i != 7]
        w[:, [dst2[i] for i in keep]] = c[:, [src2[i] for i in keep]]
    ops.kv_block_copy(gpu, cpu, torch.tensor(src2, dtype=torch.int32).pin_memory(),
                      torch.tensor(dst2, dtype=torch.int32).pin_memory())
    torch.cuda.synchronize()
    for gp, w in zip(gpu, want):
        assert torch.equal(_bits(gp.cpu()), _bits(w))


def test_block_copy_rejects_pageable_host_memory():
    gpu = [torch.zeros((2, 4, 2, 16, 64), dtype=torch.bfloat16, device=DEV)]
    cpu = [torch.zeros((2, 4, 2, 16, 64), dtype=torch.bfloat16)]      # not pinned
    ids = torch.zeros(1, dtype=torch.int32, device=DEV)
    with pytest.raises(ValueError):
        ops.kv_block_copy(cpu, gpu, ids, ids)


def _runner(model, nb, n_cpu=0):
    r = ModelRunner(ModelConfig(**CFG), device=DEV, model=model)
    r.init_kv_cache(nb, n_cpu)
    return r


@torch.no_grad()
def test_swapped_sequence_decodes_exactly_as_an_unswapped_one():
    cfg = ModelConfig(**CFG)
    base = random_init_(build_model(cfg), seed=21)
    ma, mb = build_model(cfg), build_model(cfg)
    ma.load_state_dict(base.state_dict())
    mb.load_state_dict(base.state_dict())
    a, b = _runner(ma, 64), _runner(mb, 64, n_cpu=32)
    prompt = np.random.default_rng(2).integers(0, cfg.vocab_size, 50).tolist()
    sa = SeqState(1, "a", prompt, SamplingParams(temperature=0.0))
    sb = SeqState(1, "b", prompt, SamplingParams(temperature=0.0))
    sa.blocks = [0, 1, 2, 3, 4]
    sb.blocks = [10, 11, 12, 13, 14]

    def step(prefill):
        la = a.forward(a.prepare_inputs([sa], is_prefill=prefill))
        lb = b.forward(b.prepare_inputs([sb], is_prefill=prefill))
        torch.cuda.synchronize()
        assert torch.equal(_bits(la), _bits(lb))
        tok = int(la.argmax(-1)[0])
        sa.tokens.append(tok)
        sb.tokens.append(tok)

    step(True)
    for _ in range(3):
        step(False)
    cpu_ids = [5, 9, 6, 30, 0]
    b.swap(dict(zip(sb.blocks, cpu_ids)), to_cpu=True)
    for pool in b.kv_caches:                           # the GPU copies are gone
        pool[:, sb.blocks] = torch.randn_like(pool[:, sb.blocks])
    new_ids = [40, 17, 33, 63, 2]
    b.swap(dict(zip(cpu_ids, new_ids)), to_cpu=False)
    torch.cuda.synchronize()
    for pa, pb in zip(a.kv_caches, b.kv_caches):
        assert torch.equal(_bits(pa[:, sa.blocks]), _bits(pb[:, new_ids]))
    sb.blocks = new_ids
    for _ in range(4):
        step(False)


@torch.no_grad()
def test_engine_with_cpu_pool_swaps_and_finishes():
    cfg = ModelConfig(**CFG)
    per_block = 2 * 2 * 16 * 64 * 2 * cfg.num_hidden_layers
    eng = LLMEngine(cfg, max_gpu_blocks=24, cpu_swap_bytes=40 * per_block, seed=4,
                    max_num_seqs=8, max_num_batched_tokens=4096)
    assert eng.allocator.num_free_cpu_blocks == 40
    swaps = {"in": 0, "out": 0}
    real_swap = eng.runner.swap

    def counting_swap(mapping, to_cpu):
        swaps["out" if to_cpu else "in"] += len(mapping)
        real_swap(mapping, to_cpu)
    eng.runner.swap = counting_swap
    rng = np.random.default_rng(3)
    want = {}
    for i in range(6):
        n_out = int(rng.integers(20, 60))
        want[f"s{i}"] = n_out
        eng.add_request(f"s{i}", rng.integers(0, cfg.vocab_size, int(rng.integers(20, 60))).tolist(),
                        SamplingParams(temperature=0.0, max_new_tokens=n_out))
    got = {}
    steps = 0
    while eng.has_unfinished_requests() and steps < 2000:
        got.update(eng.step())
        steps += 1
    assert {k: len(v) for k, v in got.items()} == want
    assert swaps["out"] > 0 and swaps["in"] == swaps["out"]
    assert eng.allocator.num_free_gpu_blocks == 24 and eng.allocator.num_free_cpu_blocks == 40
