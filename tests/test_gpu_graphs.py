"""Decode steps replayed from captured HIP graphs agree with eager decode steps.

The graphs read their metadata from the runner's device-resident rows, which the host
updates with one scatter per step.  Every replay is checked against an eager forward of
the same batch (same weights, same cache, same metadata built from scratch on the host),
with unrelated eager work and synchronisations between the replays; the batch shrinks and
reorders across steps, so rows leave, refill and several buckets are replayed more than
once.  The tokens fed to the next step are the graph's own greedy tokens (written into the
next input ids on the device).  Tolerance as for attention: |graph - eager| <= 2e-2 +
1e-2 |eager| (the padded graph batch may select different GEMM kernels than the eager one).
"""
import numpy as np
import pytest
import torch

from needle_amd.backend.block_allocator import BlockAllocator
from needle_amd.backend.request import SamplingParams, SeqState
from needle_amd.model.config import ModelConfig
from needle_amd.model.runner import ModelRunner

pytestmark = pytest.mark.gpu

CFG = dict(model_type="qwen2", hidden_size=256, num_hidden_layers=2, num_attention_heads=4,
           num_key_value_heads=2, intermediate_size=512, vocab_size=1000,
           max_position_embeddings=512, rms_norm_eps=1e-6, rope_theta=1e6)


def _close(a, b):
    a = a.float().cpu().numpy().astype(np.float64)
    b = b.float().cpu().numpy().astype(np.float64)
    assert np.isfinite(a).all()
    assert (np.abs(a - b) - (2e-2 + 1e-2 * np.abs(b))).max() <= 0, float(np.abs(a - b).max())


def _setup(buckets, lens, seed=5, nb=160, max_model_len=512):
    cfg = ModelConfig(**dict(CFG, max_position_embeddings=max_model_len))
    r = ModelRunner(cfg, device="cuda:0", seed=11)
    r.init_kv_cache(nb)
    r.enable_decode_graphs(max_model_len=max_model_len, buckets=buckets)
    alloc = BlockAllocator(nb - 1, 0, 16)                 # the last block is the scratch block
    rng = np.random.default_rng(seed)
    seqs = []
    for i, n in enumerate(lens):
        s = SeqState(i + 1, f"g{i}", rng.integers(0, cfg.vocab_size, n).tolist(),
                     SamplingParams(temperature=0.0, max_new_tokens=64))
        s.blocks = alloc.allocate_gpu_blocks((n + 1 + 15) // 16 + 4)
        seqs.append(s)
    r.forward(r.prepare_inputs(seqs, is_prefill=True))
    for s in seqs:
        s.kv_ready = True
        s.tokens.append(int(rng.integers(0, cfg.vocab_size)))
    return r, seqs


def _graph_logits(r, live):
    bucket = min(k for k in r._graphs if k >= len(live))
    logits = r._graphs[bucket][1]
    where = r._rows.row_of()
    return logits[torch.tensor([where[id(s)] for s in live], device=logits.device)]


@torch.no_grad()
def test_graph_replays_match_eager_decode():
    r, seqs = _setup((1, 2, 4, 8), [3, 17, 40, 64, 9, 100, 33])
    x = torch.randn(512, 512, device="cuda:0")
    rng = np.random.default_rng(9)
    for step in range(10):
        live = seqs[:max(1, len(seqs) - step)]             # 7, 6, 5, ... sequences
        live = [live[i] for i in rng.permutation(len(live))]
        toks = r._graph_decode(live)
        assert toks is not None
        g = _graph_logits(r, live).clone()
        torch.cuda.synchronize()
        y = x @ x                                          # unrelated eager work between replays
        e = r.forward(r.prepare_inputs(live, is_prefill=False))
        torch.cuda.synchronize()
        _close(g, e)
        assert toks == g.argmax(-1).tolist()
        for s, t in zip(live, toks):
            s.tokens.append(t)
        del y


@torch.no_grad()
def test_larger_eager_batch_does_not_free_a_captured_workspace():
    """Graphs captured for buckets 1 and 2 with 8192-token rows (the stream split, whose
    partials go to the layers' decode workspace); then an eager decode of 8 sequences, one
    of them 4200 tokens long, needs a larger workspace.  The captured one must stay
    allocated: replays keep writing it, and memory handed to new tensors must not change."""
    r, seqs = _setup((1, 2), [4200, 300, 260, 40, 90, 120, 33, 410], seed=6, nb=600,
                     max_model_len=8192)
    before = [len(layer.self_attn._workspaces) for layer in r.model.model.layers]
    e = r.forward(r.prepare_inputs(seqs, is_prefill=False))     # 8 sequences, eager
    torch.cuda.synchronize()
    after = [len(layer.self_attn._workspaces) for layer in r.model.model.layers]
    assert all(a == b + 1 for a, b in zip(after, before)), (before, after)
    junk = [torch.full((1 << 18,), 7.0, device="cuda:0") for _ in range(16)]
    for s, t in zip(seqs, e.argmax(-1).tolist()):
        s.tokens.append(t)
    r._rows.forget_tokens()
    live = seqs[:2]
    for _ in range(3):
        toks = r._graph_decode(live)
        g = _graph_logits(r, live).clone()
        ref = r.forward(r.prepare_inputs(live, is_prefill=False))
        torch.cuda.synchronize()
        _close(g, ref)
        for s, t in zip(live, toks):
            s.tokens.append(t)
    assert all(bool((j == 7.0).all()) for j in junk)
