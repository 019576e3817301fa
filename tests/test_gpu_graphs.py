"""Decode steps replayed from captured HIP graphs agree with eager decode steps.

Every replay is checked against an eager forward of the same batch (same weights,
same cache, same metadata), with unrelated eager work and synchronisations between
the replays; the batch shrinks across steps so several buckets are replayed more
than once.  Tolerance as for attention: |graph - eager| <= 2e-2 + 1e-2 |eager| (the
padded graph batch may select different GEMM kernels than the eager one).
"""
import numpy as np
import pytest
import torch

from needle_amd.backend.block_allocator import BlockAllocator
from needle_amd.backend.sequence import Request, SamplingParams, Sequence
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


@torch.no_grad()
def test_graph_replays_match_eager_decode():
    cfg = ModelConfig(**CFG)
    r = ModelRunner(cfg, device="cuda:0", seed=11)
    nb = 96
    r.init_kv_cache(nb)
    r.enable_decode_graphs(max_model_len=512, buckets=(1, 2, 4, 8))
    alloc = BlockAllocator(nb - 1, 0, 16)                 # the last block is the scratch block
    rng = np.random.default_rng(5)
    seqs, tables = [], {}
    for i, n in enumerate([3, 17, 40, 64, 9, 100, 33]):
        req = Request(f"g{i}", rng.integers(0, cfg.vocab_size, n).tolist(),
                      SamplingParams(temperature=0.0, max_new_tokens=64))
        s = Sequence(i + 1, req, list(req.prompt_token_ids), [], 16)
        tables[s.seq_id] = alloc.allocate_gpu_blocks((n + 1 + 15) // 16 + 4)
        seqs.append(s)
    r.forward(r.prepare_inputs(seqs, tables, is_prefill=True))
    for s in seqs:
        s.prefilled = True
        s.append_token(int(rng.integers(0, cfg.vocab_size)))
    x = torch.randn(512, 512, device="cuda:0")
    replays = 0
    for step in range(8):
        live = seqs[:max(1, len(seqs) - step)]             # 7, 6, 5, ... sequences
        g = r._graph_decode(live, tables)
        assert g is not None
        g = g.clone()
        torch.cuda.synchronize()
        y = x @ x                                          # unrelated eager work between replays
        e = r.forward(r.prepare_inputs(live, tables, is_prefill=False))
        torch.cuda.synchronize()
        _close(g, e)
        replays += 1
        for s, t in zip(live, e.argmax(-1).tolist()):
            s.append_token(t)
        del y
    assert replays == 8
