"""Host-side pieces of the continuous-batching driver: sampler and batch metadata."""
import torch

from needle_amd.backend.sequence import Request, SamplingParams, Sequence
from needle_amd.model.config import ModelConfig
from needle_amd.model.runner import ModelRunner
from needle_amd.model.sampler import sample


def test_greedy_and_degenerate_stochastic_rows_agree():
    torch.manual_seed(0)
    logits = torch.randn(5, 50)
    want = logits.argmax(-1).tolist()
    assert sample(logits, [SamplingParams(temperature=0.0)] * 5) == want
    g = torch.Generator().manual_seed(1)
    # top_k = 1 (and a tiny top_p) leave only the argmax
    assert sample(logits, [SamplingParams(temperature=0.7, top_k=1)] * 5, g) == want
    assert sample(logits, [SamplingParams(temperature=0.7, top_p=1e-6)] * 5, g) == want


def _seq(seq_id, toks, gen=0):
    req = Request(f"r{seq_id}", list(toks[:len(toks) - gen]), SamplingParams(temperature=0))
    s = Sequence(seq_id, req, list(toks), [], 16)
    s.num_generated_tokens = gen
    return s


def test_prepare_inputs_matches_the_reference_rules():
    cfg = ModelConfig(hidden_size=128, num_hidden_layers=1, num_attention_heads=2,
                      num_key_value_heads=1, intermediate_size=64, vocab_size=32,
                      max_position_embeddings=64)
    r = ModelRunner(cfg, device="cpu")
    r.init_kv_cache(10)
    a, b = _seq(1, list(range(5))), _seq(2, list(range(20)))
    tables = {1: [3], 2: [7, 2]}
    inp = r.prepare_inputs([a, b], tables, is_prefill=True)
    assert inp.input_ids.tolist() == list(range(5)) + list(range(20))
    assert inp.position_ids.tolist() == list(range(5)) + list(range(20))
    assert inp.cu_seqlens.tolist() == [0, 5, 25] and inp.cu_seqlens.dtype == torch.int32
    assert inp.context_lens.tolist() == [0, 0]
    assert inp.block_table.tolist() == [[3, 9], [7, 2]]   # padded with num_blocks - 1
    assert inp.max_seqlen == 20 and inp.is_prefill
    a.prefilled = b.prefilled = True
    inp = r.prepare_inputs([a, b], tables, is_prefill=False)
    assert inp.input_ids.tolist() == [4, 19] and inp.position_ids.tolist() == [4, 19]
    assert inp.context_lens.tolist() == [4, 19] and inp.cu_seqlens.tolist() == [0, 1, 2]
