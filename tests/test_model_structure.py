"""The model's residual stream against the reference's decoder layer, on the CPU.

needle_amd/model/qwen2.py hands each layer's residual stream to the RMSNorm that follows it
(the next layer's input norm, or the final norm), which forms `x + residual` itself; the
reference's layer adds the residual explicitly (needle/model/qwen2.py:52-65):
    residual = h; h = input_layernorm(h); h = self_attn(h, ...); h = residual + h
    residual = h; h = post_attention_layernorm(h); h = mlp(h); h = residual + h
and its model applies the final norm to the last layer's output (qwen2.py:85-90).  Run op for
op with the same modules and weights on the CPU (torch's ops, the oracle's attention seams),
both orders must give the same logits bit for bit, for mixed prefill and decode steps of a
toy Qwen2 and for a toy Llama (no q/k/v bias).
"""
import types

import pytest
import torch

import logits_spread as ls
from needle_amd import e2e
from needle_amd.backend.request import SamplingParams, SeqState
from needle_amd.model.config import ModelConfig
from needle_amd.model.qwen2 import build_model, random_init_
from needle_amd.model.runner import ModelRunner

TOY = dict(hidden_size=256, num_hidden_layers=3, num_attention_heads=4,
           num_key_value_heads=2, intermediate_size=512, vocab_size=1000,
           max_position_embeddings=2048, rms_norm_eps=1e-6, rope_theta=1e6)


def reference_forward(model, batch, kv_caches):
    """The reference's decoder stack (qwen2.py:52-65, :80-90, :100-109) on the same modules."""
    m = model.model
    cos, sin = m.rotary_emb.get_cos_sin(batch.positions)
    h = m.embed_tokens(batch.input_ids)
    for i, layer in enumerate(m.layers):
        residual = h
        x = layer.input_layernorm(h)
        x = layer.self_attn(x, batch.positions, kv_caches[i], batch.block_table,
                            batch.cu_seqlens, batch.context_lens, batch.max_seqlen,
                            batch.is_prefill, cos, sin)
        h = residual + x
        residual = h
        x = layer.mlp(layer.post_attention_layernorm(h))
        h = residual + x
    h = m.norm(h)
    last = h[batch.cu_seqlens[1:].long() - 1] if batch.is_prefill else h
    return model.lm_head(last)


@pytest.mark.parametrize("model_type,dtype", [("qwen2", torch.bfloat16), ("llama", torch.bfloat16),
                                              ("qwen2", torch.float32)])
@torch.no_grad()
def test_residual_stream_matches_the_reference_layer(model_type, dtype):
    cfg = ModelConfig(model_type=model_type, **TOY)
    runners = []
    for _ in range(2):
        model = random_init_(build_model(cfg), e2e.E2E_SEED)
        r = ModelRunner(cfg, 16, dtype=str(dtype).split(".")[1], device="cpu", model=model)
        for layer in r.model.model.layers:          # the oracle's attention seams
            att = layer.self_attn
            att.fuse_rope = False
            att._prefill = types.MethodType(ls._prefill(None), att)
            att._decode = types.MethodType(ls._decode(None), att)
        r.init_kv_cache(400)
        runners.append(r)
    new, ref = runners
    sched = ls.scheduler(400)
    g = torch.Generator().manual_seed(7)
    for i in range(5):       # prompts of 20-90 tokens; the first two stop early (mixed steps)
        n = int(torch.randint(20, 90, (1,), generator=g))
        prompt = torch.randint(0, TOY["vocab_size"], (n,), generator=g).tolist()
        sched.add(SeqState(i + 1, f"r{i}", prompt,
                           SamplingParams(temperature=0.0, max_new_tokens=3 if i < 2 else 7)))
    forwards = 0
    while sched.pending():
        plan = sched.schedule()
        picks = []
        for group, pre in ((plan.prefill, True), (plan.decode, False)):
            if not group:
                continue
            a = new.forward(new.prepare_inputs(group, pre))
            b = reference_forward(ref.model, ref.prepare_inputs(group, pre), ref.kv_caches)
            assert a.dtype == dtype and torch.equal(a, b), f"forward {forwards} differs"
            picks += a.float().argmax(-1).tolist()
            forwards += 1
        for s in plan.prefill:
            s.kv_ready = True
        for s, t in zip(plan.seqs, picks):
            if s.push(t):
                sched.finish(s)
    for x, y in zip(new.kv_caches, ref.kv_caches):
        assert torch.equal(x, y)
    assert forwards >= 6


@pytest.mark.parametrize("bias", [True, False])
def test_fused_projection_check(bias):
    """fused_outputs uses the one GEMM over the fused weight only while every layer's weight
    (and bias) is still the view fuse_linears made at that layer's own rows; otherwise each
    layer runs its own GEMM.  Two equal-sized layers with their parameters swapped stay
    views of the fused tensor, at each other's rows: the check must see that too."""
    from torch import nn
    from needle_amd.layers.attention import _still_fused, fuse_linears, fused_outputs

    def layers():
        torch.manual_seed(5)
        mods = [nn.Linear(32, n, bias=bias, dtype=torch.float64) for n in (48, 16, 16)]
        return mods, fuse_linears(*mods)

    x = torch.randn(5, 32, dtype=torch.float64)
    mods, fused = layers()
    assert _still_fused(fused, mods)
    want = [m(x) for m in mods]
    for got, ref in zip(fused_outputs(fused, mods, x), want):
        torch.testing.assert_close(got, ref, rtol=1e-12, atol=1e-12)

    mods, fused = layers()                     # k and v parameters swapped: views, wrong rows
    mods[1].weight, mods[2].weight = mods[2].weight, mods[1].weight
    if bias:
        mods[1].bias, mods[2].bias = mods[2].bias, mods[1].bias
    assert not _still_fused(fused, mods)
    for got, m in zip(fused_outputs(fused, mods, x), mods):
        assert torch.equal(got, m(x))

    mods, fused = layers()                     # a replaced weight (a load that assigns)
    mods[0].weight = nn.Parameter(mods[0].weight.detach().clone())
    assert not _still_fused(fused, mods)

    mods, fused = layers()                     # a moved layer gets storage of its own
    mods[2].to(torch.float32)
    assert not _still_fused(fused, mods)

    if bias:
        mods, fused = layers()                 # only a bias replaced
        mods[2].bias = nn.Parameter(mods[2].bias.detach().clone())
        assert not _still_fused(fused, mods)
        mods, fused = layers()                 # a bias dropped
        mods[1].bias = None
        assert not _still_fused(fused, mods)
