"""The drop-in Attention layer against the reference's Attention.forward (oracle).

One Qwen2-0.5B-shaped layer (qkv bias, 14/2 heads, head_dim 64), one Llama-3-8B-shaped
layer and one with Qwen2-7B's heads (28/4, head_dim 128, qkv bias): a prefill of three
prompts, then two decode steps,
with the same weights on the GPU layer and on the CPU oracle.  Outputs agree
to the bf16 parity tolerance |gpu - ref| <= 2e-2 + 1e-2 |ref|.  The pools are
compared to the same tolerance after every call (not bit for bit) because the k/v projections run through different
GEMM implementations on the GPU and the CPU; the append itself is checked bit
for bit in test_gpu_append.py.
"""
import numpy as np
import pytest
import torch

from oracle import paged_ref
from needle_amd import workloads as wl
from needle_amd.layers.attention import Attention
from needle_amd.layers.rope import RotaryEmbedding
from needle_amd.model.config import QWEN2_0_5B, ModelConfig

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _close(got, want):
    got = got.detach().float().cpu().numpy().astype(np.float64)
    want = want.detach().float().cpu().numpy().astype(np.float64)
    excess = np.abs(got - want) - (2e-2 + 1e-2 * np.abs(want))
    assert np.isfinite(got).all() and excess.max() <= 0, float(np.abs(got - want).max())


@pytest.mark.parametrize("cfg,bias,lens", [
    (ModelConfig(**QWEN2_0_5B), True, [5, 33, 17]),
    (ModelConfig(hidden_size=4096, num_attention_heads=32, num_key_value_heads=8,
                 rope_theta=500000.0, max_position_embeddings=8192), False, [5, 33, 17]),
    # Qwen2-7B heads (28 / 4, head_dim 128): a group of 7, so a prefill workgroup's eight
    # jobs span two 32-row subtiles; prompts of several subtiles each
    (ModelConfig(hidden_size=3584, num_attention_heads=28, num_key_value_heads=4,
                 rope_theta=1e6, max_position_embeddings=4096), True, [300, 129, 70])])
@torch.no_grad()  # the runner calls the model under no_grad (runner.py:143, 151)
def test_prefill_then_decode_matches_reference(cfg, bias, lens):
    torch.manual_seed(0)
    layer = Attention(cfg, 0, qkv_bias=bias)
    for p in layer.parameters():
        torch.nn.init.normal_(p, std=0.02)
    layer = layer.to(torch.bfloat16)
    weights = {k: v.detach().clone() for k, v in layer.state_dict().items()}
    layer = layer.to(DEV)
    rope = RotaryEmbedding(cfg.head_dim, 4096, cfg.rope_theta).to(torch.bfloat16)

    hkv, d, bs = cfg.num_key_value_heads, cfg.head_dim, 16
    steps = 2
    blocks = [(n + steps + bs - 1) // bs for n in lens]
    nb = sum(blocks) + 4
    tables = wl.tables_by_permutation(blocks, nb, seed=7)
    bt = wl.pad_tables(tables, nb)
    pool_ref = torch.zeros((2, nb, hkv, bs, d), dtype=torch.bfloat16)
    pool_gpu = pool_ref.to(DEV)

    # prefill (runner.py:204-218: context 0, positions 0..n-1)
    t = sum(lens)
    x = torch.randn((t, cfg.hidden_size)).to(torch.bfloat16)
    pos = torch.cat([torch.arange(n) for n in lens])
    cos, sin = rope.get_cos_sin(pos)
    cu = torch.tensor([0] + np.cumsum(lens).tolist(), dtype=torch.int32)
    ctx = torch.zeros(len(lens), dtype=torch.int32)
    want = paged_ref.attention_forward(weights, x, pool_ref, bt, cu, ctx, True, cos, sin,
                                       cfg.num_attention_heads, hkv, d)
    got = layer(x.to(DEV), pos.to(DEV), pool_gpu, bt.to(DEV), cu.to(DEV), ctx.to(DEV),
                max(lens), True, cos.to(DEV), sin.to(DEV))
    torch.cuda.synchronize()
    _close(got, want)
    _close(pool_gpu, pool_ref)

    # decode steps (runner.py:209-218: one token, context = length - 1)
    cur = list(lens)
    for _ in range(steps):
        x = torch.randn((len(lens), cfg.hidden_size)).to(torch.bfloat16)
        pos = torch.tensor(cur)
        cos, sin = rope.get_cos_sin(pos)
        ctx = torch.tensor(cur, dtype=torch.int32)
        cu = torch.arange(len(lens) + 1, dtype=torch.int32)
        want = paged_ref.attention_forward(weights, x, pool_ref, bt, cu, ctx, False, cos, sin,
                                           cfg.num_attention_heads, hkv, d)
        got = layer(x.to(DEV), pos.to(DEV), pool_gpu, bt.to(DEV), cu.to(DEV), ctx.to(DEV), 1,
                    False, cos.to(DEV), sin.to(DEV))
        torch.cuda.synchronize()
        _close(got, want)
        _close(pool_gpu, pool_ref)
        cur = [c + 1 for c in cur]
