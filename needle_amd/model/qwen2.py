"""Qwen2 / Llama decoder models around the paged-KV Attention.

Structure and parameter names follow needle/model/qwen2.py:22-109 and
needle/model/llama.py:18-140 of the reference:
  decoder layer = RMSNorm -> Attention (+residual) -> RMSNorm -> SwiGLU MLP (+residual)
  (qwen2.py:52-65); SwiGLU = down(silu(gate(x)) * up(x)) (llama.py:36-37);
  each residual add is done by the RMSNorm that follows it (the next layer's input norm,
  or the final norm), so a layer returns its MLP output and the residual stream apart
  (the same values: the norm rounds x + residual to the dtype first, as the add did);
  Qwen2 adds biases to q/k/v (qwen2.py:22-39); the causal-LM head applies
  lm_head to the last token of each prefill sequence, or to every decode token
  (qwen2.py:100-109).
Tensor parallelism is not built (one GPU).
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from .. import ops
from ..layers.attention import Attention, fuse_linears, fused_outputs
from ..layers.norm import RMSNorm
from ..layers.rope import RotaryEmbedding
from .config import ModelConfig


class MLP(nn.Module):
    def __init__(self, config: ModelConfig):
        super().__init__()
        self.gate_proj = nn.Linear(config.hidden_size, config.intermediate_size, bias=False)
        self.up_proj = nn.Linear(config.hidden_size, config.intermediate_size, bias=False)
        self.down_proj = nn.Linear(config.intermediate_size, config.hidden_size, bias=False)
        self._gate_up = None   # fused gate/up projection (fuse_projections)

    def fuse_projections(self) -> None:
        """One GEMM for the gate and up projections (they read the same input)."""
        self._gate_up = fuse_linears(self.gate_proj, self.up_proj)

    def forward(self, x):
        gate, up = fused_outputs(self._gate_up, (self.gate_proj, self.up_proj), x)
        if x.is_cuda:   # one HIP kernel, torch's roundings
            shape = gate.shape
            act = ops.silu_mul(gate.reshape(-1, shape[-1]), up.reshape(-1, shape[-1]))
            return self.down_proj(act.view(shape))
        return self.down_proj(F.silu(gate) * up)


class DecoderLayer(nn.Module):
    def __init__(self, config: ModelConfig, layer_idx: int, qkv_bias: bool):
        super().__init__()
        self.self_attn = Attention(config, layer_idx, qkv_bias=qkv_bias)
        self.mlp = MLP(config)
        self.input_layernorm = RMSNorm(config.hidden_size, eps=config.rms_norm_eps)
        self.post_attention_layernorm = RMSNorm(config.hidden_size, eps=config.rms_norm_eps)

    def forward(self, hidden_states, positions, kv_cache, block_table, cu_seqlens, context_lens,
                max_seqlen, is_prefill, cos, sin, residual=None):
        """Returns (MLP output, residual stream): the layer's output is their sum, which the
        next RMSNorm forms (qwen2.py:58-65).  residual is None for the first layer, whose
        input is the residual stream itself."""
        if residual is None:
            residual = hidden_states
            h = self.input_layernorm(hidden_states)
        else:
            h, residual = self.input_layernorm(hidden_states, residual)
        h = self.self_attn(h, positions, kv_cache, block_table, cu_seqlens, context_lens,
                           max_seqlen, is_prefill, cos, sin)
        h, residual = self.post_attention_layernorm(h, residual)
        return self.mlp(h), residual


class DecoderModel(nn.Module):
    def __init__(self, config: ModelConfig, qkv_bias: bool):
        super().__init__()
        self.embed_tokens = nn.Embedding(config.vocab_size, config.hidden_size)
        self.layers = nn.ModuleList(
            [DecoderLayer(config, i, qkv_bias) for i in range(config.num_hidden_layers)])
        self.norm = RMSNorm(config.hidden_size, eps=config.rms_norm_eps)
        self.rotary_emb = RotaryEmbedding(config.head_dim, config.max_position_embeddings,
                                          config.rope_theta)

    def forward(self, input_ids, positions, kv_caches, block_table, cu_seqlens, context_lens,
                max_seqlen, is_prefill):
        cos, sin = self.rotary_emb.get_cos_sin(positions)
        h = self.embed_tokens(input_ids)
        residual = None
        for i, layer in enumerate(self.layers):
            h, residual = layer(h, positions, kv_caches[i], block_table, cu_seqlens,
                                context_lens, max_seqlen, is_prefill, cos, sin, residual)
        return self.norm(h, residual)[0]


class CausalLM(nn.Module):
    """Qwen2ForCausalLM (qkv_bias=True) / LlamaForCausalLM (qkv_bias=False)."""

    def __init__(self, config: ModelConfig, qkv_bias: bool):
        super().__init__()
        self.config = config
        self.model = DecoderModel(config, qkv_bias)
        self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False)

    def forward(self, input_ids, positions, kv_caches, block_table, cu_seqlens, context_lens,
                max_seqlen, is_prefill):
        h = self.model(input_ids, positions, kv_caches, block_table, cu_seqlens, context_lens,
                       max_seqlen, is_prefill)
        last = h[cu_seqlens[1:].long() - 1] if is_prefill else h
        return self.lm_head(last)


def fuse_projections(model: nn.Module) -> nn.Module:
    """Runs every layer's q/k/v and gate/up projections as one GEMM each (the weights
    concatenated, the parameters views of them); call once the weights are in place and the
    model is on its device."""
    for m in model.modules():
        if m is not model and hasattr(m, "fuse_projections"):
            m.fuse_projections()
    return model


def build_model(config: ModelConfig) -> CausalLM:
    """needle/model/__init__.py:8: qwen2 -> Qwen2ForCausalLM, otherwise Llama."""
    return CausalLM(config, qkv_bias=config.model_type == "qwen2")


@torch.no_grad()
def random_init_(model: nn.Module, seed: int, std: float = 0.02) -> nn.Module:
    """Synthetic weights: every Linear/Embedding weight and bias ~N(0, std), norms = 1."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    for name, p in model.named_parameters():
        if name.endswith("layernorm.weight") or name.endswith("norm.weight"):
            p.fill_(1.0)
        else:
            p.copy_(torch.randn(p.shape, generator=g) * std)
    return model
