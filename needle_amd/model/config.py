"""Model configuration: the fields of a HuggingFace config.json that the model and the
attention layer read.

Same fields, defaults and derivation as needle/model/config.py:10-31 of the reference
(head_dim = hidden_size // num_attention_heads, config.py:28-29).  The benchmark models are
random-init, so nothing here reads a checkpoint directory.
"""
from __future__ import annotations

from dataclasses import dataclass, field


@dataclass
class ModelConfig:
    model_type: str = "llama"
    hidden_size: int = 4096
    num_hidden_layers: int = 32
    num_attention_heads: int = 32
    num_key_value_heads: int = 32
    intermediate_size: int = 11008
    vocab_size: int = 32000
    max_position_embeddings: int = 4096
    rms_norm_eps: float = 1e-5
    rope_theta: float = 10000.0
    hidden_act: str = "silu"
    head_dim: int = field(init=False)

    def __post_init__(self):
        self.head_dim = self.hidden_size // self.num_attention_heads

    @property
    def num_kv_heads(self) -> int:
        return self.num_key_value_heads


QWEN2_0_5B = dict(model_type="qwen2", hidden_size=896, num_hidden_layers=24,
                  num_attention_heads=14, num_key_value_heads=2, intermediate_size=4864,
                  vocab_size=151936, max_position_embeddings=32768, rms_norm_eps=1e-6,
                  rope_theta=1000000.0)
