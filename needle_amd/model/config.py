"""Model configuration parsed from a HuggingFace config.json.

Same fields, defaults and derivation as needle/model/config.py:10-65 of the
reference (head_dim = hidden_size // num_attention_heads, config.py:28-29).
"""
from __future__ import annotations

import json
from dataclasses import dataclass, field
from pathlib import Path


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

    @property
    def is_gqa(self) -> bool:
        return self.num_key_value_heads != self.num_attention_heads

    @classmethod
    def from_pretrained(cls, model_path: str) -> "ModelConfig":
        path = Path(model_path) / "config.json"
        if not path.exists():
            raise FileNotFoundError(f"config.json not found in {model_path}")
        with open(path) as f:
            return cls.from_dict(json.load(f))

    @classmethod
    def from_dict(cls, cfg: dict) -> "ModelConfig":
        return cls(
            model_type=cfg.get("model_type", "llama"),
            hidden_size=cfg.get("hidden_size", 4096),
            num_hidden_layers=cfg.get("num_hidden_layers", 32),
            num_attention_heads=cfg.get("num_attention_heads", 32),
            num_key_value_heads=cfg.get("num_key_value_heads", cfg.get("num_attention_heads", 32)),
            intermediate_size=cfg.get("intermediate_size", 11008),
            vocab_size=cfg.get("vocab_size", 32000),
            max_position_embeddings=cfg.get("max_position_embeddings", 4096),
            rms_norm_eps=cfg.get("rms_norm_eps", 1e-5),
            rope_theta=cfg.get("rope_theta", 10000.0),
            hidden_act=cfg.get("hidden_act", "silu"),
        )


QWEN2_0_5B = dict(model_type="qwen2", hidden_size=896, num_hidden_layers=24,
                  num_attention_heads=14, num_key_value_heads=2, intermediate_size=4864,
                  vocab_size=151936, max_position_embeddings=32768, rms_norm_eps=1e-6,
                  rope_theta=1000000.0)
