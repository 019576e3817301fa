"""Rotary embedding cos/sin tables (reference needle/layers/rope.py:10-27).

inv_freq = 1 / base^(2i/D); table[t] = cat(t*inv_freq, t*inv_freq); cos/sin in
fp32, cast with the model dtype by module.to(dtype) (needle/model/runner.py:34).
"""
from __future__ import annotations

import torch
import torch.nn as nn


class RotaryEmbedding(nn.Module):
    def __init__(self, head_dim: int, max_seq_len: int, base: float = 10000.0):
        super().__init__()
        inv_freq = 1.0 / (base ** (torch.arange(0, head_dim, 2).float() / head_dim))
        self.register_buffer("inv_freq", inv_freq, persistent=False)
        t = torch.arange(max_seq_len, dtype=torch.float32)
        freqs = torch.outer(t, inv_freq)
        emb = torch.cat([freqs, freqs], dim=-1)
        self.register_buffer("cos_cached", emb.cos(), persistent=False)
        self.register_buffer("sin_cached", emb.sin(), persistent=False)

    def get_cos_sin(self, positions: torch.Tensor):
        return self.cos_cached[positions], self.sin_cached[positions]
