"""Drop-in replacement for needle/layers/attention.py:Attention on MI355X.

Same constructor, the same forward() signature and meaning
(attention.py:36-96), the same parameter names (q_proj/k_proj/v_proj/o_proj),
and the same KV pool layout [2, num_blocks, num_kv_heads, block_size,
head_dim].  Projections stay torch GEMMs (attention.py:84-86).  The rest of
forward is, bit-exact with the reference's bf16 rounding of RoPE (attention.py:88,
277-288):

  prefill (attention.py:88, 102-107): ndl_rope_kv_append with q = NULL (RoPE of k, the
          append of k and v), then ndl_rope_varlen_prefill, which rotates each query row
          as it reads q: no rotated q is written or read back
  decode  (attention.py:88, 140-159): ndl_rope_paged_decode_append, one launch for RoPE,
          the append and the attention (plus the merge launch of the stream split)

The reference's two seams stay available with their own signatures, taking
q and k already rotated, for callers that apply RoPE themselves
(fuse_rope = False selects them inside forward):

  _prefill  (attention.py:102-107): ndl_kv_append (varlen) + ndl_varlen_prefill
  _decode   (attention.py:140-159): ndl_paged_decode_append (the one-token-per-sequence
                                    append and the attention in one launch)

No host synchronisation happens on either path: the decode split-K grid is
sized from block_table's width, prefill from max_seqlen (both host-known).

Tensor parallelism (tp_size > 1) is not built: one GPU holds every head.
With context_lens > 0 in prefill the cached prefix is attended; the
reference ignores it there (its TODO.md:29-32 records that as a bug), and its
runner only ever passes 0 for prefill (runner.py:204-208).
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn

from .. import ops
from ..model.config import ModelConfig


def apply_rope(q, k, cos, sin):
    """attention.py:277-283: x*cos + rotate_half(x)*sin on q [T,H,D] and k [T,Hkv,D]."""
    cos = cos.unsqueeze(1)
    sin = sin.unsqueeze(1)
    return q * cos + rotate_half(q) * sin, k * cos + rotate_half(k) * sin


def rotate_half(x):
    """attention.py:286-288."""
    half = x.shape[-1] // 2
    return torch.cat([-x[..., half:], x[..., :half]], dim=-1)


class Attention(nn.Module):
    """MHA / GQA attention over the paged KV cache (reference attention.py:33)."""

    def __init__(self, config: ModelConfig, layer_idx: int, tp_size: int = 1, tp_rank: int = 0,
                 qkv_bias: bool = False):
        super().__init__()
        if tp_size != 1:
            raise NotImplementedError("needle_amd runs every head on one GPU (tp_size=1)")
        self.layer_idx = layer_idx
        self.num_heads = config.num_attention_heads
        self.num_kv_heads = config.num_key_value_heads
        self.head_dim = config.head_dim
        self.scale = 1.0 / math.sqrt(self.head_dim)
        hidden = config.hidden_size
        self.q_proj = nn.Linear(hidden, self.num_heads * self.head_dim, bias=qkv_bias)
        self.k_proj = nn.Linear(hidden, self.num_kv_heads * self.head_dim, bias=qkv_bias)
        self.v_proj = nn.Linear(hidden, self.num_kv_heads * self.head_dim, bias=qkv_bias)
        self.o_proj = nn.Linear(self.num_heads * self.head_dim, hidden, bias=False)
        # Decode workspaces, newest last.  A grown workspace never frees the older ones: a
        # HIP graph captured with an older one keeps writing it on every replay.
        self._workspaces = []
        self.fuse_rope = True

    def forward(self, hidden_states: torch.Tensor, positions: torch.Tensor,
                kv_cache: torch.Tensor, block_table: torch.Tensor, cu_seqlens: torch.Tensor,
                context_lens: torch.Tensor, max_seqlen: int, is_prefill: bool,
                cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
        total = hidden_states.shape[0]
        q = self.q_proj(hidden_states).view(total, self.num_heads, self.head_dim)
        k = self.k_proj(hidden_states).view(total, self.num_kv_heads, self.head_dim)
        v = self.v_proj(hidden_states).view(total, self.num_kv_heads, self.head_dim)
        if self.fuse_rope:
            if is_prefill:
                ops.rope_kv_append(None, k, v, cos, sin, kv_cache, block_table, context_lens,
                                   cu_seqlens)
                out = self._prefill_attend(q, kv_cache, block_table, cu_seqlens, context_lens,
                                           max_seqlen, cos=cos, sin=sin)
            else:
                out = self._decode_attend(q, kv_cache, block_table, context_lens, new_k=k,
                                          new_v=v, cos=cos, sin=sin)
        else:
            q, k = apply_rope(q, k, cos, sin)
            if is_prefill:
                out = self._prefill(q, k, v, kv_cache, block_table, cu_seqlens, context_lens,
                                    max_seqlen)
            else:
                out = self._decode(q, k, v, kv_cache, block_table, context_lens)
        return self.o_proj(out.view(total, self.num_heads * self.head_dim))

    def _prefill(self, q, k, v, kv_cache, block_table, cu_seqlens, context_lens, max_seqlen):
        ops.write_kv(k, v, kv_cache, block_table, cu_seqlens, context_lens)
        return self._prefill_attend(q, kv_cache, block_table, cu_seqlens, context_lens,
                                    max_seqlen)

    def _prefill_attend(self, q, kv_cache, block_table, cu_seqlens, context_lens, max_seqlen,
                        cos=None, sin=None):
        """Prefill attention; with cos/sin, q is the raw projection, rotated in the kernel."""
        return ops.varlen_prefill(q, kv_cache, block_table, cu_seqlens, context_lens,
                                  int(max_seqlen), self.scale, self.num_heads,
                                  self.num_kv_heads, self.head_dim, cos=cos, sin=sin)

    def _decode(self, q, k, v, kv_cache, block_table, context_lens):
        return self._decode_attend(q, kv_cache, block_table, context_lens, new_k=k, new_v=v)

    def _decode_attend(self, q, kv_cache, block_table, context_lens, new_k=None, new_v=None,
                       cos=None, sin=None):
        need = ops.decode_workspace_bytes(q.shape[0], self.num_heads, self.num_kv_heads,
                                          self.head_dim, block_table.shape[1], kv_cache.shape[3])
        ws = self._workspaces[-1] if self._workspaces else None
        if ws is None or ws.numel() < need or ws.device != q.device:
            ws = ops.decode_workspace(need, q.device)
            self._workspaces.append(ws)
        return ops.paged_decode(q, kv_cache, block_table, context_lens, self.scale,
                                self.num_heads, self.num_kv_heads, self.head_dim,
                                workspace=ws, new_k=new_k, new_v=new_v, cos=cos, sin=sin)
