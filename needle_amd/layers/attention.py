"""Drop-in replacement for needle/layers/attention.py:Attention on MI355X.

Same constructor, the same forward() signature and meaning
(attention.py:36-96), the same parameter names (q_proj/k_proj/v_proj/o_proj),
and the same KV pool layout [2, num_blocks, num_kv_heads, block_size,
head_dim].  Projections stay torch GEMMs (attention.py:84-86); fuse_projections()
runs the three as one GEMM over their concatenated weights.  The rest of
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
import torch.nn.functional as F

from .. import ops
from ..model.config import ModelConfig


def fuse_linears(*mods: nn.Linear):
    """Puts the weights (and biases) of Linear layers that read the same input into one
    tensor, each layer's parameters becoming views of it, so that one GEMM serves them all
    (F.linear over the fused weight, its output split).  Parameter names, values and
    sharing with in-place updates are unchanged; the fused (weight, bias or None) is returned.
    Moving the layers afterwards gives them separate storage again, which fused_outputs
    detects."""
    rows = [m.weight.shape[0] for m in mods]
    w = torch.cat([m.weight.detach() for m in mods], 0)
    b = None
    if mods[0].bias is not None:
        b = torch.cat([m.bias.detach() for m in mods], 0)
    r0 = 0
    for m, r in zip(mods, rows):
        m.weight = nn.Parameter(w[r0:r0 + r], requires_grad=m.weight.requires_grad)
        if b is not None:
            m.bias = nn.Parameter(b[r0:r0 + r], requires_grad=m.bias.requires_grad)
        r0 += r
    return (w, b)


def _still_fused(fused, mods) -> bool:
    """True while every layer's weight (and bias) is the view fuse_linears made of the fused
    tensor (a later .to() or a replaced parameter gives it storage of its own)."""
    w, b = fused
    # Row r0 of the fused tensor starts r0 * stride(0) elements in; comparing addresses that
    # way avoids building a slice per layer on every forward.
    wp, ws, dev = w.data_ptr(), w.stride(0) * w.element_size(), w.device
    bp, bs = (b.data_ptr(), b.element_size()) if b is not None else (0, 0)
    r0 = 0
    for m in mods:
        p = m._parameters  # the dict nn.Module.__getattr__ would search, read once
        mw, mb = p["weight"], p.get("bias")
        if mw.data_ptr() != wp + r0 * ws or mw.device != dev:
            return False
        if b is not None and (mb is None or mb.data_ptr() != bp + r0 * bs):
            return False
        r0 += mw.shape[0]
    return r0 == w.shape[0]


def fused_outputs(fused, mods, x):
    """The outputs of the Linear layers mods on x: one GEMM over the fused weight while their
    parameters are still views of it (fuse_linears), otherwise one per layer."""
    if fused is not None and _still_fused(fused, mods):
        w, b = fused
        return F.linear(x, w, b).split([m.weight.shape[0] for m in mods], dim=-1)
    return tuple(m(x) for m in mods)


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
        self._qkv = None   # fused q/k/v projection (fuse_projections)

    def fuse_projections(self) -> None:
        """One GEMM for the q, k and v projections (they read the same input), their
        parameters becoming views of one tensor; call after the weights are in place."""
        self._qkv = fuse_linears(self.q_proj, self.k_proj, self.v_proj)

    def forward(self, hidden_states: torch.Tensor, positions: torch.Tensor,
                kv_cache: torch.Tensor, block_table: torch.Tensor, cu_seqlens: torch.Tensor,
                context_lens: torch.Tensor, max_seqlen: int, is_prefill: bool,
                cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
        total = hidden_states.shape[0]
        q, k, v = fused_outputs(self._qkv, (self.q_proj, self.k_proj, self.v_proj),
                                hidden_states)
        q = q.view(total, self.num_heads, self.head_dim)
        k = k.view(total, self.num_kv_heads, self.head_dim)
        v = v.view(total, self.num_kv_heads, self.head_dim)
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
