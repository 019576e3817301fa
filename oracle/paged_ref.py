"""Op-for-op CPU restatement of the reference torch path (TEST INFRASTRUCTURE).

Follows needle/layers/attention.py of mitu626/needle v0.1.0.  All tensors are
CPU torch tensors; dtypes are whatever the caller passes (the reference runs
the model dtype, bf16), and every torch op runs in that dtype exactly as the
reference's does, so rounding matches op for op.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def slot_of_tokens(block_table: torch.Tensor, cu_seqlens: torch.Tensor,
                   context_lens: torch.Tensor, block_size: int):
    """(phys, block_off) of every packed token.

    attention.py:217-237: abs_pos = ctx_i + (t - cu_i); col = min(abs_pos // bs, W-1);
    phys = block_table[seq_idx, col]; off = abs_pos % bs.
    """
    batch = cu_seqlens.shape[0] - 1
    seq_lengths = (cu_seqlens[1:] - cu_seqlens[:-1]).long()          # :219
    ctx = context_lens.tolist()                                         # :222
    lens = seq_lengths.tolist()                                         # :223
    if batch == 0 or sum(lens) == 0:
        empty = torch.zeros(0, dtype=torch.long)
        return empty, empty
    abs_pos = torch.cat([torch.arange(int(ctx[i]), int(ctx[i]) + int(lens[i]), dtype=torch.long)
                         for i in range(batch)])                        # :224-229
    seq_idx = torch.repeat_interleave(torch.arange(batch, dtype=torch.long), seq_lengths)  # :231
    col = (abs_pos // block_size).clamp(max=block_table.shape[1] - 1)   # :235
    phys = block_table[seq_idx, col].long()                             # :236
    off = (abs_pos % block_size).long()                                 # :237
    return phys, off


def write_kv(k, v, kv_cache, block_table, cu_seqlens, context_lens) -> None:
    """attention.py:204-246, in place on kv_cache."""
    block_size = kv_cache.shape[3]
    phys, off = slot_of_tokens(block_table, cu_seqlens, context_lens, block_size)
    if phys.numel() == 0:
        return
    kv0, kv1 = kv_cache[0], kv_cache[1]                                 # :242-243
    for h in range(kv_cache.shape[2]):                                  # :244
        kv0[phys, h, off] = k[:, h, :]                                  # :245
        kv1[phys, h, off] = v[:, h, :]                                  # :246


def decode_append(k, v, kv_cache, block_table, context_lens) -> None:
    """attention.py:141-154: one new token per sequence, in place on kv_cache."""
    num_seqs = k.shape[0]
    block_size = kv_cache.shape[3]
    ctx = context_lens.long()                                           # :143
    col = (ctx // block_size).clamp(max=block_table.shape[1] - 1)       # :144
    phys = block_table[torch.arange(num_seqs), col].long()              # :145
    off = (ctx % block_size).long()                                     # :146
    for h in range(kv_cache.shape[2]):                                  # :152
        kv_cache[0, phys, h, off, :] = k[:, h, :]                       # :153
        kv_cache[1, phys, h, off, :] = v[:, h, :]                       # :154


def decode_pytorch(q, kv_cache, block_table, context_lens, scale,
                   num_heads, num_kv_heads, head_dim):
    """attention.py:291-310 (_decode_pytorch), returns [B, H, D] in q's dtype."""
    num_seqs = q.shape[0]
    block_size = kv_cache.shape[3]
    outputs = []
    ctx_lens = context_lens.tolist()                                    # :297
    for i in range(num_seqs):                                           # :298
        ctx_len = int(ctx_lens[i]) + 1                                  # :299
        nb = (ctx_len + block_size - 1) // block_size                   # :300
        phys = block_table[i, :nb]                                      # :301
        k_full = kv_cache[0][phys].transpose(0, 1).reshape(num_kv_heads, -1, head_dim)[:, :ctx_len]
        v_full = kv_cache[1][phys].transpose(0, 1).reshape(num_kv_heads, -1, head_dim)[:, :ctx_len]
        expand = num_heads // num_kv_heads                              # :304
        k_exp = k_full.repeat_interleave(expand, dim=0)                 # :305
        v_exp = v_full.repeat_interleave(expand, dim=0)                 # :306
        attn_w = torch.einsum("hd,hsd->hs", q[i], k_exp) * scale        # :307
        out_i = torch.einsum("hs,hsd->hd", attn_w.softmax(dim=-1), v_exp)  # :308
        outputs.append(out_i)
    return torch.stack(outputs, dim=0)                                  # :310


def prefill_pytorch(q, k, v, cu_seqlens, num_heads, num_kv_heads):
    """attention.py:120-134 (_prefill_pytorch): per-sequence causal SDPA on fresh k/v."""
    outputs = []
    cu = cu_seqlens.tolist()                                            # :122
    for i in range(len(cu) - 1):                                        # :123
        s, e = int(cu[i]), int(cu[i + 1])
        qi = q[s:e].unsqueeze(0).transpose(1, 2)                        # :125
        ki = k[s:e].unsqueeze(0).transpose(1, 2)                        # :126
        vi = v[s:e].unsqueeze(0).transpose(1, 2)                        # :127
        if num_kv_heads != num_heads:                                   # :128
            factor = num_heads // num_kv_heads
            ki = ki.repeat_interleave(factor, dim=1)                    # :130
            vi = vi.repeat_interleave(factor, dim=1)                    # :131
        out_i = F.scaled_dot_product_attention(qi, ki, vi, is_causal=True)  # :132
        outputs.append(out_i.transpose(1, 2).squeeze(0))                # :133
    return torch.cat(outputs, dim=0)                                    # :134


def prefill(q, k, v, kv_cache, block_table, cu_seqlens, context_lens, num_heads, num_kv_heads):
    """attention.py:102-107 (_prefill without FlashInfer): write_kv, then causal SDPA."""
    write_kv(k, v, kv_cache, block_table, cu_seqlens, context_lens)
    return prefill_pytorch(q, k, v, cu_seqlens, num_heads, num_kv_heads)


def decode(q, k, v, kv_cache, block_table, context_lens, scale, num_heads, num_kv_heads,
           head_dim):
    """attention.py:140-159 (_decode without FlashInfer): append, then paged decode."""
    decode_append(k, v, kv_cache, block_table, context_lens)
    return decode_pytorch(q, kv_cache, block_table, context_lens, scale,
                          num_heads, num_kv_heads, head_dim)


def rotate_half(x):
    """attention.py:286-288."""
    half = x.shape[-1] // 2
    return torch.cat([-x[..., half:], x[..., :half]], dim=-1)


def apply_rope(q, k, cos, sin):
    """attention.py:277-283."""
    cos = cos.unsqueeze(1)
    sin = sin.unsqueeze(1)
    return q * cos + rotate_half(q) * sin, k * cos + rotate_half(k) * sin


def attention_forward(weights, hidden_states, kv_cache, block_table, cu_seqlens, context_lens,
                      is_prefill, cos, sin, num_heads, num_kv_heads, head_dim):
    """attention.py:83-96 (Attention.forward, torch fallback path) with explicit weights.

    weights: dict with q_proj/k_proj/v_proj/o_proj '.weight' (and optional
    q/k/v '.bias') as the reference's Linear layers hold them (linear.py:49-50,
    88-89); the projections are F.linear(x, w, b) (linear.py:54, 93-97).
    """
    t = hidden_states.shape[0]
    q = F.linear(hidden_states, weights["q_proj.weight"], weights.get("q_proj.bias"))
    k = F.linear(hidden_states, weights["k_proj.weight"], weights.get("k_proj.bias"))
    v = F.linear(hidden_states, weights["v_proj.weight"], weights.get("v_proj.bias"))
    q = q.view(t, num_heads, head_dim)
    k = k.view(t, num_kv_heads, head_dim)
    v = v.view(t, num_kv_heads, head_dim)
    q, k = apply_rope(q, k, cos, sin)
    scale = 1.0 / (head_dim ** 0.5)
    if is_prefill:
        out = prefill(q, k, v, kv_cache, block_table, cu_seqlens, context_lens, num_heads,
                      num_kv_heads)
    else:
        out = decode(q, k, v, kv_cache, block_table, context_lens, scale, num_heads,
                     num_kv_heads, head_dim)
    return F.linear(out.reshape(t, num_heads * head_dim), weights["o_proj.weight"])
