"""Independent fp64 closed forms and brute-force loops (TEST INFRASTRUCTURE).

These restate the mathematics of the reference path position by position,
with none of paged_ref's tensor idioms (no block gather + transpose +
reshape, no repeat_interleave), so that a wrong index, a transposed operand
or a wrong GQA mapping in either formulation shows up as a mismatch:

  append_bruteforce   reference attention.py:141-154 / 204-246, one Python
                      loop iteration per (token, kv head, element)
  decode_fp64         softmax(scale * q.k) v over positions 0..L-1,
                      L = min(ctx + 1, W * bs) (attention.py:299-303),
                      query head h -> kv head h // g (attention.py:304-306)
  prefill_fp64        causal softmax attention per sequence; position p of a
                      query attends cache positions 0..p of its own sequence
"""
from __future__ import annotations

import numpy as np
import torch


def _np64(t: torch.Tensor) -> np.ndarray:
    return t.detach().to(torch.float64).cpu().numpy()


def append_bruteforce(k, v, kv_cache, block_table, cu_seqlens, context_lens):
    """Returns a new cache with every token written, one element at a time."""
    cache = kv_cache.clone()
    bs = cache.shape[3]
    w = block_table.shape[1]
    bt = block_table.tolist()
    ctx = context_lens.tolist()
    cu = cu_seqlens.tolist() if cu_seqlens is not None else list(range(len(ctx) + 1))
    for i in range(len(ctx)):
        for t in range(cu[i], cu[i + 1]):
            pos = ctx[i] + (t - cu[i])
            col = pos // bs
            if col > w - 1:
                col = w - 1
            blk = bt[i][col]
            off = pos % bs
            for h in range(cache.shape[2]):
                for e in range(cache.shape[4]):
                    cache[0, blk, h, off, e] = k[t, h, e]
                    cache[1, blk, h, off, e] = v[t, h, e]
    return cache


def _kv_rows(kv_np, bt_row, kvh, n_pos, bs):
    """K and V rows of positions 0..n_pos-1 for one sequence and kv head."""
    kr = np.empty((n_pos, kv_np.shape[-1]))
    vr = np.empty((n_pos, kv_np.shape[-1]))
    for p in range(n_pos):
        blk = bt_row[min(p // bs, len(bt_row) - 1)]
        kr[p] = kv_np[0, blk, kvh, p % bs]
        vr[p] = kv_np[1, blk, kvh, p % bs]
    return kr, vr


def _softmax_attend(qv, kr, vr, scale):
    s = (kr @ qv) * scale
    s = s - s.max()
    w = np.exp(s)
    return (w @ vr) / w.sum()


def decode_fp64(q, kv_cache, block_table, context_lens, scale, num_heads, num_kv_heads):
    """[B, H, D] float64."""
    qn = _np64(q)
    kvn = _np64(kv_cache)
    bs = kv_cache.shape[3]
    w = block_table.shape[1]
    g = num_heads // num_kv_heads
    bt = block_table.tolist()
    out = np.zeros((q.shape[0], num_heads, q.shape[2]))
    for i, c in enumerate(context_lens.tolist()):
        n = min(c + 1, w * bs)
        if n <= 0:
            continue
        for kvh in range(num_kv_heads):
            kr, vr = _kv_rows(kvn, bt[i], kvh, n, bs)
            for h in range(kvh * g, (kvh + 1) * g):
                out[i, h] = _softmax_attend(qn[i, h], kr, vr, scale)
    return out


def prefill_fp64(q, kv_cache, block_table, cu_seqlens, context_lens, scale,
                 num_heads, num_kv_heads):
    """[T, H, D] float64; reads K/V of every position through block_table."""
    qn = _np64(q)
    kvn = _np64(kv_cache)
    bs = kv_cache.shape[3]
    g = num_heads // num_kv_heads
    bt = block_table.tolist()
    cu = cu_seqlens.tolist()
    ctx = context_lens.tolist()
    out = np.zeros((q.shape[0], num_heads, q.shape[2]))
    for i in range(len(ctx)):
        n_tok = cu[i + 1] - cu[i]
        if n_tok == 0:
            continue
        last = ctx[i] + n_tok
        for kvh in range(num_kv_heads):
            kr, vr = _kv_rows(kvn, bt[i], kvh, last, bs)
            for t in range(cu[i], cu[i + 1]):
                p = ctx[i] + (t - cu[i])
                for h in range(kvh * g, (kvh + 1) * g):
                    out[t, h] = _softmax_attend(qn[t, h], kr[:p + 1], vr[:p + 1], scale)
    return out


def dense_causal_fp64(q, k, v, cu_seqlens, scale, num_heads, num_kv_heads):
    """Causal attention on contiguous per-sequence q/k/v (no cache), [T, H, D] float64."""
    qn, kn, vn = _np64(q), _np64(k), _np64(v)
    g = num_heads // num_kv_heads
    cu = cu_seqlens.tolist()
    out = np.zeros((q.shape[0], num_heads, q.shape[2]))
    for i in range(len(cu) - 1):
        s, e = cu[i], cu[i + 1]
        for h in range(num_heads):
            kvh = h // g
            for t in range(s, e):
                out[t, h] = _softmax_attend(qn[t, h], kn[s:t + 1, kvh], vn[s:t + 1, kvh], scale)
    return out
