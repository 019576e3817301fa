"""Seeded synthetic inputs for the paged-KV path at the benchmark shapes.

Named cases (CASES):
  qwen2-0.5b-decode     Qwen2-0.5B layer decode: 14/2 heads, head_dim 64, 8
                        sequences, context U{32..512}, 512-block pool, table =
                        random permutation
  llama3-8b-decode      Llama-3-8B layer decode: 32/8 heads, head_dim 128, 64
                        sequences, context U{512..4096}, random non-contiguous tables
  qwen2-7b-prefill      Qwen2-7B varlen prefill: 28/4 heads, head_dim 128, 16
                        prompts U{128..2048} packed by cu_seqlens
  llama3-8b-long-decode Llama-3-8B long-context decode: 256 sequences, context
                        lognormal(median 8192, sigma 1.0) clipped to [1024, 32768],
                        tables from 10,000 seeded alloc/free cycles of BlockAllocator

Values are bf16 ~N(0, 1).  Cache slots no sequence owns hold random bit
patterns (NaN and Inf included) so that a stray read or write shows.  The
block table is padded with num_blocks - 1 exactly as the reference runner
pads it (needle/model/runner.py:226-235).
"""
from __future__ import annotations

import math
import random
from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np
import torch

from .backend.block_allocator import BlockAllocator

BLOCK_SIZE = 16


@dataclass(frozen=True)
class HeadShape:
    num_heads: int
    num_kv_heads: int
    head_dim: int
    block_size: int = BLOCK_SIZE

    @property
    def group(self) -> int:
        return self.num_heads // self.num_kv_heads

    @property
    def scale(self) -> float:
        return 1.0 / math.sqrt(self.head_dim)   # attention.py:48


QWEN2_05B = HeadShape(14, 2, 64)
LLAMA3_8B = HeadShape(32, 8, 128)
QWEN2_7B = HeadShape(28, 4, 128)


@dataclass
class PagedCase:
    shape: HeadShape
    q: torch.Tensor                 # decode [B, H, D]; prefill [T, H, D]
    k: torch.Tensor                 # new tokens [T, Hkv, D]
    v: torch.Tensor
    kv_cache: torch.Tensor          # [2, NB, Hkv, bs, D]
    block_table: torch.Tensor       # int32 [B, W]
    context_lens: torch.Tensor      # int32 [B]
    cu_seqlens: Optional[torch.Tensor]  # int32 [B + 1] (prefill) or None (decode)
    ctx: List[int] = field(default_factory=list)       # host copies
    new_lens: List[int] = field(default_factory=list)
    tables: List[List[int]] = field(default_factory=list)

    @property
    def num_seqs(self) -> int:
        return len(self.ctx)

    @property
    def num_blocks(self) -> int:
        return self.kv_cache.shape[1]

    @property
    def max_seqlen(self) -> int:
        return max(self.new_lens) if self.new_lens else 0

    def to(self, device) -> "PagedCase":
        mv = lambda t: None if t is None else t.to(device)   # noqa: E731
        return PagedCase(self.shape, mv(self.q), mv(self.k), mv(self.v), mv(self.kv_cache),
                         mv(self.block_table), mv(self.context_lens), mv(self.cu_seqlens),
                         list(self.ctx), list(self.new_lens), [list(t) for t in self.tables])


# ----------------------------------------------------------------------------
# block tables
# ----------------------------------------------------------------------------

def tables_by_permutation(blocks_per_seq: List[int], num_blocks: int, seed: int) -> List[List[int]]:
    """Disjoint random blocks per sequence: a seeded permutation of the pool, cut in order."""
    need = sum(blocks_per_seq)
    if need > num_blocks:
        raise ValueError(f"pool of {num_blocks} blocks cannot hold {need}")
    perm = np.random.default_rng(seed).permutation(num_blocks).tolist()
    out, pos = [], 0
    for n in blocks_per_seq:
        out.append(perm[pos:pos + n])
        pos += n
    return out


def tables_by_allocator(blocks_per_seq: List[int], num_blocks: int, seed: int,
                        cycles: int = 10_000) -> List[List[int]]:
    """Tables from `cycles` seeded alloc/free rounds of BlockAllocator, then per-sequence allocation.

    Each round allocates a chunk of 1..64 blocks (a short-lived sequence) and,
    with probability 1/2 or when the pool is short, frees a random live chunk.
    All live chunks are then freed in random order, which leaves the FIFO free
    list scrambled, and every sequence takes its blocks from it in order.
    """
    rng = random.Random(seed)
    alloc = BlockAllocator(num_blocks, 0, BLOCK_SIZE)
    live: List[List[int]] = []
    for _ in range(cycles):
        n = rng.randint(1, 64)
        while not alloc.can_allocate_gpu(n) and live:
            alloc.free_gpu_blocks(live.pop(rng.randrange(len(live))))
        if alloc.can_allocate_gpu(n):
            live.append(alloc.allocate_gpu_blocks(n))
        if live and rng.random() < 0.5:
            alloc.free_gpu_blocks(live.pop(rng.randrange(len(live))))
    rng.shuffle(live)
    for chunk in live:
        alloc.free_gpu_blocks(chunk)
    return [alloc.allocate_gpu_blocks(n) for n in blocks_per_seq]


def pad_tables(tables: List[List[int]], num_blocks: int) -> torch.Tensor:
    """runner.py:220-235: pad every row to the longest with the dummy id num_blocks - 1."""
    width = max(1, max((len(t) for t in tables), default=1))
    dummy = num_blocks - 1
    rows = [t + [dummy] * (width - len(t)) for t in tables]
    return torch.tensor(rows, dtype=torch.int32)


# ----------------------------------------------------------------------------
# pool filling
# ----------------------------------------------------------------------------

def _fill_pool(shape: HeadShape, num_blocks: int, tables, valid_lens, gen, device, dtype,
               garbage: bool) -> torch.Tensor:
    bs = shape.block_size
    pool = torch.randn((2, num_blocks, shape.num_kv_heads, bs, shape.head_dim),
                       generator=gen, device=device, dtype=torch.float32).to(dtype)
    if not garbage:
        return pool
    valid = torch.zeros((num_blocks, bs), dtype=torch.bool)
    for tab, n in zip(tables, valid_lens):
        if n <= 0:
            continue
        pos = torch.arange(n)
        blk = torch.tensor(tab, dtype=torch.long)[torch.clamp(pos // bs, max=len(tab) - 1)]
        valid[blk, pos % bs] = True
    invalid = (~valid).to(device)
    bits_dtype = {2: torch.int16, 4: torch.int32}[pool.element_size()]
    view = pool.view(bits_dtype).permute(1, 3, 0, 2, 4)   # [NB, bs, 2, Hkv, D]
    n_bad = int(invalid.sum())
    if n_bad:
        lim = 1 << (8 * pool.element_size() - 1)
        bits = torch.randint(-lim, lim, (n_bad, 2, shape.num_kv_heads, shape.head_dim),
                             generator=gen, device=device, dtype=torch.int64).to(bits_dtype)
        view[invalid] = bits
    return pool


def _gen(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def decode_case(shape: HeadShape, ctx_lens: List[int], *, seed: int, device="cpu",
                num_blocks: Optional[int] = None, table: str = "perm", garbage: bool = True,
                dtype=torch.bfloat16, slack: float = 1.1) -> PagedCase:
    """One decode step: q/k/v for one new token per sequence plus a pool holding ctx_i tokens.

    The table covers position ctx_i (the slot the new token goes to), as the
    scheduler guarantees (needle/backend/scheduler.py:111-118).
    """
    bs = shape.block_size
    blocks = [(c + 1 + bs - 1) // bs for c in ctx_lens]
    if num_blocks is None:
        num_blocks = max(int(math.ceil(sum(blocks) * slack)), sum(blocks) + 1)
    if table == "perm":
        tables = tables_by_permutation(blocks, num_blocks, seed)
    elif table == "allocator":
        tables = tables_by_allocator(blocks, num_blocks, seed)
    else:
        raise ValueError(table)
    gen = _gen(seed, device)
    b, h, hkv, d = len(ctx_lens), shape.num_heads, shape.num_kv_heads, shape.head_dim
    pool = _fill_pool(shape, num_blocks, tables, ctx_lens, gen, device, dtype, garbage)
    q = torch.randn((b, h, d), generator=gen, device=device).to(dtype)
    k = torch.randn((b, hkv, d), generator=gen, device=device).to(dtype)
    v = torch.randn((b, hkv, d), generator=gen, device=device).to(dtype)
    return PagedCase(shape, q, k, v, pool, pad_tables(tables, num_blocks).to(device),
                     torch.tensor(ctx_lens, dtype=torch.int32, device=device), None,
                     list(ctx_lens), [1] * b, tables)


def prefill_case(shape: HeadShape, seq_lens: List[int], *, seed: int, device="cpu",
                 ctx_lens: Optional[List[int]] = None, num_blocks: Optional[int] = None,
                 table: str = "perm", garbage: bool = True, dtype=torch.bfloat16,
                 slack: float = 1.1) -> PagedCase:
    """Packed prompts (cu_seqlens) plus a pool holding ctx_i cached prefix tokens (default 0)."""
    bs = shape.block_size
    if ctx_lens is None:
        ctx_lens = [0] * len(seq_lens)
    blocks = [max(1, (c + n + bs - 1) // bs) for c, n in zip(ctx_lens, seq_lens)]
    if num_blocks is None:
        num_blocks = max(int(math.ceil(sum(blocks) * slack)), sum(blocks) + 1)
    if table == "perm":
        tables = tables_by_permutation(blocks, num_blocks, seed)
    elif table == "allocator":
        tables = tables_by_allocator(blocks, num_blocks, seed)
    else:
        raise ValueError(table)
    gen = _gen(seed, device)
    t, h, hkv, d = sum(seq_lens), shape.num_heads, shape.num_kv_heads, shape.head_dim
    pool = _fill_pool(shape, num_blocks, tables, ctx_lens, gen, device, dtype, garbage)
    q = torch.randn((t, h, d), generator=gen, device=device).to(dtype)
    k = torch.randn((t, hkv, d), generator=gen, device=device).to(dtype)
    v = torch.randn((t, hkv, d), generator=gen, device=device).to(dtype)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(seq_lens)]).tolist(), dtype=torch.int32,
                      device=device)
    return PagedCase(shape, q, k, v, pool, pad_tables(tables, num_blocks).to(device),
                     torch.tensor(ctx_lens, dtype=torch.int32, device=device), cu,
                     list(ctx_lens), list(seq_lens), tables)


# ----------------------------------------------------------------------------
# the benchmark configurations
# ----------------------------------------------------------------------------

def qwen05b_decode_ctx(seed: int = 1001) -> List[int]:
    return np.random.default_rng(seed).integers(32, 512, size=8, endpoint=True).tolist()


def llama8b_decode_ctx(seed: int = 1002, batch: int = 64) -> List[int]:
    return np.random.default_rng(seed).integers(512, 4096, size=batch, endpoint=True).tolist()


def qwen7b_prefill_lens(seed: int = 1003, prompts: int = 16) -> List[int]:
    return np.random.default_rng(seed).integers(128, 2048, size=prompts, endpoint=True).tolist()


LONG_CONTEXT_SIGMA = 1.0


def llama8b_long_ctx(seed: int = 1005, batch: int = 256, sigma: float = LONG_CONTEXT_SIGMA) -> List[int]:
    r = np.random.default_rng(seed).lognormal(math.log(8192.0), sigma, size=batch)
    return np.clip(np.round(r), 1024, 32768).astype(np.int64).tolist()


CASES = ("qwen2-0.5b-decode", "llama3-8b-decode", "qwen2-7b-prefill", "llama3-8b-long-decode")


def config_case(name: str, device="cpu", garbage: bool = True) -> PagedCase:
    """Full-size inputs of one named case (see CASES)."""
    if name == "qwen2-0.5b-decode":
        return decode_case(QWEN2_05B, qwen05b_decode_ctx(), seed=1001, device=device,
                           num_blocks=512, garbage=garbage)
    if name == "llama3-8b-decode":
        return decode_case(LLAMA3_8B, llama8b_decode_ctx(), seed=1002, device=device,
                           garbage=garbage)
    if name == "qwen2-7b-prefill":
        return prefill_case(QWEN2_7B, qwen7b_prefill_lens(), seed=1003, device=device,
                            garbage=garbage)
    if name == "llama3-8b-long-decode":
        return decode_case(LLAMA3_8B, llama8b_long_ctx(), seed=1005, device=device,
                           table="allocator", garbage=garbage)
    raise ValueError(f"unknown case {name!r}; known: {', '.join(CASES)}")


# ----------------------------------------------------------------------------
# algorithmic work
# ----------------------------------------------------------------------------

def decode_bytes(shape: HeadShape, ctx_lens: List[int], width: int) -> int:
    """HBM bytes a decode step must move: each attended K/V row once, q in, out out, table, lens."""
    bs, hkv, d, h = shape.block_size, shape.num_kv_heads, shape.head_dim, shape.num_heads
    lens = [max(0, min(c + 1, width * bs)) for c in ctx_lens]
    kv = sum(lens) * hkv * d * 2 * 2
    qo = 2 * len(ctx_lens) * h * d * 2
    tab = 4 * sum((n + bs - 1) // bs for n in lens) + 4 * len(ctx_lens)
    return kv + qo + tab


def append_bytes(shape: HeadShape, num_tokens: int, num_seqs: int, varlen: bool) -> int:
    """Bytes an append must move: read the k and v rows, write them into the pool, read indices."""
    rows = num_tokens * shape.num_kv_heads * shape.head_dim * 2 * 2   # k and v, bf16
    idx = 4 * num_seqs * 2 + (4 * (num_seqs + 1) if varlen else 0)    # ctx + table entry (+cu)
    return 2 * rows + idx


def prefill_flops(shape: HeadShape, seq_lens: List[int], ctx_lens: Optional[List[int]] = None) -> int:
    """4 * H * D per attended (query, key) pair: causal pairs sum_i sum_p (ctx_i + p + 1)."""
    if ctx_lens is None:
        ctx_lens = [0] * len(seq_lens)
    pairs = sum(n * c + n * (n + 1) // 2 for n, c in zip(seq_lens, ctx_lens))
    return 4 * shape.num_heads * shape.head_dim * pairs
