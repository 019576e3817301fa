"""ModelRunner: KV pools, batch metadata and the forwards of one engine step.

Contract with the attention path (reference needle/model/runner.py:65-94, 194-249):
  * one KV pool per layer, [2, num_blocks, num_kv_heads, block_size, head_dim] in the
    model dtype, zero-initialised, plus an optional pinned CPU pool for swapping;
  * prefill feeds every token of a sequence with context 0, decode its newest token with
    context length-1; positions ctx..ctx+n; cu_seqlens is the prefix sum of the token
    counts; block_table rows are padded with num_blocks-1 to the widest row; a step with
    both prefill and decode sequences runs two forwards.

How this runner feeds the device:
  * an eager batch goes to the device as one pinned int64 buffer (one copy, then views);
  * decode steps can replay HIP graphs captured per batch-size bucket
    (enable_decode_graphs).  Their metadata stays on the device between steps
    (_DecodeRows): a sequence keeps its row for as long as it decodes, the step's
    greedy tokens are written into the next step's input ids inside the graph, and the
    host sends only what changed (context lengths, new rows, new blocks) as one small
    scatter.  Padding rows point at a scratch block the allocator never hands out;
  * sampling is greedy: one device argmax and one host copy for the whole batch;
  * swapping moves every block of every layer in one ndl_kv_block_copy launch per
    direction (the reference issues one copy per layer and block, runner.py:175-192).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, List, Optional

import numpy as np
import torch

from .. import ops
from ..backend.request import SeqState
from ..backend.scheduler import StepPlan
from .config import ModelConfig
from .qwen2 import build_model, fuse_projections, random_init_
from .sampler import check_greedy, sample


@dataclass
class Batch:
    """The metadata of one forward (the arguments of Attention.forward besides q/k/v)."""
    input_ids: torch.Tensor
    positions: torch.Tensor
    cu_seqlens: torch.Tensor
    max_seqlen: int
    block_table: torch.Tensor
    context_lens: torch.Tensor
    is_prefill: bool


class _DecodeRows:
    """Device-resident metadata of the graph-replayed decode batch.

    One int32 device buffer holds, per row r < capacity: the next input token, the
    context length and the block-table row.  Row r belongs to one sequence for as long as
    it keeps decoding; a leaving sequence's row is filled with the last row's sequence and
    the last row is reset to padding (token 0, context 0, every entry the scratch block).
    Every step the host sends (flat index, value) pairs for what changed and applies them
    with one scatter: the context lengths of the live rows, the rows that were filled, the
    block ids a sequence gained.  The tokens of greedy rows are written by the graph itself.

    A sequence's block list is either grown by append (a new block at a block edge) or
    replaced by a new list object (admission, swap-out, swap-in, release): the scheduler
    never rewrites one in place.  A row whose sequence holds a different list object than
    at the last sync (it was swapped or recomputed while the steps in between ran eagerly)
    is sent whole again.
    """

    def __init__(self, capacity: int, width: int, scratch_block: int, device):
        self.capacity, self.width, self.scratch = capacity, width, scratch_block
        self.meta = torch.zeros(capacity * (2 + width), dtype=torch.int32, device=device)
        self.tok = self.meta[:capacity]
        self.ctx = self.meta[capacity:2 * capacity]
        self.table = self.meta[2 * capacity:].view(capacity, width)
        self.table.fill_(scratch_block)
        self.rows: List[SeqState] = []
        self.sent_blocks: List[int] = []     # table entries the device holds, per row
        self.sent_list: List[Optional[List[int]]] = []  # the block list they came from
        self.dirty: List[bool] = []          # row refilled: send all of it
        self.tok_on_device: List[bool] = []  # the graph wrote this row's newest token
        self._staging: List[torch.Tensor] = []
        self._staging_np: list = []
        self._events: list = [None, None]
        self._recorded = [False, False]
        self._turn = 0
        self._dev_pairs = torch.empty(0, dtype=torch.int32, device=device)

    def fits(self, seqs: List[SeqState], block_size: int) -> bool:
        return len(seqs) <= self.capacity and all(
            len(s.blocks) <= self.width and s.length <= self.width * block_size for s in seqs)

    def forget_tokens(self) -> None:
        """The newest tokens did not come from a replay (an eager decode step ran)."""
        self.tok_on_device = [False] * len(self.rows)

    def sync(self, seqs: List[SeqState]) -> None:
        """Make rows 0..len(seqs)-1 hold exactly `seqs` (in any order) on the device."""
        live = {id(s) for s in seqs}
        upd: Dict[int, int] = {}          # flat index -> value; a later write wins
        cap, w = self.capacity, self.width
        # leaving sequences: refill their rows from the end, reset each vacated last row
        r = 0
        while r < len(self.rows):
            if id(self.rows[r]) in live:
                r += 1
                continue
            last = len(self.rows) - 1
            upd[last] = 0
            upd[cap + last] = 0
            base = 2 * cap + last * w
            for j in range(self.sent_blocks[last]):
                upd[base + j] = self.scratch
            if r != last:
                # row r keeps its own old entries on the device until the refill below
                self.rows[r] = self.rows[last]
                self.dirty[r] = True
                self.tok_on_device[r] = False
            self.rows.pop()
            self.sent_blocks.pop()
            self.sent_list.pop()
            self.dirty.pop()
            self.tok_on_device.pop()
        # arriving sequences take the rows after the last one (all padding on the device)
        present = {id(s) for s in self.rows}
        for s in seqs:
            if id(s) not in present:
                self.rows.append(s)
                self.sent_blocks.append(0)
                self.sent_list.append(None)
                self.dirty.append(True)
                self.tok_on_device.append(False)
        for r, s in enumerate(self.rows):
            base = 2 * cap + r * w
            nb = len(s.blocks)
            sent = self.sent_blocks[r]
            if self.dirty[r] or self.sent_list[r] is not s.blocks or nb < sent:
                # a refilled row, or a block list replaced since the last sync
                for j in range(nb, sent):              # entries past the new list's end
                    upd[base + j] = self.scratch
                sent = 0
                self.dirty[r] = False
            for j in range(sent, nb):
                upd[base + j] = s.blocks[j]
            self.sent_blocks[r] = nb
            self.sent_list[r] = s.blocks
            upd[cap + r] = s.length - 1
            if not (self.tok_on_device[r] and s.params.greedy):
                upd[r] = s.last_token
        self._scatter(list(upd.keys()), list(upd.values()))

    def _scatter(self, idx: List[int], val: List[int]) -> None:
        n = len(idx)
        if n == 0:
            return
        if self.meta.device.type != "cuda":          # host-side model of the same updates
            self.meta[torch.tensor(idx, dtype=torch.long)] = torch.tensor(val, dtype=torch.int32)
            return
        if 2 * n > self._dev_pairs.numel():
            size = max(8192, 4 * n)
            self._staging = [torch.empty(size, dtype=torch.int32).pin_memory()
                             for _ in range(2)]
            self._staging_np = [h.numpy() for h in self._staging]
            self._events = [torch.cuda.Event(), torch.cuda.Event()]
            self._recorded = [False, False]
            self._dev_pairs = torch.empty(size, dtype=torch.int32, device=self.meta.device)
        t = self._turn
        self._turn ^= 1
        if self._recorded[t]:
            self._events[t].synchronize()        # the copy that last read this buffer
        arr = self._staging_np[t]
        arr[:n] = idx
        arr[n:2 * n] = val
        dev = self._dev_pairs[:2 * n]
        dev.copy_(self._staging[t][:2 * n], non_blocking=True)
        self._events[t].record()
        self._recorded[t] = True
        self.meta.index_put_((dev[:n],), dev[n:2 * n])   # int32 indices: no widening kernel

    def row_of(self) -> Dict[int, int]:
        return {id(s): r for r, s in enumerate(self.rows)}


class ModelRunner:
    DEFAULT_BUCKETS = (1, 2, 4, 8, 12, 16, 24, 32, 48, 64, 96, 128, 192, 256)

    def __init__(self, model_config: ModelConfig, block_size: int = 16, dtype: str = "bfloat16",
                 device: str = "cuda:0", seed: int = 0, model: Optional[torch.nn.Module] = None,
                 fuse: bool = True):
        self.model_config = model_config
        self.block_size = block_size
        self.device = torch.device(device)
        self.dtype = getattr(torch, dtype)
        if model is None:
            model = random_init_(build_model(model_config), seed)
        self.model = model.to(device=self.device, dtype=self.dtype).eval()
        if fuse:   # q/k/v and gate/up as one GEMM each
            fuse_projections(self.model)
        self.kv_caches: List[torch.Tensor] = []
        self.cpu_kv_caches: List[torch.Tensor] = []
        self._graphs: Dict[int, tuple] = {}
        self._rows: Optional[_DecodeRows] = None

    # ------------------------------------------------------------------ pools

    def bytes_per_block(self) -> int:
        cfg = self.model_config
        return (2 * cfg.num_kv_heads * self.block_size * cfg.head_dim
                * torch.finfo(self.dtype).bits // 8 * cfg.num_hidden_layers)

    def profile_memory(self, gpu_memory_utilization: float = 0.90, max_gpu_blocks: int = 0,
                       cpu_swap_bytes: int = 0):
        """Blocks that fit in this share of the free device memory (optionally capped), and
        the CPU swap pool's blocks for cpu_swap_bytes (runner.py:44-63 sizes that pool at
        half the GPU pool, ~128 GB of pinned memory on this GPU, so here the caller says)."""
        if self.device.type != "cuda":
            return (max_gpu_blocks or 512), cpu_swap_bytes // self.bytes_per_block()
        free, _total = torch.cuda.mem_get_info(self.device)
        n = max(1, int(free * gpu_memory_utilization) // self.bytes_per_block())
        if max_gpu_blocks:
            n = min(n, max_gpu_blocks)
        return n, cpu_swap_bytes // self.bytes_per_block()

    def init_kv_cache(self, num_gpu_blocks: int, num_cpu_blocks: int = 0) -> None:
        cfg = self.model_config
        shape = (2, num_gpu_blocks, cfg.num_kv_heads, self.block_size, cfg.head_dim)
        self.kv_caches = [torch.zeros(shape, dtype=self.dtype, device=self.device)
                          for _ in range(cfg.num_hidden_layers)]
        self.cpu_kv_caches = []
        if num_cpu_blocks > 0:
            cshape = (2, num_cpu_blocks, cfg.num_kv_heads, self.block_size, cfg.head_dim)
            self.cpu_kv_caches = [torch.zeros(cshape, dtype=self.dtype, pin_memory=True)
                                  for _ in range(cfg.num_hidden_layers)]

    @property
    def scratch_block(self) -> int:
        """The last pool block: padding rows of captured decode batches read and write
        here.  An engine with decode graphs keeps it out of the allocator."""
        return self.kv_caches[0].shape[1] - 1

    # ------------------------------------------------------------------ one step

    @torch.no_grad()
    def execute(self, plan: StepPlan) -> List[int]:
        """Run one planned step; returns the next token of every sequence of plan.seqs."""
        # swap-in before swap-out: a CPU block released by a swap-in can be taken by a
        # swap-out of the same step, and a sequence swapped in can be evicted again
        if plan.swap_in:
            self.swap(plan.swap_in, to_cpu=False)
        if plan.swap_out:
            self.swap(plan.swap_out, to_cpu=True)
        tokens: List[int] = []
        if plan.prefill:
            tokens += self._sample(plan.prefill, self.forward(self.prepare_inputs(
                plan.prefill, is_prefill=True)))
            for s in plan.prefill:
                s.kv_ready = True
        if plan.decode:
            toks = self._graph_decode(plan.decode) if self._graphs else None
            if toks is None:
                toks = self._sample(plan.decode, self.forward(self.prepare_inputs(
                    plan.decode, is_prefill=False)))
                if self._rows is not None:
                    self._rows.forget_tokens()
            tokens += toks
        return tokens

    def _sample(self, seqs: List[SeqState], logits: torch.Tensor) -> List[int]:
        return sample(logits, [s.params for s in seqs])

    def forward(self, batch: Batch) -> torch.Tensor:
        return self.model(batch.input_ids, batch.positions, self.kv_caches, batch.block_table,
                          batch.cu_seqlens, batch.context_lens, batch.max_seqlen,
                          batch.is_prefill)

    def prepare_inputs(self, seqs: List[SeqState], is_prefill: bool) -> Batch:
        ids: List[int] = []
        pos: List[int] = []
        cu: List[int] = [0]
        ctx: List[int] = []
        for s in seqs:
            if is_prefill:
                toks, c = s.tokens, 0
            else:
                toks, c = [s.last_token], s.length - 1
            ids += toks
            pos += range(c, c + len(toks))
            cu.append(cu[-1] + len(toks))
            ctx.append(c)
        n_tok, n_seq = len(ids), len(seqs)
        width = max((len(s.blocks) for s in seqs), default=1) or 1
        pad = (self.kv_caches[0].shape[1] if self.kv_caches else 1) - 1
        host = np.full(2 * n_tok + (n_seq + 1) + n_seq * width + n_seq, pad, dtype=np.int64)
        host[:n_tok] = ids
        host[n_tok:2 * n_tok] = pos
        o = 2 * n_tok
        host[o:o + n_seq + 1] = cu
        o += n_seq + 1
        tab = host[o:o + n_seq * width].reshape(n_seq, width)
        for i, s in enumerate(seqs):
            tab[i, :len(s.blocks)] = s.blocks
        o += n_seq * width
        host[o:o + n_seq] = ctx
        t = torch.from_numpy(host)
        if self.device.type == "cuda":
            t = t.pin_memory()
        dev = t.to(self.device, non_blocking=True)
        o = 2 * n_tok
        return Batch(input_ids=dev[:n_tok], positions=dev[n_tok:o],
                     cu_seqlens=dev[o:o + n_seq + 1].to(torch.int32),
                     max_seqlen=max(cu[i + 1] - cu[i] for i in range(n_seq)) if n_seq else 1,
                     block_table=dev[o + n_seq + 1:o + n_seq + 1 + n_seq * width]
                     .to(torch.int32).view(n_seq, width),
                     context_lens=dev[o + n_seq + 1 + n_seq * width:].to(torch.int32),
                     is_prefill=is_prefill)

    # ------------------------------------------------------------------ decode graphs

    @torch.no_grad()
    def enable_decode_graphs(self, max_model_len: int, buckets=DEFAULT_BUCKETS) -> None:
        """Capture one decode graph per batch bucket, largest first in one memory pool."""
        width = -(-max_model_len // self.block_size)
        cap = max(buckets)
        rows = _DecodeRows(cap, width, self.scratch_block, self.device)
        self._rows = rows
        self._cu = torch.arange(cap + 1, dtype=torch.int32, device=self.device)
        pool = torch.cuda.graph_pool_handle()
        for b in sorted(buckets, reverse=True):
            self._decode_body(b)                 # warm-up: loads kernels, sizes workspaces
            torch.cuda.synchronize(self.device)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, pool=pool):
                logits = self._decode_body(b)
            self._graphs[b] = (g, logits)
        torch.cuda.synchronize(self.device)

    def _decode_body(self, b: int) -> torch.Tensor:
        """The captured decode step of the first b rows: the forward, then the greedy
        argmax of every row (ndl_greedy_argmax, which records no memset), written into the
        rows' input tokens for the next step."""
        rows = self._rows
        ctx = rows.ctx[:b]
        logits = self.model(rows.tok[:b], ctx.long(), self.kv_caches, rows.table[:b],
                            self._cu[:b + 1], ctx, 1, False)
        ops.greedy_argmax(logits, out=rows.tok[:b])
        return logits

    def _graph_decode(self, seqs: List[SeqState]) -> Optional[List[int]]:
        rows = self._rows
        if not rows.fits(seqs, self.block_size):
            return None
        for s in seqs:
            check_greedy(s.params)
        b = len(seqs)
        bucket = next((k for k in sorted(self._graphs) if k >= b), None)
        if bucket is None:
            return None
        rows.sync(seqs)
        g, _ = self._graphs[bucket]
        g.replay()                               # the next step's input ids stay on the device
        greedy = rows.tok[:b].tolist()           # one host copy (row order)
        where = rows.row_of()
        order = [where[id(s)] for s in seqs]
        out = [greedy[r] for r in order]
        for r in range(b):
            rows.tok_on_device[r] = True
        return out

    # ------------------------------------------------------------------ swapping

    def swap(self, mapping: Dict[int, int], to_cpu: bool) -> None:
        """Copy the blocks of `mapping` (source id -> destination id) of every layer between
        the GPU pools and the pinned CPU pools, in one launch."""
        if not mapping or not self.cpu_kv_caches:
            return
        ids = torch.tensor([list(mapping.keys()), list(mapping.values())], dtype=torch.int32)
        ids = ids.pin_memory().to(self.device, non_blocking=True)
        src, dst = (self.kv_caches, self.cpu_kv_caches) if to_cpu else \
            (self.cpu_kv_caches, self.kv_caches)
        ops.kv_block_copy(dst, src, ids[0], ids[1])
