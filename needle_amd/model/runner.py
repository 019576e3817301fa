"""ModelRunner: KV pools, batch metadata and one forward per step.

Follows needle/model/runner.py:14-249 of the reference:
  * one KV pool per layer, [2, num_blocks, num_kv_heads, block_size, head_dim] in the
    model dtype, zero-initialised (:65-78), plus an optional pinned CPU swap pool (:80-94);
  * _prepare_inputs (:194-249): prefill feeds every token with context 0, decode the
    last token with context length-1; positions ctx..ctx+n; cu_seqlens; block_table
    padded with the dummy id num_blocks-1; max_seqlen from the host lists;
  * a batch holding both prefill and decode sequences runs two forwards (:121-148).
Differences:
  * the metadata goes to the device in one pinned copy instead of five tensors;
  * greedy sampling is one device argmax with one host copy for the whole batch
    (the reference syncs once per sequence, sampler.py:24-29); non-greedy requests
    use needle_amd.model.sampler;
  * swapping copies all moved blocks of a layer with one gather and one scatter
    (the reference copies one block at a time, runner.py:187-192);
  * optionally, decode forwards replay HIP graphs captured per batch-size bucket
    (enable_decode_graphs): the ~30 kernels of each layer launch from one graph
    instead of one Python call each.  Rows beyond the live batch point at a
    reserved scratch block that the allocator never hands out.
"""
from __future__ import annotations

from typing import List, Optional

import torch

from ..backend.sequence import ExecuteInput, ExecuteOutput, SchedulerOutput
from .config import ModelConfig
from .qwen2 import build_model, random_init_
from .sampler import sample


class ModelRunner:
    def __init__(self, model_config: ModelConfig, block_size: int = 16, dtype: str = "bfloat16",
                 device: str = "cuda:0", seed: int = 0, model: Optional[torch.nn.Module] = None):
        self.model_config = model_config
        self.block_size = block_size
        self.device = torch.device(device)
        self.dtype = getattr(torch, dtype)
        if model is None:
            model = random_init_(build_model(model_config), seed)
        self.model = model.to(device=self.device, dtype=self.dtype).eval()
        self.kv_caches: List[torch.Tensor] = []
        self.cpu_kv_caches: List[torch.Tensor] = []
        self._graphs = {}
        self._graph_width = 0

    def bytes_per_block(self) -> int:
        cfg = self.model_config
        return (2 * cfg.num_kv_heads * self.block_size * cfg.head_dim
                * torch.finfo(self.dtype).bits // 8 * cfg.num_hidden_layers)

    def profile_memory(self, gpu_memory_utilization: float = 0.90, max_gpu_blocks: int = 0,
                       cpu_swap_bytes: int = 0):
        """runner.py:44-63: blocks that fit in the free device memory (optionally capped),
        and a CPU swap pool of cpu_swap_bytes (the reference sizes it at half the GPU pool)."""
        if self.device.type != "cuda":                       # runner.py:46-47
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

    @torch.no_grad()
    def execute(self, sched_out: SchedulerOutput) -> ExecuteOutput:
        if sched_out.swap_out_map and self.cpu_kv_caches:
            self._swap(sched_out.swap_out_map, to_cpu=True)
        if sched_out.swap_in_map and self.cpu_kv_caches:
            self._swap(sched_out.swap_in_map, to_cpu=False)
        logits = []
        groups = [g for g in (sched_out.prefill_seqs, sched_out.decode_seqs) if g]
        for seqs in groups:
            prefill = not seqs[0].prefilled
            out = None if prefill or not self._graphs else \
                self._graph_decode(seqs, sched_out.block_tables)
            if out is None:
                out = self.forward(self.prepare_inputs(seqs, sched_out.block_tables, prefill))
            logits.append(out)
        all_seqs = sched_out.prefill_seqs + sched_out.decode_seqs
        logits = logits[0] if len(logits) == 1 else torch.cat(logits, dim=0)
        tokens = sample(logits, [s.request.sampling_params for s in all_seqs])
        for s in sched_out.prefill_seqs:
            s.prefilled = True
        return ExecuteOutput(seq_ids=[s.seq_id for s in all_seqs], next_token_ids=tokens)

    # ------------------------------------------------------------------ decode graphs

    DEFAULT_BUCKETS = (1, 2, 4, 8, 12, 16, 24, 32, 48, 64, 96, 128, 192, 256)

    @property
    def scratch_block(self) -> int:
        """The last pool block: padding rows of captured decode batches write here.
        The engine keeps it out of the allocator when graphs are enabled."""
        return self.kv_caches[0].shape[1] - 1

    @torch.no_grad()
    def enable_decode_graphs(self, max_model_len: int, buckets=DEFAULT_BUCKETS) -> None:
        """Capture one decode graph per batch bucket (largest first, so workspaces the
        first capture sizes are never reallocated under a later graph)."""
        bs = self.block_size
        width = (max_model_len + bs - 1) // bs
        bmax = max(buckets)
        dev = self.device
        self._graph_width = width
        self._st_ids = torch.zeros(bmax, dtype=torch.int64, device=dev)
        self._st_pos = torch.zeros(bmax, dtype=torch.int64, device=dev)
        self._st_ctx = torch.zeros(bmax, dtype=torch.int32, device=dev)
        self._st_bt = torch.full((bmax, width), self.scratch_block, dtype=torch.int32, device=dev)
        self._st_cu = torch.arange(bmax + 1, dtype=torch.int32, device=dev)
        pool = torch.cuda.graph_pool_handle()
        for b in sorted(buckets, reverse=True):
            args = (self._st_ids[:b], self._st_pos[:b], self.kv_caches, self._st_bt[:b],
                    self._st_cu[:b + 1], self._st_ctx[:b], 1, False)
            self.model(*args)                       # warm-up: sizes workspaces, loads kernels
            torch.cuda.synchronize(dev)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, pool=pool):
                out = self.model(*args)
            self._graphs[b] = (g, out)
        torch.cuda.synchronize(dev)

    def _graph_decode(self, seqs, block_tables):
        b = len(seqs)
        bucket = next((k for k in sorted(self._graphs) if k >= b), None)
        if bucket is None or any(s.length > self._graph_width * self.block_size for s in seqs):
            return None
        width, scratch = self._graph_width, self.scratch_block
        ids = [s.last_token_id for s in seqs] + [0] * (bucket - b)
        ctx = [s.length - 1 for s in seqs] + [0] * (bucket - b)
        table: List[int] = []
        for s in seqs:
            row = block_tables.get(s.seq_id, [])
            table.extend(row + [scratch] * (width - len(row)))
        table.extend([scratch] * (width * (bucket - b)))
        host = torch.tensor(ids + ctx + table, dtype=torch.int64).pin_memory()
        dev = host.to(self.device, non_blocking=True)
        self._st_ids[:bucket].copy_(dev[:bucket])
        self._st_pos[:bucket].copy_(dev[bucket:2 * bucket])
        self._st_ctx[:bucket].copy_(dev[bucket:2 * bucket])
        self._st_bt[:bucket].copy_(dev[2 * bucket:].view(bucket, width))
        g, out = self._graphs[bucket]
        g.replay()
        return out[:b]

    def forward(self, inp: ExecuteInput) -> torch.Tensor:
        return self.model(inp.input_ids, inp.position_ids, self.kv_caches, inp.block_table,
                          inp.cu_seqlens, inp.context_lens, inp.max_seqlen, inp.is_prefill)

    def prepare_inputs(self, seqs, block_tables, is_prefill: bool) -> ExecuteInput:
        ids: List[int] = []
        pos: List[int] = []
        cu: List[int] = [0]
        ctx: List[int] = []
        for s in seqs:
            if is_prefill:
                toks, c = s.token_ids, 0
            else:
                toks, c = [s.last_token_id], s.length - 1
            ids.extend(toks)
            pos.extend(range(c, c + len(toks)))
            cu.append(cu[-1] + len(toks))
            ctx.append(c)
        width = max((len(block_tables.get(s.seq_id, [])) for s in seqs), default=1) or 1
        dummy = (self.kv_caches[0].shape[1] if self.kv_caches else 1) - 1
        table: List[int] = []
        for s in seqs:
            row = block_tables.get(s.seq_id, [])
            table.extend(row + [dummy] * (width - len(row)))
        n_tok, n_seq = len(ids), len(seqs)
        # One pinned int64 staging buffer -> one host-to-device copy.
        host = torch.tensor(ids + pos + cu + table + ctx, dtype=torch.int64)
        if self.device.type == "cuda":
            host = host.pin_memory()
        dev = host.to(self.device, non_blocking=True)
        o = 0
        input_ids = dev[o:o + n_tok]; o += n_tok
        positions = dev[o:o + n_tok]; o += n_tok
        cu_t = dev[o:o + n_seq + 1].to(torch.int32); o += n_seq + 1
        bt = dev[o:o + n_seq * width].to(torch.int32).view(n_seq, width); o += n_seq * width
        ctx_t = dev[o:o + n_seq].to(torch.int32)
        max_seqlen = max(cu[i + 1] - cu[i] for i in range(n_seq)) if n_seq else 1
        return ExecuteInput(input_ids=input_ids, position_ids=positions, cu_seqlens=cu_t,
                            max_seqlen=max_seqlen, block_table=bt, context_lens=ctx_t,
                            is_prefill=is_prefill)

    def _swap(self, mapping: dict, to_cpu: bool) -> None:
        src = torch.tensor(list(mapping.keys()), dtype=torch.long)
        dst = torch.tensor(list(mapping.values()), dtype=torch.long)
        for gpu, cpu in zip(self.kv_caches, self.cpu_kv_caches):
            if to_cpu:
                cpu[:, dst] = gpu[:, src.to(self.device)].cpu()
            else:
                gpu[:, dst.to(self.device)] = cpu[:, src].to(self.device)
