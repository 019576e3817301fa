"""torch-facing wrappers of the HIP paged-KV operations.

Each function mirrors one seam of needle/layers/attention.py (rms_norm and
silu_mul: the decoder layer's elementwise ops around it, needle/model/qwen2.py:52-65)
and forwards device pointers to the C ABI (include/needle_amd.h) on torch's current
stream.  Nothing here computes on the host: the HIP library is required.

Argument meaning follows the reference:
  kv_cache      [2, num_blocks, num_kv_heads, block_size, head_dim]   (attention.py:9-10)
  block_table   int32 [num_seqs, max_blocks_per_seq]                  (runner.py:220-235)
  context_lens  int32 [num_seqs], tokens already cached               (runner.py:204-218)
  cu_seqlens    int32 [num_seqs + 1], packed token offsets           (runner.py:217)
"""
from __future__ import annotations

import os
from typing import Optional

import torch

from . import _lib

_DTYPES = {torch.bfloat16: _lib.NDL_DTYPE_BF16, torch.float16: _lib.NDL_DTYPE_F16,
           torch.float32: _lib.NDL_DTYPE_F32}


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(dev: torch.device) -> int:
    """The raw handle of torch's current stream on dev (what current_stream(dev).cuda_stream
    gives, without building a Stream object on every call where torch exposes the handle)."""
    if _raw_stream is None:
        return torch.cuda.current_stream(dev).cuda_stream
    idx = dev.index
    return _raw_stream(torch.cuda.current_device() if idx is None else idx)


def _require(cond: bool, msg: str, exc=ValueError) -> None:
    if not cond:
        raise exc(msg)


def _check_cache(kv_cache: torch.Tensor) -> None:
    if kv_cache.dim() != 5 or kv_cache.shape[0] != 2:
        raise ValueError("kv_cache must be [2, num_blocks, num_kv_heads, block_size, "
                         f"head_dim], got {tuple(kv_cache.shape)}")
    _require(kv_cache.is_cuda, "kv_cache must be a GPU tensor")
    _require(kv_cache.is_contiguous(), "kv_cache must be contiguous")
    if kv_cache.dtype not in _DTYPES:
        raise TypeError(f"unsupported kv_cache dtype {kv_cache.dtype}")


def _check_int32(name: str, t: torch.Tensor, dim: int, device) -> None:
    # Messages are formatted only on failure: these checks run on every launch.
    if t.dtype != torch.int32:
        raise TypeError(f"{name} must be int32, got {t.dtype}")
    if t.dim() != dim:
        raise ValueError(f"{name} must have {dim} dims, got {t.dim()}")
    if t.device != device:
        raise ValueError(f"{name} must be on {device}, got {t.device}")
    if t.stride(-1) != 1:
        raise ValueError(f"{name} must be contiguous along its last dim")


def _rows(name: str, x: torch.Tensor, n_heads: int, head_dim: int, device) -> int:
    """Token stride of a [T, n_heads, head_dim] tensor with contiguous inner rows."""
    if x.dim() != 3 or x.shape[1] != n_heads or x.shape[2] != head_dim:
        raise ValueError(f"{name} must be [T, {n_heads}, {head_dim}], got {tuple(x.shape)}")
    if x.device != device:
        raise ValueError(f"{name} must be on {device}")
    if x.stride(2) != 1 or x.stride(1) != head_dim:
        raise ValueError(f"{name} rows must be contiguous (strides {x.stride()})")
    return x.stride(0) if x.shape[0] > 1 else n_heads * head_dim


def _validate_enabled() -> bool:
    return os.environ.get("NEEDLE_AMD_VALIDATE", "") not in ("", "0")


def _validate_slots(block_table, num_blocks, name="block_table") -> None:
    """Opt-in host check (syncs) that mirrors the reference's index errors."""
    if block_table.numel() == 0:
        return
    lo, hi = int(block_table.min()), int(block_table.max())
    if lo < 0 or hi >= num_blocks:
        raise IndexError(f"{name} holds block id outside [0, {num_blocks}): [{lo}, {hi}]")


def kv_append(k: torch.Tensor, v: torch.Tensor, kv_cache: torch.Tensor,
              block_table: torch.Tensor, context_lens: torch.Tensor,
              cu_seqlens: Optional[torch.Tensor] = None) -> None:
    """Scatter k/v [T, Hkv, D] into kv_cache in place.

    cu_seqlens=None is the decode form (attention.py:141-154: token i belongs
    to sequence i); otherwise the varlen form of _write_kv (attention.py:204-246).
    """
    _check_cache(kv_cache)
    dev = kv_cache.device
    _, num_blocks, hkv, bs, d = kv_cache.shape
    _require(k.dtype == kv_cache.dtype and v.dtype == kv_cache.dtype,
             "k/v dtype must match kv_cache", TypeError)
    ks = _rows("k", k, hkv, d, dev)
    vs = _rows("v", v, hkv, d, dev)
    _require(k.shape[0] == v.shape[0], "k and v token counts differ")
    _check_int32("block_table", block_table, 2, dev)
    _check_int32("context_lens", context_lens, 1, dev)
    n_seqs = block_table.shape[0]
    _require(context_lens.shape[0] == n_seqs, "context_lens/block_table batch mismatch")
    n_tok = k.shape[0]
    if cu_seqlens is None:
        _require(n_tok == n_seqs, f"decode append needs one token per sequence "
                 f"({n_tok} tokens, {n_seqs} sequences)")
    else:
        _check_int32("cu_seqlens", cu_seqlens, 1, dev)
        _require(cu_seqlens.shape[0] == n_seqs + 1, "cu_seqlens must be [num_seqs + 1]")
    if n_tok == 0:
        return
    _require(block_table.shape[1] > 0, "block_table has no columns")
    if _validate_enabled():
        _validate_slots(block_table, num_blocks)
    lib = _lib.load()
    rc = lib.ndl_kv_append(
        kv_cache.data_ptr(), num_blocks, hkv, bs, d, _DTYPES[kv_cache.dtype],
        k.data_ptr(), ks, v.data_ptr(), vs,
        block_table.data_ptr(), block_table.stride(0), block_table.shape[1],
        _ptr(cu_seqlens), context_lens.data_ptr(), n_seqs, n_tok, _stream(dev))
    _lib.check(rc, "ndl_kv_append")


def rope_kv_append(q: Optional[torch.Tensor], k: torch.Tensor, v: torch.Tensor,
                   cos: torch.Tensor, sin: torch.Tensor, kv_cache: torch.Tensor,
                   block_table: torch.Tensor, context_lens: torch.Tensor,
                   cu_seqlens: Optional[torch.Tensor] = None,
                   out: Optional[torch.Tensor] = None) -> Optional[torch.Tensor]:
    """Rotate q/k by (cos, sin) and append rotated k and v to kv_cache; returns rotated q.

    Same result as _apply_rope (attention.py:88, :277-288) followed by the append
    of attention.py:141-154 (cu_seqlens=None) or _write_kv (:204-246), bit for bit.
    q [T, H, D], k/v [T, Hkv, D], cos/sin [T, D] in the cache dtype (bf16, fp16 or fp32).
    q=None rotates and appends k (and appends v) only, and returns None: the form that
    precedes rope_varlen_prefill, which rotates q itself.
    """
    _check_cache(kv_cache)
    dev = kv_cache.device
    _, num_blocks, hkv, bs, d = kv_cache.shape
    for name, x in (("q", q), ("k", k), ("v", v), ("cos", cos), ("sin", sin)):
        if x is not None and x.dtype != kv_cache.dtype:
            raise TypeError(f"{name} dtype must match kv_cache")
    ks = _rows("k", k, hkv, d, dev)
    vs = _rows("v", v, hkv, d, dev)
    n_tok = k.shape[0]
    if q is not None:
        if q.dim() != 3:
            raise ValueError(f"q must be [T, H, {d}], got {tuple(q.shape)}")
        h = q.shape[1]
        qs = _rows("q", q, h, d, dev)
        _require(q.shape[0] == n_tok, "q/k/v token counts differ")
        if h % hkv:
            raise ValueError(f"num_heads {h} not a multiple of num_kv_heads {hkv}")
    else:
        _require(out is None, "out is the rotated q: pass q with it")
        h, qs = hkv, 0
    _require(v.shape[0] == n_tok, "q/k/v token counts differ")
    if d % 16:
        raise ValueError(f"head_dim {d} must be a multiple of 16")
    for name, x in (("cos", cos), ("sin", sin)):
        if x.dim() != 2 or x.shape[0] != n_tok or x.shape[1] != d:
            raise ValueError(f"{name} must be [{n_tok}, {d}], got {tuple(x.shape)}")
        if x.device != dev or x.stride(1) != 1:
            raise ValueError(f"{name} rows must be contiguous on {dev}")
    _require(cos.stride(0) == sin.stride(0) or n_tok <= 1, "cos and sin token strides differ")
    cs = cos.stride(0) if n_tok > 1 else d
    _check_int32("block_table", block_table, 2, dev)
    _check_int32("context_lens", context_lens, 1, dev)
    n_seqs = block_table.shape[0]
    _require(context_lens.shape[0] == n_seqs, "context_lens/block_table batch mismatch")
    if cu_seqlens is None:
        _require(n_tok == n_seqs, f"decode append needs one token per sequence "
                 f"({n_tok} tokens, {n_seqs} sequences)")
    else:
        _check_int32("cu_seqlens", cu_seqlens, 1, dev)
        _require(cu_seqlens.shape[0] == n_seqs + 1, "cu_seqlens must be [num_seqs + 1]")
    if q is None:
        pass
    elif out is None:
        out = torch.empty((n_tok, h, d), dtype=q.dtype, device=dev)
    else:
        _require(out.shape == (n_tok, h, d) and out.is_contiguous() and out.dtype == q.dtype
                 and out.device == dev, "out must be a contiguous [T, H, D] tensor like q")
    if n_tok == 0:
        return out
    _require(block_table.shape[1] > 0, "block_table has no columns")
    if _validate_enabled():
        _validate_slots(block_table, num_blocks)
    lib = _lib.load()
    rc = lib.ndl_rope_kv_append(
        _ptr(out), _ptr(q), qs, k.data_ptr(), ks, v.data_ptr(), vs,
        cos.data_ptr(), sin.data_ptr(), cs,
        kv_cache.data_ptr(), num_blocks, h, hkv, bs, d, _DTYPES[kv_cache.dtype],
        block_table.data_ptr(), block_table.stride(0), block_table.shape[1],
        _ptr(cu_seqlens), context_lens.data_ptr(), n_seqs, n_tok, _stream(dev))
    _lib.check(rc, "ndl_rope_kv_append")
    return out


def write_kv(k, v, kv_cache, block_table, cu_seqlens, context_lens) -> None:
    """Same signature and effect as the reference _write_kv (attention.py:204-246)."""
    kv_append(k, v, kv_cache, block_table, context_lens, cu_seqlens=cu_seqlens)


def decode_workspace_bytes(num_seqs: int, num_heads: int, num_kv_heads: int, head_dim: int,
                           max_blocks_per_seq: int, block_size: int = 16,
                           partition_tokens: int = 0) -> int:
    return int(_lib.load().ndl_paged_decode_workspace_bytes(
        num_seqs, num_heads, num_kv_heads, head_dim, max_blocks_per_seq, block_size,
        partition_tokens))


def paged_decode(q: torch.Tensor, kv_cache: torch.Tensor, block_table: torch.Tensor,
                 context_lens: torch.Tensor, scale: float, num_heads: int, num_kv_heads: int,
                 head_dim: int, *, partition_tokens: int = 0,
                 out: Optional[torch.Tensor] = None,
                 workspace: Optional[torch.Tensor] = None,
                 new_k: Optional[torch.Tensor] = None,
                 new_v: Optional[torch.Tensor] = None,
                 cos: Optional[torch.Tensor] = None,
                 sin: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Paged decode attention; same signature as _decode_pytorch (attention.py:291).

    Sequence i attends min(context_lens[i] + 1, W * block_size) cached tokens.
    Returns [num_seqs, num_heads, head_dim] in q's dtype.  partition_tokens: 0 lets the
    library choose the split; -1 asks for one 8-wave workgroup per (kv head, sequence);
    a positive multiple of 16 asks for the stream split with that many tokens per wave.

    new_k / new_v ([num_seqs, num_kv_heads, head_dim]): the decode append of this step
    (attention.py:141-154) done in the same launch, with the same cache bytes and output as
    kv_append followed by paged_decode.  Requires that no two sequences attend the same
    block (as BlockAllocator's tables guarantee).

    cos / sin ([num_seqs, head_dim], with new_k / new_v): q and new_k are the projections'
    outputs, not yet rotated; the launch applies the rotary embedding of attention.py:88 to
    both first (bit-identical to rope_kv_append followed by paged_decode).
    """
    _check_cache(kv_cache)
    dev = kv_cache.device
    _, num_blocks, hkv, bs, d = kv_cache.shape
    _require(hkv == num_kv_heads and d == head_dim, "kv_cache shape disagrees with head counts")
    _require(q.dtype == kv_cache.dtype, "q dtype must match kv_cache", TypeError)
    qs = _rows("q", q, num_heads, head_dim, dev)
    _check_int32("block_table", block_table, 2, dev)
    _check_int32("context_lens", context_lens, 1, dev)
    n_seqs = q.shape[0]
    _require(block_table.shape[0] == n_seqs and context_lens.shape[0] == n_seqs,
             "q / block_table / context_lens batch mismatch")
    if out is None:
        out = torch.empty((n_seqs, num_heads, head_dim), dtype=q.dtype, device=dev)
    else:
        _require(out.shape == (n_seqs, num_heads, head_dim) and out.is_contiguous()
                 and out.dtype == q.dtype and out.device == dev, "bad out tensor")
    if n_seqs == 0:
        return out
    _require(block_table.shape[1] > 0, "block_table has no columns")
    if _validate_enabled():
        _validate_slots(block_table, num_blocks)
    lib = _lib.load()
    w = block_table.shape[1]
    need = int(lib.ndl_paged_decode_workspace_bytes(
        n_seqs, num_heads, num_kv_heads, head_dim, w, bs, partition_tokens))
    _require(need > 0, "unsupported decode shape")
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = decode_workspace(need, dev)
    if new_k is None and new_v is None:
        _require(cos is None and sin is None, "cos / sin need new_k / new_v")
        rc = lib.ndl_paged_decode(
            out.data_ptr(), q.data_ptr(), qs, kv_cache.data_ptr(), num_blocks,
            block_table.data_ptr(), block_table.stride(0), w,
            context_lens.data_ptr(), n_seqs, num_heads, num_kv_heads, head_dim, bs,
            _DTYPES[q.dtype], float(scale), partition_tokens, workspace.data_ptr(), need,
            _stream(dev))
        _lib.check(rc, "ndl_paged_decode")
        return out
    _require(new_k is not None and new_v is not None, "new_k and new_v go together")
    for name, x in (("new_k", new_k), ("new_v", new_v)):
        _require(x.dtype == kv_cache.dtype, f"{name} dtype must match kv_cache", TypeError)
        _require(x.shape[0] == n_seqs, f"{name} must have one row per sequence")
    ks = _rows("new_k", new_k, num_kv_heads, head_dim, dev)
    vs = _rows("new_v", new_v, num_kv_heads, head_dim, dev)
    if cos is not None or sin is not None:
        _require(cos is not None and sin is not None, "cos and sin go together")
        for name, x in (("cos", cos), ("sin", sin)):
            _require(x.dtype == kv_cache.dtype, f"{name} dtype must match kv_cache", TypeError)
            _require(x.dim() == 2 and x.shape[0] == n_seqs and x.shape[1] == head_dim,
                     f"{name} must be [{n_seqs}, {head_dim}], got {tuple(x.shape)}")
            _require(x.device == dev and x.stride(1) == 1, f"{name} rows must be contiguous")
        _require(cos.stride(0) == sin.stride(0) or n_seqs <= 1, "cos and sin strides differ")
        cs = cos.stride(0) if n_seqs > 1 else head_dim
        rc = lib.ndl_rope_paged_decode_append(
            out.data_ptr(), q.data_ptr(), qs, new_k.data_ptr(), ks, new_v.data_ptr(), vs,
            cos.data_ptr(), sin.data_ptr(), cs,
            kv_cache.data_ptr(), num_blocks, block_table.data_ptr(), block_table.stride(0), w,
            context_lens.data_ptr(), n_seqs, num_heads, num_kv_heads, head_dim, bs,
            _DTYPES[q.dtype], float(scale), partition_tokens, workspace.data_ptr(), need,
            _stream(dev))
        _lib.check(rc, "ndl_rope_paged_decode_append")
        return out
    rc = lib.ndl_paged_decode_append(
        out.data_ptr(), q.data_ptr(), qs, new_k.data_ptr(), ks, new_v.data_ptr(), vs,
        kv_cache.data_ptr(), num_blocks, block_table.data_ptr(), block_table.stride(0), w,
        context_lens.data_ptr(), n_seqs, num_heads, num_kv_heads, head_dim, bs,
        _DTYPES[q.dtype], float(scale), partition_tokens, workspace.data_ptr(), need,
        _stream(dev))
    _lib.check(rc, "ndl_paged_decode_append")
    return out


def decode_workspace(nbytes: int, device) -> torch.Tensor:
    """Scratch for ndl_paged_decode (no contents are assumed; calls that share one must
    run in stream order)."""
    return torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)


def varlen_prefill(q: torch.Tensor, kv_cache: torch.Tensor, block_table: torch.Tensor,
                   cu_seqlens: torch.Tensor, context_lens: torch.Tensor, max_seqlen: int,
                   scale: float, num_heads: int, num_kv_heads: int, head_dim: int, *,
                   max_context_len: int = 0, out: Optional[torch.Tensor] = None,
                   cos: Optional[torch.Tensor] = None,
                   sin: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Causal attention of packed prompts over the paged cache (after kv_append).

    Equals the reference _prefill_pytorch (attention.py:120-134) when every
    context_lens entry is 0; with a cached prefix the prefix is attended too.
    Returns [num_tokens, num_heads, head_dim].
    With cos/sin ([T, D] rows of the packed tokens), q is the raw projection and each row
    is rotated inside the kernel (ndl_rope_varlen_prefill): the output is bit-identical to
    rope_kv_append's rotated q fed to this function, with k already rotated in the cache
    (rope_kv_append with q=None).
    """
    _check_cache(kv_cache)
    dev = kv_cache.device
    _, num_blocks, hkv, bs, d = kv_cache.shape
    _require(hkv == num_kv_heads and d == head_dim, "kv_cache shape disagrees with head counts")
    _require(q.dtype == kv_cache.dtype, "q dtype must match kv_cache", TypeError)
    qs = _rows("q", q, num_heads, head_dim, dev)
    _check_int32("block_table", block_table, 2, dev)
    _check_int32("cu_seqlens", cu_seqlens, 1, dev)
    _check_int32("context_lens", context_lens, 1, dev)
    n_seqs = block_table.shape[0]
    _require(cu_seqlens.shape[0] == n_seqs + 1 and context_lens.shape[0] == n_seqs,
             "cu_seqlens / context_lens / block_table batch mismatch")
    n_tok = q.shape[0]
    _require((cos is None) == (sin is None), "pass both cos and sin, or neither")
    cs = 0
    if cos is not None:
        for name, x in (("cos", cos), ("sin", sin)):
            if x.dtype != q.dtype:
                raise TypeError(f"{name} dtype must match q")
            if x.dim() != 2 or x.shape[0] != n_tok or x.shape[1] != head_dim:
                raise ValueError(f"{name} must be [{n_tok}, {head_dim}], got {tuple(x.shape)}")
            if x.device != dev or x.stride(1) != 1:
                raise ValueError(f"{name} rows must be contiguous on {dev}")
        _require(cos.stride(0) == sin.stride(0) or n_tok <= 1, "cos and sin token strides differ")
        cs = cos.stride(0) if n_tok > 1 else head_dim
    if out is None:
        out = torch.empty((n_tok, num_heads, head_dim), dtype=q.dtype, device=dev)
    else:
        _require(out.shape == (n_tok, num_heads, head_dim) and out.is_contiguous()
                 and out.dtype == q.dtype and out.device == dev,
                 f"out must be a contiguous {q.dtype} [{n_tok}, {num_heads}, {head_dim}] "
                 f"tensor on {dev}")
    if n_tok == 0 or n_seqs == 0:
        return out
    _require(block_table.shape[1] > 0, "block_table has no columns")
    if _validate_enabled():
        _validate_slots(block_table, num_blocks)
    lib = _lib.load()
    tail = (kv_cache.data_ptr(), num_blocks,
            block_table.data_ptr(), block_table.stride(0), block_table.shape[1],
            cu_seqlens.data_ptr(), context_lens.data_ptr(), n_seqs, n_tok, int(max_seqlen),
            int(max_context_len), num_heads, num_kv_heads, head_dim, bs, _DTYPES[q.dtype],
            float(scale), _stream(dev))
    if cos is None:
        rc = lib.ndl_varlen_prefill(out.data_ptr(), q.data_ptr(), qs, *tail)
        _lib.check(rc, "ndl_varlen_prefill")
    else:
        rc = lib.ndl_rope_varlen_prefill(out.data_ptr(), q.data_ptr(), qs, cos.data_ptr(),
                                         sin.data_ptr(), cs, *tail)
        _lib.check(rc, "ndl_rope_varlen_prefill")
    return out


def kv_block_copy(dst_pools, src_pools, src_ids: torch.Tensor, dst_ids: torch.Tensor) -> None:
    """Copy block src_ids[j] to block dst_ids[j] in every layer's pool, both planes, in one
    launch (the KV swap copies; the reference copies per layer and block,
    runner.py:175-192).

    dst_pools / src_pools: equal-length lists of [2, NB, Hkv, bs, D] tensors, each on the GPU
    or in pinned CPU memory (pin_memory=True).  src_ids / dst_ids: int32 [pairs] on the GPU or
    pinned.  Enqueued on the current stream of the GPU the pools (or ids) live on.
    """
    import ctypes
    _require(len(dst_pools) == len(src_pools), "dst_pools and src_pools differ in length")
    if not dst_pools:
        return
    ref = dst_pools[0]
    _require(ref.dim() == 5 and ref.shape[0] == 2, "pools must be [2, NB, Hkv, bs, D]")
    dev = next((t.device for t in list(dst_pools) + list(src_pools) + [src_ids, dst_ids]
                if t.is_cuda), None)
    _require(dev is not None, "at least one of the pools or ids must be on the GPU")

    def check_pool(t, nb):
        _require(t.dim() == 5 and tuple(t.shape[2:]) == tuple(ref.shape[2:]) and t.shape[0] == 2
                 and t.shape[1] == nb, f"pool shape {tuple(t.shape)} differs from its set")
        _require(t.dtype == ref.dtype and t.dtype in _DTYPES, "pools must share one supported dtype",
                 TypeError)
        _require(t.is_contiguous(), "pools must be contiguous")
        _require(t.device == dev or (t.device.type == "cpu" and t.is_pinned()),
                 "a CPU pool must be pinned (pin_memory=True)")

    dst_nb, src_nb = dst_pools[0].shape[1], src_pools[0].shape[1]
    for t in dst_pools:
        check_pool(t, dst_nb)
    for t in src_pools:
        check_pool(t, src_nb)
    for name, t in (("src_ids", src_ids), ("dst_ids", dst_ids)):
        _require(t.dtype == torch.int32 and t.dim() == 1 and t.is_contiguous(),
                 f"{name} must be a contiguous int32 vector", TypeError)
        _require(t.device == dev or (t.device.type == "cpu" and t.is_pinned()),
                 f"{name} must be on {dev} or pinned")
    _require(src_ids.numel() == dst_ids.numel(), "src_ids and dst_ids differ in length")
    n = src_ids.numel()
    if n == 0:
        return
    arr = ctypes.c_void_p * len(dst_pools)
    dsts = arr(*[t.data_ptr() for t in dst_pools])
    srcs = arr(*[t.data_ptr() for t in src_pools])
    _, _, hkv, bs, d = ref.shape
    lib = _lib.load()
    rc = lib.ndl_kv_block_copy(dsts, dst_nb, srcs, src_nb, len(dst_pools), hkv, bs, d,
                               _DTYPES[ref.dtype], src_ids.data_ptr(), dst_ids.data_ptr(), n,
                               _stream(dev))
    _lib.check(rc, "ndl_kv_block_copy")


def _row_stride(name: str, x: torch.Tensor, width: int, dtype, device) -> int:
    """Row stride of a [rows, width] tensor whose rows are contiguous and 16-byte aligned."""
    if x.dim() != 2 or x.shape[1] != width:
        raise ValueError(f"{name} must be [rows, {width}], got {tuple(x.shape)}")
    if x.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {x.dtype}")
    if x.device != device:
        raise ValueError(f"{name} must be on {device}, got {x.device}")
    if x.stride(1) != 1 and x.shape[1] != 1:
        raise ValueError(f"{name} rows must be contiguous")
    stride = x.stride(0) if x.shape[0] > 1 else width
    if stride % 8 or x.data_ptr() % 16:
        raise ValueError(f"{name} rows must start 16-byte aligned (row stride {stride})")
    return stride


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float,
             residual: Optional[torch.Tensor] = None):
    """RMSNorm of the rows of x (needle/layers/norm.py:14-17), in one kernel.

    Without residual: returns weight * round(x * rsqrt(mean(x^2) + eps)).
    With residual: h = round(x + residual) (the decoder layer's residual add,
    needle/model/qwen2.py:58, :63) and returns (norm of h, h) as new tensors.
    x: [rows, hidden] with contiguous rows; residual: [rows, hidden]; weight: [hidden];
    one dtype (bfloat16, float16 or float32), on one GPU.
    """
    _require(x.is_cuda, "x must be a GPU tensor")
    if x.dtype not in _DTYPES:
        raise TypeError(f"unsupported dtype {x.dtype}")
    if x.dim() != 2:
        raise ValueError(f"x must be [rows, hidden], got {tuple(x.shape)}")
    rows, hidden = x.shape
    stride = _row_stride("x", x, hidden, x.dtype, x.device)
    if (weight.shape != (hidden,) or weight.dtype != x.dtype or weight.device != x.device
            or not weight.is_contiguous()):
        raise ValueError(f"weight must be a contiguous [{hidden}] {x.dtype} tensor on {x.device}")
    out = torch.empty((rows, hidden), dtype=x.dtype, device=x.device)
    res_out = None
    if residual is not None:
        if residual.shape != x.shape or not residual.is_contiguous():
            raise ValueError(f"residual must be a contiguous {tuple(x.shape)} tensor")
        _row_stride("residual", residual, hidden, x.dtype, x.device)
        res_out = torch.empty_like(out)
    lib = _lib.load()
    rc = lib.ndl_rms_norm(out.data_ptr(), _ptr(res_out), x.data_ptr(), stride, _ptr(residual),
                          weight.data_ptr(), rows, hidden, float(eps), _DTYPES[x.dtype],
                          _stream(x.device))
    _lib.check(rc, "ndl_rms_norm")
    return out if residual is None else (out, res_out)


def silu_mul(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """silu(gate) * up of the SwiGLU MLP (needle/model/llama.py:37), in one kernel, with
    torch's roundings (the SiLU rounded to the dtype, then the product).  gate, up:
    [rows, intermediate] with contiguous rows (e.g. the two halves of one fused gate/up
    projection output); returns a new [rows, intermediate] tensor."""
    _require(gate.is_cuda, "gate must be a GPU tensor")
    if gate.dtype not in _DTYPES:
        raise TypeError(f"unsupported dtype {gate.dtype}")
    if gate.dim() != 2:
        raise ValueError(f"gate must be [rows, intermediate], got {tuple(gate.shape)}")
    rows, inter = gate.shape
    gs = _row_stride("gate", gate, inter, gate.dtype, gate.device)
    us = _row_stride("up", up, inter, gate.dtype, gate.device)
    if up.shape[0] != rows:
        raise ValueError(f"up has {up.shape[0]} rows, gate {rows}")
    out = torch.empty((rows, inter), dtype=gate.dtype, device=gate.device)
    lib = _lib.load()
    rc = lib.ndl_silu_mul(out.data_ptr(), gate.data_ptr(), gs, up.data_ptr(), us, rows, inter,
                          _DTYPES[gate.dtype], _stream(gate.device))
    _lib.check(rc, "ndl_silu_mul")
    return out


def greedy_argmax(logits: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The index of each row's maximum, in torch's argmax order (needle/model/sampler.py:
    27-28, for the whole batch: one or two launches, the slices' partials in a workspace
    allocated here, from the graph's pool under capture).  logits: [rows, vocab]; the kernel
    reads contiguous rows that start 16-byte aligned, and other rows (a vocabulary that is not
    a multiple of 8 elements wide, a column slice, a transposed view) are first copied into
    such a buffer on the GPU.  out: int32 or int64 [rows] on the same GPU (a new int64 tensor
    by default).  Graph-capturable."""
    _require(logits.is_cuda, "logits must be a GPU tensor")
    if logits.dtype not in _DTYPES:
        raise TypeError(f"unsupported dtype {logits.dtype}")
    if logits.dim() != 2:
        raise ValueError(f"logits must be [rows, vocab], got {tuple(logits.shape)}")
    rows, vocab = logits.shape
    if rows > 0 and vocab > 0:
        st = logits.stride(0) if rows > 1 else vocab
        if (logits.stride(1) != 1 and vocab > 1) or st % 8 or logits.data_ptr() % 16:
            padded = torch.empty((rows, (vocab + 7) // 8 * 8), dtype=logits.dtype,
                                 device=logits.device)
            padded[:, :vocab].copy_(logits)
            logits = padded[:, :vocab]
    stride = _row_stride("logits", logits, vocab, logits.dtype, logits.device)
    if out is None:
        out = torch.empty(rows, dtype=torch.int64, device=logits.device)
    if (out.dtype not in (torch.int32, torch.int64) or out.shape != (rows,) or
            not out.is_contiguous() or out.device != logits.device):
        raise ValueError(f"out must be a contiguous int32 or int64 [{rows}] tensor on "
                         f"{logits.device}")
    lib = _lib.load()
    nbytes = lib.ndl_greedy_argmax_workspace_bytes(rows, vocab) if rows > 0 else 0
    ws = torch.empty(nbytes, dtype=torch.uint8, device=logits.device) if nbytes else None
    rc = lib.ndl_greedy_argmax(out.data_ptr(), int(out.dtype == torch.int64),
                               logits.data_ptr(), stride, rows, vocab, _DTYPES[logits.dtype],
                               _ptr(ws), nbytes, _stream(logits.device))
    _lib.check(rc, "ndl_greedy_argmax")
    return out
