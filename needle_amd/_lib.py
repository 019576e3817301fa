"""ctypes binding of libneedle_amd.so (the C ABI declared in include/needle_amd.h).

torch is imported first so that the HIP runtime torch ships is the one the
library binds to (both carry the SONAME libamdhip64.so.7).  A missing library
is an error: there is no fallback path.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch  # noqa: F401  (loads torch's HIP runtime before ours)

_PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = _PKG_DIR / "libneedle_amd.so"

NDL_ABI_VERSION = 8
NDL_DECODE_STATIC_SCRATCH_BYTES = 16 << 20
NDL_DTYPE_BF16 = 0
NDL_DTYPE_F16 = 1
NDL_DTYPE_F32 = 2

# Every extern "C" symbol include/needle_amd.h declares.
EXPORTED_SYMBOLS = (
    "ndl_abi_version",
    "ndl_strerror",
    "ndl_kv_append",
    "ndl_rope_kv_append",
    "ndl_paged_decode_workspace_bytes",
    "ndl_paged_decode",
    "ndl_paged_decode_append",
    "ndl_paged_decode_append_noalloc",
    "ndl_rope_paged_decode_append",
    "ndl_varlen_prefill",
    "ndl_rope_varlen_prefill",
    "ndl_kv_block_copy",
    "ndl_rms_norm",
    "ndl_silu_mul",
    "ndl_greedy_argmax_workspace_bytes",
    "ndl_greedy_argmax",
)

_c_i32 = ctypes.c_int
_c_i64 = ctypes.c_int64
_c_p = ctypes.c_void_p
_c_f32 = ctypes.c_float
_c_sz = ctypes.c_size_t

_SIGNATURES = {
    "ndl_abi_version": (_c_i32, []),
    "ndl_strerror": (ctypes.c_char_p, [_c_i32]),
    "ndl_kv_append": (_c_i32, [
        _c_p, _c_i64, _c_i32, _c_i32, _c_i32, _c_i32,   # cache, NB, Hkv, bs, D, dtype
        _c_p, _c_i64, _c_p, _c_i64,                     # k, k stride, v, v stride
        _c_p, _c_i64, _c_i32,                           # block_table, row stride, W
        _c_p, _c_p, _c_i32, _c_i64, _c_p,               # cu, ctx, B, T, stream
    ]),
    "ndl_rope_kv_append": (_c_i32, [
        _c_p, _c_p, _c_i64,                             # q_out, q, q stride
        _c_p, _c_i64, _c_p, _c_i64,                     # k, k stride, v, v stride
        _c_p, _c_p, _c_i64,                             # cos, sin, cos/sin stride
        _c_p, _c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32,  # cache, NB, H, Hkv, bs, D, dtype
        _c_p, _c_i64, _c_i32,                           # block_table, row stride, W
        _c_p, _c_p, _c_i32, _c_i64, _c_p,               # cu, ctx, B, T, stream
    ]),
    "ndl_paged_decode_workspace_bytes": (_c_sz, [_c_i32] * 7),
    "ndl_paged_decode": (_c_i32, [
        _c_p, _c_p, _c_i64,                             # out, q, q stride
        _c_p, _c_i64,                                   # cache, NB
        _c_p, _c_i64, _c_i32,                           # block_table, row stride, W
        _c_p, _c_i32,                                   # ctx, B
        _c_i32, _c_i32, _c_i32, _c_i32, _c_i32,         # H, Hkv, D, bs, dtype
        _c_f32, _c_i32,                                 # scale, partition
        _c_p, _c_sz, _c_p,                              # workspace, bytes, stream
    ]),
    "ndl_paged_decode_append": (_c_i32, [
        _c_p, _c_p, _c_i64,                             # out, q, q stride
        _c_p, _c_i64, _c_p, _c_i64,                     # k, k stride, v, v stride
        _c_p, _c_i64,                                   # cache, NB
        _c_p, _c_i64, _c_i32,                           # block_table, row stride, W
        _c_p, _c_i32,                                   # ctx, B
        _c_i32, _c_i32, _c_i32, _c_i32, _c_i32,         # H, Hkv, D, bs, dtype
        _c_f32, _c_i32,                                 # scale, partition
        _c_p, _c_sz, _c_p,                              # workspace, bytes, stream
    ]),
    "ndl_paged_decode_append_noalloc": (_c_i32, [
        _c_p, _c_p, _c_i64,                             # out, q, q stride
        _c_p, _c_i64, _c_p, _c_i64,                     # k, k stride, v, v stride
        _c_p, _c_i64,                                   # cache, NB
        _c_p, _c_i64, _c_i32,                           # block_table, row stride, W
        _c_p, _c_i32,                                   # ctx, B
        _c_i32, _c_i32, _c_i32, _c_i32, _c_i32,         # H, Hkv, D, bs, dtype
        _c_f32, _c_i32, _c_p,                           # scale, partition, stream
    ]),
    "ndl_rope_paged_decode_append": (_c_i32, [
        _c_p, _c_p, _c_i64,                             # out, q, q stride
        _c_p, _c_i64, _c_p, _c_i64,                     # k, k stride, v, v stride
        _c_p, _c_p, _c_i64,                             # cos, sin, cos/sin stride
        _c_p, _c_i64,                                   # cache, NB
        _c_p, _c_i64, _c_i32,                           # block_table, row stride, W
        _c_p, _c_i32,                                   # ctx, B
        _c_i32, _c_i32, _c_i32, _c_i32, _c_i32,         # H, Hkv, D, bs, dtype
        _c_f32, _c_i32,                                 # scale, partition
        _c_p, _c_sz, _c_p,                              # workspace, bytes, stream
    ]),
    "ndl_varlen_prefill": (_c_i32, [
        _c_p, _c_p, _c_i64,                             # out, q, q stride
        _c_p, _c_i64,                                   # cache, NB
        _c_p, _c_i64, _c_i32,                           # block_table, row stride, W
        _c_p, _c_p, _c_i32, _c_i64, _c_i32, _c_i32,     # cu, ctx, B, T, max_seqlen, max_ctx
        _c_i32, _c_i32, _c_i32, _c_i32, _c_i32,         # H, Hkv, D, bs, dtype
        _c_f32, _c_p,                                   # scale, stream
    ]),
    "ndl_rope_varlen_prefill": (_c_i32, [
        _c_p, _c_p, _c_i64,                             # out, q, q stride
        _c_p, _c_p, _c_i64,                             # cos, sin, cos/sin stride
        _c_p, _c_i64,                                   # cache, NB
        _c_p, _c_i64, _c_i32,                           # block_table, row stride, W
        _c_p, _c_p, _c_i32, _c_i64, _c_i32, _c_i32,     # cu, ctx, B, T, max_seqlen, max_ctx
        _c_i32, _c_i32, _c_i32, _c_i32, _c_i32,         # H, Hkv, D, bs, dtype
        _c_f32, _c_p,                                   # scale, stream
    ]),
    "ndl_kv_block_copy": (_c_i32, [
        _c_p, _c_i64, _c_p, _c_i64,                     # dst pools, dst NB, src pools, src NB
        _c_i32, _c_i32, _c_i32, _c_i32, _c_i32,         # layers, Hkv, bs, D, dtype
        _c_p, _c_p, _c_i32, _c_p,                       # src ids, dst ids, pairs, stream
    ]),
    "ndl_rms_norm": (_c_i32, [
        _c_p, _c_p, _c_p, _c_i64,                       # out, residual out, x, x stride
        _c_p, _c_p, _c_i64, _c_i32,                     # residual, weight, rows, hidden
        _c_f32, _c_i32, _c_p,                           # eps, dtype, stream
    ]),
    "ndl_silu_mul": (_c_i32, [
        _c_p, _c_p, _c_i64, _c_p, _c_i64,               # out, gate, stride, up, stride
        _c_i64, _c_i32, _c_i32, _c_p,                   # rows, intermediate, dtype, stream
    ]),
    "ndl_greedy_argmax_workspace_bytes": (_c_sz, [_c_i64, _c_i32]),   # rows, vocab
    "ndl_greedy_argmax": (_c_i32, [
        _c_p, _c_i32, _c_p, _c_i64,                     # out, out int64, logits, stride
        _c_i64, _c_i32, _c_i32,                         # rows, vocab, dtype
        _c_p, _c_sz, _c_p,                              # workspace, bytes, stream
    ]),
}

_LIB = None


class NeedleAmdError(RuntimeError):
    """A non-zero status returned through the C ABI."""


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raise if it has not been built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    path = Path(os.environ.get("NEEDLE_AMD_LIB", LIB_PATH))
    if not path.exists():
        raise NeedleAmdError(
            f"{path} not found: build it with `make -C needle_amd/csrc` "
            "(or __graft_entry__.build()); there is no non-HIP fallback")
    lib = ctypes.CDLL(str(path), mode=ctypes.RTLD_GLOBAL)
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    ver = lib.ndl_abi_version()
    if ver != NDL_ABI_VERSION:
        raise NeedleAmdError(f"ABI version {ver} != expected {NDL_ABI_VERSION}")
    _LIB = lib
    return lib


def check(status: int, what: str) -> None:
    if status != 0:
        msg = load().ndl_strerror(status).decode()
        raise NeedleAmdError(f"{what}: status {status} ({msg})")
