"""The C ABI library loads and exports what include/needle_amd.h declares.

No kernel runs here (no GPU): only host-side entry points (version, status
text, workspace sizing) and argument rejection paths that return before any
HIP call.
"""
import ctypes
import re
from pathlib import Path

import pytest

from needle_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "needle_amd.h"


def declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ndl_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def test_header_and_binding_agree():
    assert declared_symbols() == sorted(_lib.EXPORTED_SYMBOLS)


def test_every_declared_symbol_is_exported(lib):
    raw = ctypes.CDLL(str(_lib.LIB_PATH))
    for name in declared_symbols():
        assert hasattr(raw, name), name


def test_version_and_status_text(lib):
    assert lib.ndl_abi_version() == _lib.NDL_ABI_VERSION
    assert lib.ndl_strerror(0) == b"ok"
    for code in (-1, -2, -3, -4, -5, -6):
        assert lib.ndl_strerror(code) and lib.ndl_strerror(code) != b"unknown status"
    assert lib.ndl_strerror(-99) == b"unknown status"


def test_decode_workspace_sizing(lib):
    # 2 sequences x 32 heads over 8 kv heads, W = 64 blocks, 256 tokens (16 stream slots)
    # per wave; each sequence takes its tiles and one empty slot of the stream
    # -> ceil(2 * (64 + 1) / 16) = 9 waves per kv head, 9 + 2 segment slots per kv head,
    # one (m, l) pair and one head_dim row per (kv head, segment, group head).
    n = lib.ndl_paged_decode_workspace_bytes(2, 32, 8, 128, 64, 16, 256)
    slots = 8 * (9 + 2) * 4
    ml = (slots * 2 * 4 + 255) // 256 * 256
    assert n == ml + slots * 128 * 4
    # automatic split, stream form (a table of 257 blocks needs more than 16 tiles per
    # wave of an 8-wave workgroup): the resident waves of the device (2048 when there is
    # none to ask) shared by the 8 kv heads; same slot formula
    n = lib.ndl_paged_decode_workspace_bytes(2, 32, 8, 128, 257, 16, 0)
    fits = [w for w in range(1, 4096)
            if n == (8 * (w + 2) * 4 * 8 + 255) // 256 * 256 + 8 * (w + 2) * 4 * 128 * 4]
    assert len(fits) == 1
    # one 8-wave workgroup per (kv head, sequence): nothing leaves the workgroup, a
    # nominal 256 bytes; chosen automatically for 2 x 8 workgroups of 64-block tables
    assert lib.ndl_paged_decode_workspace_bytes(2, 32, 8, 128, 64, 16, -1) == 256
    assert lib.ndl_paged_decode_workspace_bytes(2, 32, 8, 128, 64, 16, 0) == 256
    assert lib.ndl_paged_decode_workspace_bytes(2, 32, 8, 128, 64, 16, -2) == 0
    # unsupported block size / partition not a multiple of 16 / heads not a multiple
    assert lib.ndl_paged_decode_workspace_bytes(2, 32, 8, 128, 64, 48, 256) == 0
    assert lib.ndl_paged_decode_workspace_bytes(2, 32, 8, 128, 64, 16, 100) == 0
    assert lib.ndl_paged_decode_workspace_bytes(2, 32, 6, 128, 64, 16, 0) == 0


def test_rejections_before_any_launch(lib):
    # unsupported dtype / head_dim / block size return without touching a device
    rc = lib.ndl_kv_append(None, 1, 1, 16, 128, 7, None, 0, None, 0, None, 1, 1, None, None,
                           1, 1, None)
    assert rc == -2
    rc = lib.ndl_paged_decode(None, None, 0, None, 1, None, 1, 1, None, 1, 4, 1, 96, 16, 0,
                              1.0, 0, None, 0, None)
    assert rc == -2
    # block sizes: powers of two from 16 to 1024 pass the size check (and fail here on the
    # null arguments); others are not built
    def dec_bs(bs):
        return lib.ndl_paged_decode(None, None, 0, None, 1, None, 1, 1, None, 1, 4, 1, 128, bs,
                                    0, 1.0, 0, None, 0, None)

    def pre_bs(bs):
        return lib.ndl_varlen_prefill(None, None, 4 * 128, None, 1, None, 1, 1, None, None, 1,
                                      1, 1, 0, 4, 1, 128, bs, 0, 1.0, None)
    for bs in (16, 32, 64, 128, 256, 1024):
        assert dec_bs(bs) == -1 and pre_bs(bs) == -1, bs
    for bs in (0, 8, 24, 48, 2048):
        assert dec_bs(bs) == -2 and pre_bs(bs) == -2, bs
    assert lib.ndl_paged_decode_workspace_bytes(2, 32, 8, 128, 64, 8, 0) == 0
    # the split is sized in 16-token tiles: 64 columns of 64 tokens = 256 tiles per row,
    # past the per-sequence split's cap at head_dim 128, so the stream split's workspace
    assert lib.ndl_paged_decode_workspace_bytes(2, 32, 8, 128, 64, 64, 0) > 256
    assert lib.ndl_paged_decode_workspace_bytes(2, 32, 8, 128, 64, 64, 256) == \
        lib.ndl_paged_decode_workspace_bytes(2, 32, 8, 128, 256, 16, 256)
    rc = lib.ndl_paged_decode(None, None, 0, None, 1, None, 1, 1, None, 1, 40, 2, 128, 16, 0,
                              1.0, 0, None, 0, None)
    assert rc == -2  # group 20 > 16
    # a non-multiple-of-16 partition
    rc = lib.ndl_paged_decode(None, None, 512, None, 1, None, 1, 1, None, 1, 4, 1, 128, 16, 0,
                              1.0, 24, None, 0, None)
    assert rc == -1
    # rope_kv_append: an unknown dtype, a head_dim not a multiple of 16, null inputs (fp16
    # passes the dtype check and fails on them)
    def rope(dtype=0, d=128, t=1, q=None):
        return lib.ndl_rope_kv_append(None, q, 4 * d, None, d, None, d, None, None, d,
                                      None, 1, 4, 1, 16, d, dtype, None, 1, 1, None, None, 1, t,
                                      None)
    assert rope(dtype=7) == -2
    assert rope(dtype=1) == -1
    assert rope(d=72) == -2
    assert rope(t=0) == 0
    assert rope() == -1
    # rope_varlen_prefill: cos/sin are required (the plain entry point takes none); an
    # unsupported dtype is refused before any launch
    def rope_prefill(cos=None, dtype=0, cs=128):
        return lib.ndl_rope_varlen_prefill(None, None, 4 * 128, cos, cos, cs, None, 1, None, 1,
                                           1, None, None, 1, 1, 1, 0, 4, 1, 128, 16, dtype, 1.0,
                                           None)
    assert rope_prefill() == -1
    assert rope_prefill(cos=1 << 20, dtype=7) == -2
    assert rope_prefill(cos=1 << 20, cs=100) == -1
    # the allocation-free decode: a shape whose partials exceed the static array is refused
    # after the argument checks and before any device call (1000 sequences x 1000 blocks at
    # 16 tokens per wave); the aligned stand-in addresses are never dereferenced
    assert lib.ndl_paged_decode_workspace_bytes(1000, 32, 8, 128, 1000, 16, 16) > \
        _lib.NDL_DECODE_STATIC_SCRATCH_BYTES
    fake = 1 << 20
    rc = lib.ndl_paged_decode_append_noalloc(fake, fake, 4096, fake, 1024, fake, 1024, fake,
                                             16000, fake, 1000, 1000, fake, 1000, 32, 8, 128, 16,
                                             0, 1.0, 16, None)
    assert rc == -5 and lib.ndl_strerror(rc) != b"unknown status"
    # ... and an unsupported shape gets the workspace entry point's own status
    rc = lib.ndl_paged_decode_append_noalloc(None, None, 4096, None, 1024, None, 1024, None, 1,
                                             None, 1, 1, None, 1, 32, 8, 96, 16, 0, 1.0, 0, None)
    assert rc == -1 or rc == -2
    # nothing to do: zero tokens / sequences
    assert lib.ndl_kv_append(None, 1, 1, 16, 128, 0, None, 128, None, 128, None, 1, 1, None,
                             None, 1, 0, None) == 0


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_LIB", None)
    monkeypatch.setenv("NEEDLE_AMD_LIB", str(tmp_path / "nope.so"))
    with pytest.raises(_lib.NeedleAmdError):
        _lib.load()
