"""Checks on the generated gfx950 code that the kernels' correctness relies on.

varlen_prefill issues its direct global->LDS loads from inline asm that writes
M0; M0 is reserved, so the compiler cannot be told about the clobber.  That is
sound only while nothing else in the prefill kernels uses M0.

RoPE is bit-exact against the reference only while every product and every sum
is rounded to the element format on its own (needle/layers/attention.py:277-283
in float16 or bfloat16).  The fp32 product of two fp16 values is exact, so the
compiler may narrow it to an fp16 multiply; a fused fp16 multiply-add formed
from that would skip the product's rounding.
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "needle_amd", "csrc")
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

pytestmark = pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")


def prefill_flags():
    """The extra compiler flags the Makefile gives varlen_prefill.hip (PREFILL_FLAGS, which
    the Makefile keeps only when this toolchain accepts them)."""
    out = subprocess.check_output(["make", "-s", "-C", CSRC, "print-prefill-flags"], text=True)
    return out.split()


@pytest.fixture(scope="module")
def device_asm(tmp_path_factory):
    """name -> lines of the gfx950 assembly of needle_amd/csrc/<name>.hip, built with the
    Makefile's flags, compiled once per module."""
    cache = {}
    out_dir = tmp_path_factory.mktemp("asm")

    def get(name):
        if name not in cache:
            asm = out_dir / f"{name}.s"
            extra = prefill_flags() if name == "varlen_prefill" else []
            subprocess.check_call([HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17",
                                   "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                                   "-I" + os.path.join(ROOT, "include"), *extra, "-S",
                                   "--cuda-device-only", os.path.join(CSRC, f"{name}.hip"),
                                   "-o", str(asm)], stderr=subprocess.DEVNULL)
            cache[name] = asm.read_text().splitlines()
        return cache[name]
    return get


def test_prefill_kernels_use_m0_only_for_direct_lds_loads(device_asm):
    lines = device_asm("varlen_prefill")
    kernels = [i for i, l in enumerate(lines)
               if re.match(r"_ZN3ndl21varlen_prefill_kernel.*:", l)]
    assert len(kernels) == 8          # head_dim 64 and 128, with and without RoPE of q, bf16 and fp16
    for start in kernels:
        end = next(i for i in range(start, len(lines)) if lines[i].startswith(".Lfunc_end"))
        body = [l.strip() for l in lines[start:end] if not l.strip().startswith(";")]
        uses = [l for l in body if re.search(r"\bm0\b", l)]
        assert uses, "expected the direct-load M0 writes"
        for i, l in enumerate(body):
            if not re.search(r"\bm0\b", l):
                continue
            assert l.startswith("s_mov_b32 m0, s"), l
            assert body[i + 1] == "s_nop 0" and re.match(r"global_load_lds_dword(x4)? ", body[i + 2]), \
                body[i:i + 3]


# fused multiply-adds that round once where RoPE rounds twice; v_fma_mix*_f16 with an addend
# of 0 is a product rounded once to fp16 (the attention outputs' conversion) and is allowed
_F16_FMA = re.compile(r"^(v_pk_fma_f16|v_fma_f16|v_fmac_f16\w*|v_fmamk_f16|v_fmaak_f16|"
                      r"v_pk_mad_f16|v_mad_f16|v_mac_f16\w*|v_fma_dot2\w*|v_mad_mix\w*)\b")
_MIX = re.compile(r"^v_fma_mix(lo|hi)?_f(16|32)\s+(\S+),\s*(\S+),\s*(\S+),\s*(\S+)")


@pytest.mark.parametrize("name", ["kv_append", "rope_append", "paged_decode", "varlen_prefill"])
def test_no_fused_fp16_multiply_add(device_asm, name):
    bad = []
    for l in device_asm(name):
        s = l.strip()
        if _F16_FMA.match(s):
            bad.append(s)
        m = _MIX.match(s)
        if m and m.group(6) != "0":
            bad.append(s)
    assert not bad, bad[:5]
