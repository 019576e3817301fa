"""Checks on the generated gfx950 code that the kernels' correctness relies on.

varlen_prefill issues its direct global->LDS loads from inline asm that writes
M0; M0 is reserved, so the compiler cannot be told about the clobber.  That is
sound only while nothing else in the prefill kernels uses M0.
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


def prefill_flags():
    """The extra compiler flags the Makefile gives varlen_prefill.hip (PREFILL_FLAGS, which
    the Makefile keeps only when this toolchain accepts them)."""
    out = subprocess.check_output(["make", "-s", "-C", os.path.join(ROOT, "needle_amd", "csrc"),
                                   "print-prefill-flags"], text=True)
    return out.split()


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
def test_prefill_kernels_use_m0_only_for_direct_lds_loads(tmp_path):
    src = os.path.join(ROOT, "needle_amd", "csrc", "varlen_prefill.hip")
    asm = tmp_path / "vp.s"
    subprocess.check_call([HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang",
                           "-target-feature", "-Xclang", "-packed-fp32-ops",
                           "-I" + os.path.join(ROOT, "include"), *prefill_flags(), "-S",
                           "--cuda-device-only", src, "-o", str(asm)], stderr=subprocess.DEVNULL)
    lines = asm.read_text().splitlines()
    kernels = [i for i, l in enumerate(lines)
               if re.match(r"_ZN3ndl21varlen_prefill_kernel.*:", l)]
    assert len(kernels) == 4          # head_dim 64 and 128, each with and without RoPE of q
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
