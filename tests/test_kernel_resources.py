"""The search kernels must not use scratch (private) memory.

With promotion of private arrays to registers turned off (a flag the build
needs for speed), a private array indexed by a run-time value is kept in
scratch memory, where an index outside the array is an out-of-bounds memory
access on the device rather than a wrong value.  This compiles the kernel
source to device assembly with the product flags and checks every kernel's
ScratchSize."""
from __future__ import annotations

import os
import re
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
HIPCC = "/opt/rocm/bin/hipcc"


def _flags():
    mk = open(os.path.join(ROOT, "flashgann_amd", "csrc", "Makefile")).read()
    m = re.search(r"HIPFLAGS := (.*?)\n(?!\s)", mk, re.S)
    flags = m.group(1).replace("\\\n", " ").replace("$(ARCH)", "gfx950").split()
    return [f for f in flags if f != "-fPIC"]


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
def test_no_kernel_uses_scratch(tmp_path):
    out = tmp_path / "fg_search.s"
    src = os.path.join(ROOT, "flashgann_amd", "csrc", "fg_search.hip")
    cmd = [HIPCC, *_flags(), "--cuda-device-only", "-S", "-o", str(out), src]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    asm = out.read_text()
    names = re.findall(r"^(_Z\w+):\s*;\s*@", asm, re.M)
    sizes = [int(x) for x in re.findall(r"; ScratchSize: (\d+)", asm)]
    assert len(sizes) == len(names) and len(names) >= 20, (len(names), len(sizes))
    bad = [(n, s) for n, s in zip(names, sizes) if s != 0]
    assert not bad, bad
