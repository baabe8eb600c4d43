"""The search kernels must not use scratch (private) memory.

With promotion of private arrays to registers turned off (a flag the build
needs for speed), a private array indexed by a run-time value is kept in
scratch memory, where an index outside the array is an out-of-bounds memory
access on the device rather than a wrong value.  This compiles every kernel
source (the host side's and each shape class's object) to device assembly
with the product flags and checks every kernel's ScratchSize."""
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
    csrc = os.path.join(ROOT, "flashgann_amd", "csrc")
    # the host side's kernels and each shape class's object, compiled in parallel
    units = [("fg_search", os.path.join(csrc, "fg_search.hip"), [])]
    units += [(f"fg_shape{i}", os.path.join(csrc, "fg_shapes.hip"), [f"-DFG_SHAPE={i}"]) for i in range(7)]
    procs = []
    for name, src, extra in units:
        out = tmp_path / f"{name}.s"
        cmd = [HIPCC, *_flags(), *extra, "--cuda-device-only", "-S", "-o", str(out), src]
        procs.append((name, out, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)))
    names, sizes = [], []
    for name, out, p in procs:
        _, err = p.communicate(timeout=900)
        assert p.returncode == 0, (name, err[-2000:])
        asm = out.read_text()
        n = re.findall(r"^(_Z\w+):\s*;\s*@", asm, re.M)
        z = [int(x) for x in re.findall(r"; ScratchSize: (\d+)", asm)]
        assert len(z) == len(n), (name, len(n), len(z))
        names += n
        sizes += z
    assert len(names) >= 80, len(names)
    bad = [(n, s) for n, s in zip(names, sizes) if s != 0]
    assert not bad, bad
