"""Bounds the one choice of the oracle that no test here can pin: where
nvcc's default --fmad=true contracts a multiply and an add into one fused
multiply-add.  The oracle (and the kernel) fuse at six sites: the quantizer
(y - low) * inv + 0.5 (include/utils.cuh:904), the estimator's two
correction terms (:991-992, :1024-1025), the distance accumulations
(:275, :290) and the controller's rho + span * progress
(src/adaptive_search_utils.cuh:109-113).  Without the CUDA toolchain the
reference's actual choice cannot be observed, so this test measures how much
the choice can matter: it rebuilds the oracle with every one of those sites
unfused (a * b + c, rounded twice) and searches the same codebooks with both
builds.  The ids must agree on nearly every query and recall must agree
within the north star's 0.2 percentage points, on integer data (where only
the quantizer, the estimator and the controller round differently) and on
unit-normalised float data (where the exact distances round differently
too)."""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np
import pytest

from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "oracle", "fg_oracle.c")
FMA_SITES = 6


def _unfused_lib(tmp_path):
    src = open(SRC).read()
    code = [ln for ln in src.splitlines() if "fmaf(" in ln and not ln.lstrip().startswith(("*", "/*"))]
    assert len(code) == FMA_SITES, code
    anchor = "#include <string.h>\n"
    assert src.count(anchor) == 1
    # every fmaf below the includes becomes a separately rounded multiply and
    # add (the build passes -ffp-contract=off, so the compiler fuses nothing)
    src = src.replace(anchor, anchor + "#define fmaf(a, b, c) ((a) * (b) + (c))\n")
    (tmp_path / "fg_oracle.c").write_text(src)
    so = tmp_path / "liboracle_unfused.so"
    subprocess.run(["gcc", "-std=c11", "-O2", "-ffp-contract=off", "-fPIC", "-shared", "-pthread",
                    "-I", os.path.join(ROOT, "oracle"), "-o", str(so), str(tmp_path / "fg_oracle.c"), "-lm"],
                   check=True)
    lib = C.CDLL(str(so))
    lib.fgo_search_batch.argtypes = [C.POINTER(O.Index), C.POINTER(C.c_float), C.c_uint64, C.c_int, C.c_int,
                                     C.POINTER(C.c_uint32), C.c_void_p, C.c_int]
    lib.fgo_search_batch.restype = C.c_int
    return lib


def _search(lib, oix, q, K, beam):
    out = np.zeros((q.shape[0], K), np.uint32)
    rc = lib.fgo_search_batch(C.byref(oix.ix), O.ptr(q, C.c_float), q.shape[0], K, beam,
                              O.ptr(out, C.c_uint32), None, os.cpu_count() or 1)
    assert rc == 0
    return out


def _ground_truth(base, q, k):
    d = ((q.astype(np.float64) ** 2).sum(1)[:, None] - 2.0 * q.astype(np.float64) @ base.T.astype(np.float64)
         + (base.astype(np.float64) ** 2).sum(1)[None, :])
    return np.argsort(d, axis=1, kind="stable")[:, :k].astype(np.int32)


@pytest.mark.parametrize("kind", ["int", "unit"])
def test_fma_contraction_choice_is_immaterial(tmp_path, kind):
    from flashgann_amd import builder, datasets
    if kind == "int":
        base, q = datasets.integer_mixture(20000, 500, 128, 64, config=1)
        signs = datasets.signs_for(128, 1)
    else:
        base, q = datasets.normalized_mixture(20000, 500, 96, 64, config=3)
        signs = datasets.signs_for(128, 3)
    cb = builder.build_codebook(base, 32, signs, device="cpu")
    oix = O.OracleIndex.from_codebook(cb)
    q = np.ascontiguousarray(q, np.float32)
    unfused = _unfused_lib(tmp_path)
    gt = _ground_truth(base, q, 100)
    for K, beam in ((10, 64), (100, 256)):
        fused = _search(O.lib(), oix, q, K, beam)
        other = _search(unfused, oix, q, K, beam)
        same = float(np.mean((fused == other).all(axis=1)))
        r_f, r_u = O.recall(fused, gt[:, :K], K), O.recall(other, gt[:, :K], K)
        print(f"{kind} K={K} beam={beam}: identical ids on {same:.3f} of queries, "
              f"recall {r_f:.4f} fused vs {r_u:.4f} unfused")
        assert same >= 0.98, (K, beam, same)
        assert abs(r_f - r_u) <= 0.002, (K, beam, r_f, r_u)
