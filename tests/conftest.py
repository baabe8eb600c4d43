"""Shared fixtures.  GPU tests are marked `gpu`; everything else runs on the
CPU (oracle, host logic, C-ABI symbol table)."""
from __future__ import annotations

import functools
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device)")


@functools.lru_cache(maxsize=None)
def small_index(n=3000, nq=24, dim=128, comps=16, degree=32, kind="int", use_ip=False, config=1):
    """(codebook, queries, base) built on the CPU, cached per process."""
    from flashgann_amd import builder, datasets
    from flashgann_amd.codebook import padded_dim_for
    if kind == "int":
        base, q = datasets.integer_mixture(n, nq, dim, comps, config=config)
    elif kind == "unit":
        base, q = datasets.normalized_mixture(n, nq, dim, comps, config=3)
    elif kind == "box":
        base, q = datasets.unit_box_mixture(n, nq, dim, comps, config=4)
    elif kind == "aniso":
        base, q = datasets.anisotropic_unit_mixture(n, nq, dim, comps, config=5)
    else:
        raise ValueError(kind)
    signs = datasets.signs_for(padded_dim_for(dim), config)
    cb = builder.build_codebook(base, degree, signs, use_ip=use_ip, device="cpu")
    return cb, q, base


@pytest.fixture(params=["one-wave", "team"])
def search_form(request, monkeypatch):
    """Runs a GPU test once with each form of the search kernel: one wave
    per query, and the team form (two waves per query) that small launches
    use.  FLASHGANN_TEAM is read at every launch."""
    monkeypatch.setenv("FLASHGANN_TEAM", "0" if request.param == "one-wave" else "1")
    return request.param


@pytest.fixture(scope="session")
def gpu_available():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return True
