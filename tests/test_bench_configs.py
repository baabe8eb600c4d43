"""Host-side checks of the benchmark's configuration table and generators
(no GPU): every BASELINE configuration names a generator that exists and
yields the stated shape, and the generators are deterministic."""
from __future__ import annotations

import numpy as np
import pytest

import bench
from flashgann_amd import datasets
from flashgann_amd.codebook import padded_dim_for


@pytest.mark.parametrize("name", sorted(bench.CONFIGS))
def test_config_generator_shapes(name):
    c = bench.CONFIGS[name]
    base, q = getattr(datasets, c["gen"])(300, 7, c["dim"], min(c["components"], 16), config=c["cfg"])
    assert base.shape == (300, c["dim"]) and q.shape == (7, c["dim"])
    assert base.dtype == np.float32 and q.dtype == np.float32
    assert np.isfinite(base).all() and np.isfinite(q).all()
    assert padded_dim_for(c["dim"]) <= 2048
    beams = [int(b) for b in c["beams"].split(",")]
    assert all(1 <= b <= 1024 for b in beams)


def test_generators_are_deterministic_and_distinct():
    a1, q1 = datasets.anisotropic_unit_mixture(200, 5, 64, 8)
    a2, q2 = datasets.anisotropic_unit_mixture(200, 5, 64, 8)
    assert np.array_equal(a1, a2) and np.array_equal(q1, q2)
    assert np.allclose(np.linalg.norm(a1, axis=1), 1.0, atol=1e-5)
    b1, _ = datasets.integer_mixture(200, 5, 64, 8, config=1)
    b2, _ = datasets.integer_mixture(200, 5, 64, 8, config=2)
    assert not np.array_equal(b1, b2)
    assert np.array_equal(b1, np.rint(b1)) and (b1 >= 0).all()


def test_headline_config_is_c2():
    c = bench.CONFIGS["c2"]
    assert (c["n"], c["nq"], c["dim"], c["degree"], c["K"]) == (1_000_000, 10_000, 128, 32, 100)
