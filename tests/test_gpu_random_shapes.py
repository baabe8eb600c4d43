"""GPU parity over seeded random search shapes: dimension (33-1536, so
every shape class: fixed and runtime geometry, padded dimensions 64-2048),
degree (1-96, one to three tiles), K, beam (1-1024, both merge families),
metric, data family, kernel form (one wave / team) and schedule (one launch /
two).  Each case builds a small codebook on the CPU and requires the
kernel's ids and per-query work counters to equal the CPU oracle's."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import small_index

pytestmark = pytest.mark.gpu


def _case(seed):
    rng = np.random.default_rng(0xC0FFEE + seed)
    dim = int(rng.choice([33, 40, 64, 96, 100, 128, 200, 256, 512, 960, 1536]))
    degree = int(rng.choice([1, 3, 8, 16, 24, 32, 40, 48, 64, 96]))
    beam = int(rng.choice([1, 7, 16, 33, 64, 100, 128, 129, 200, 256, 300, 512, 777, 1024]))
    if degree > 64:
        beam = min(beam, 2048 - 512 * ((degree + 31) // 32))
    K = int(rng.integers(1, 150))
    kind = str(rng.choice(["int", "unit", "box"]))
    ip = bool(rng.random() < 0.4) and kind != "int"
    n = 1200 if dim >= 512 else 2500
    return dict(dim=dim, degree=degree, beam=beam, K=K, kind=kind, ip=ip, n=n,
                team=bool(rng.random() < 0.5), slice=bool(rng.random() < 0.5), runtime=bool(rng.random() < 0.3))


@pytest.mark.parametrize("seed", range(48))
def test_random_shape_matches_oracle(gpu_available, monkeypatch, seed):
    from flashgann_amd import Index
    from oracle import oracle as O
    c = _case(seed)
    print(f"random shape {seed}: {c}", flush=True)
    monkeypatch.setenv("FLASHGANN_TEAM", "1" if c["team"] else "0")
    monkeypatch.setenv("FLASHGANN_SLICE", "1" if c["slice"] else "0")
    if c["runtime"]:
        monkeypatch.setenv("FG_FORCE_RUNTIME_GEOMETRY", "1")
    cb, q, _ = small_index(n=c["n"], nq=20, dim=c["dim"], comps=12, degree=c["degree"], kind=c["kind"],
                           use_ip=c["ip"], config=3 if c["kind"] == "unit" else 4 if c["kind"] == "box" else 1)
    ix = Index.from_codebook(cb, metric=1 if c["ip"] else 0)
    ids, _, cnt = ix.search(q, c["K"], c["beam"], counters=True)
    ix.close()
    rids, rcnt = O.OracleIndex.from_codebook(cb, use_ip=c["ip"]).search(q, c["K"], c["beam"])
    assert np.array_equal(ids, rids)
    assert np.array_equal(cnt, rcnt.view(np.uint32).reshape(-1, 6))
