"""Codebook builder: graph shape, the per-edge encoding against its
definition, and the quality of the resulting RaBitQ estimates."""
from __future__ import annotations

import ctypes as C

import numpy as np

from conftest import small_index
from oracle import oracle as O


def test_graph_shape():
    cb, _, base = small_index()
    nb = cb.neighbors().astype(np.int64)
    n, deg = nb.shape
    assert deg == cb.layout.degree
    assert (nb < n).all()
    assert not (nb == np.arange(n)[:, None]).any()
    for row in nb[:500]:
        assert len(set(row.tolist())) == deg
    d = ((base[nb[:200]] - base[:200, None, :]) ** 2).sum(-1)
    assert (np.diff(d, axis=1) >= 0).all()                       # sorted by distance


def test_encoding_matches_definition():
    from flashgann_amd.builder import hadamard_rotation
    from flashgann_amd.codebook import unpack_codes
    cb, _, base = small_index()
    lay = cb.layout
    P = hadamard_rotation(cb.signs, "cpu").numpy()
    nb = cb.neighbors().astype(np.int64)
    codes = cb.codes()
    fac = cb.factors()
    rng = np.random.default_rng(0)
    for u in rng.integers(0, cb.npoints, 25):
        for j in rng.integers(0, lay.degree, 4):
            v = nb[u, j]
            r = np.zeros(lay.padded_dim)
            r[: lay.dim] = base[v].astype(np.float64) - base[u]
            y = P @ r
            bits = (y > 0).astype(np.uint8)
            assert np.array_equal(unpack_codes(codes[u, j]), bits)
            s = 2.0 * bits - 1.0
            pc = P @ np.pad(base[u].astype(np.float64), (0, lay.padded_dim - lay.dim))
            f = -2.0 * (r @ r) / np.abs(y).sum()
            assert fac[u, 1, j] == np.float32(f)
            assert fac[u, 2, j] == np.float32(f * s.sum())
            assert fac[u, 0, j] == np.float32(r @ r - f * (s @ pc))


def test_estimates_track_exact_distances():
    """RaBitQ estimates of d(q, v) via a parent u: small relative error and
    close to unbiased (the property the prune relies on)."""
    cb, q, base = small_index()
    lay = cb.layout
    L = O.lib()
    nb = cb.neighbors().astype(np.int64)
    codes = cb.codes()
    fac = cb.factors()
    rng = np.random.default_rng(1)
    rel = []
    for qi in range(8):
        qf = O.query_prepare(q[qi], cb.signs, lay.dim, lay.padded_dim)
        for u in rng.integers(0, cb.npoints, 30):
            pd = float(((q[qi].astype(np.float64) - base[u]) ** 2).sum())
            for j in range(lay.degree):
                v = nb[u, j]
                code = np.ascontiguousarray(codes[u, j])
                est = L.fgo_estimate_seq(C.byref(qf), O.ptr(code, C.c_uint8), float(fac[u, 0, j]),
                                         float(fac[u, 1, j]), float(fac[u, 2, j]), pd, lay.padded_dim)
                ex = float(((q[qi].astype(np.float64) - base[v]) ** 2).sum())
                rel.append((est - ex) / ex)
    rel = np.array(rel)
    assert abs(np.median(rel)) < 0.05
    assert np.percentile(np.abs(rel), 90) < 0.25


def test_truncated_codebook_rejected(tmp_path):
    import pytest
    from flashgann_amd import _lib
    from flashgann_amd.codebook import read_codebook, write_codebook
    cb, _, _ = small_index()
    p = str(tmp_path / "cb.index")
    write_codebook(p, cb.rows[:100], cb.signs, cb.entry)
    with open(p, "r+b") as f:
        f.truncate(4 + 100 * cb.layout.row_offset * 4)
    with pytest.raises(ValueError):
        read_codebook(p, 100, cb.layout.dim, cb.layout.degree)
    h = C.c_void_p()
    rc = _lib.lib().fg_index_load(p.encode(), 100, cb.layout.dim, cb.layout.degree, 0, C.byref(h))
    assert rc == _lib.FG_EIO


def test_graph_blocked_distances_identical():
    """The neighbour lists do not depend on the row blocking of the final
    distance pass (blocks of 7 rows against one block)."""
    import torch
    from flashgann_amd import builder, datasets
    base, _ = datasets.unit_box_mixture(400, 1, 40, 4)
    x = torch.as_tensor(base)
    a = builder.build_graph(x, 8)
    b = builder.build_graph(x, 8, dist_block_elems=7 * 8 * 40)
    assert torch.equal(a, b)


def test_ground_truth_inner_product_brute_force():
    """Exact top-k by inner product (ties by id) against numpy brute force."""
    from flashgann_amd import builder, datasets
    base, q = datasets.normalized_mixture(600, 9, 24, 6)
    gt = builder.ground_truth(base, q, 10, use_ip=True)
    s = q.astype(np.float64) @ base.astype(np.float64).T
    for i in range(q.shape[0]):
        order = sorted(range(base.shape[0]), key=lambda j: (-s[i, j], j))[:10]
        assert set(gt[i]) == set(order)
        assert np.all(np.diff(-s[i, gt[i]]) >= -1e-6)


def test_build_index_cli_round_trip(tmp_path):
    """python -m flashgann_amd.build_index writes a codebook and a ground truth
    from .fvecs files; the codebook reads back in the reference's layout and
    the oracle's search over it reaches the expected recall against that
    ground truth."""
    import subprocess
    import sys
    from flashgann_amd import datasets
    from flashgann_amd.codebook import read_codebook, read_ivecs, write_fvecs
    from flashgann_amd.metrics import compute_recall
    base, q = datasets.integer_mixture(1500, 16, 64, 8, config=1)
    bp, qp = str(tmp_path / "base.fvecs"), str(tmp_path / "query.fvecs")
    write_fvecs(bp, base)
    write_fvecs(qp, q)
    ip, gp = str(tmp_path / "cb.index"), str(tmp_path / "gt.ivecs")
    root = str(__import__("pathlib").Path(__file__).resolve().parents[1])
    for cmd in (["index", bp, ip, "--degree", "16", "--device", "cpu"],
                ["gt", bp, qp, gp, "--k", "10", "--device", "cpu"]):
        r = subprocess.run([sys.executable, "-m", "flashgann_amd.build_index"] + cmd, cwd=root,
                           capture_output=True, text=True, timeout=300)
        assert r.returncode == 0, r.stderr
    cb = read_codebook(ip, 1500, 64, 16)
    gt = read_ivecs(gp)
    assert gt.shape == (16, 10)
    out, _ = O.OracleIndex.from_codebook(cb).search(q, 10, 64)
    assert compute_recall(out, gt, 10) >= 0.9


def test_partitioned_knn_reduces_to_exact_knn():
    """Searching every cell (probes == cells) is the exact k-NN search:
    identical ids and distances to knn() on integer data, where every
    distance is exact."""
    import torch
    from flashgann_amd import builder, datasets
    base, _ = datasets.integer_mixture(4000, 1, 64, 8, config=1)
    x = torch.as_tensor(base)
    a_ids, a_d = builder.knn(x, 24)
    b_ids, b_d = builder.knn_partitioned(x, 24, cells=6, probes=6)
    assert torch.equal(a_ids, b_ids) and torch.equal(a_d, b_d)


def test_partitioned_knn_small_set_is_one_cell():
    """Under 2,500 points the partition is one cell, searched exactly."""
    import torch
    from flashgann_amd import builder, datasets
    base, _ = datasets.integer_mixture(1000, 1, 64, 4, config=1)
    x = torch.as_tensor(base)
    assert torch.equal(builder.knn(x, 16)[0], builder.knn_partitioned(x, 16)[0])


def test_partitioned_knn_never_returns_the_point_itself():
    """Cells smaller than k + 1 points: a point's own row is never one of
    its neighbours; slots without a candidate are -1 at distance inf."""
    import torch
    from flashgann_amd import builder, datasets
    base, _ = datasets.integer_mixture(60, 1, 16, 4, config=1)
    x = torch.as_tensor(base)
    ids, d = builder.knn_partitioned(x, 40, cells=6, probes=2)
    own = torch.arange(60)[:, None]
    assert not (ids == own).any()
    assert ((ids >= 0) | torch.isinf(d)).all()
    assert torch.isinf(d[ids < 0]).all()
    g = builder.build_graph(x, 16, knn_method="partitioned")
    assert not (g == own).any()


def test_partitioned_knn_overlap_on_c5_mixture():
    """Two probed cells of eight find nearly all exact neighbours of the C5
    generator's well-separated anisotropic components."""
    import torch
    from flashgann_amd import builder, datasets
    base, _ = datasets.anisotropic_unit_mixture(12000, 1, 128, 12)
    x = torch.as_tensor(base)
    a, _ = builder.knn(x, 64)
    b, _ = builder.knn_partitioned(x, 64, probes=2)
    a, b = a.numpy(), b.numpy()
    overlap = np.mean([len(np.intersect1d(a[i], b[i])) / 64 for i in range(0, 12000, 7)])
    assert overlap > 0.99, overlap
    g = builder.build_graph(x, 32, knn_method="partitioned")
    assert g.shape == (12000, 32) and (g >= 0).all()


def test_device_generator_shapes_and_determinism():
    """The device form of the C5 generator (here on the CPU device): unit
    rows, the requested shapes, the same draws for the same seed."""
    from flashgann_amd import datasets
    a, qa = datasets.anisotropic_unit_mixture_device(3000, 40, 96, 16, device="cpu", chunk=1000)
    b, qb = datasets.anisotropic_unit_mixture_device(3000, 40, 96, 16, device="cpu", chunk=700)
    assert a.shape == (3000, 96) and qa.shape == (40, 96)
    assert np.allclose(a.norm(dim=1).numpy(), 1.0, atol=1e-5)
    assert (a == b).all() and (qa == qb).all()


def test_ground_truth_recheck():
    """check_ground_truth accepts the exact ground truth (ties included) and
    flags rows whose sets hold points beyond the true k-th distance."""
    from flashgann_amd import builder, datasets
    base, q = datasets.integer_mixture(3000, 40, 64, 8, config=2)
    for ip in (False, True):
        gt = builder.ground_truth(base, q, 20, use_ip=ip)
        assert builder.check_ground_truth(base, q, gt, sample=40, use_ip=ip) == 0
        bad = gt.copy()
        bad[::5] = gt[::5][:, ::-1] + 0  # same sets: still fine
        assert builder.check_ground_truth(base, q, bad, sample=40, use_ip=ip) == 0
        # the 20 worst points: largest distance, or smallest inner product
        score = ((base[None] - q[:, None]) ** 2).sum(-1) if not ip else -(q @ base.T)
        far = np.argsort(score, axis=1)[:, -20:]
        bad[::4] = far[::4]
        assert builder.check_ground_truth(base, q, bad, sample=40, use_ip=ip) == 10


def test_connected_graph_keeps_rng_edges_and_reaches_every_node():
    """The connect=True recipe on a 64-component integer mixture, where the
    bare RNG-pruned k-NN graph reaches few nodes from the entry point: every
    node becomes reachable (BFS over the out-edges), every RNG-kept edge of
    every node is still in its list, the links added are few (one or a few
    per component), lists stay sorted by distance, and the oracle's recall on
    the repaired graph far exceeds the bare graph's (one link per component
    makes each component reachable, not easy to reach: at beam 64 the search
    finds the query's component about half the time)."""
    import torch

    from flashgann_amd import builder, datasets
    base, q = datasets.integer_mixture(12000, 100, 128, 64, config=1)
    x = torch.as_tensor(base)
    n = base.shape[0]
    entry = builder.entry_point(x)
    bare = builder.build_graph(x, 32, random_links=0, fill_random=False)
    st = {}
    g = builder.build_graph(x, 32, random_links=0, fill_random=False, connect=True, stats=st)
    reach = lambda gr: int(builder._reach(gr, torch.zeros(n, dtype=torch.bool), torch.tensor([entry])))
    assert reach(bare) < n // 4
    assert reach(g) == n
    assert 0 < st["connect_links"] <= 3 * 64
    # rows differ from the bare graph only by the links
    assert int((bare != g).any(1).sum()) <= st["connect_links"]
    # every RNG-kept candidate is still a neighbour
    cand, cd = builder.knn(x, 64)
    keep = builder._prune(cand, cd, x, 32)
    for i in range(0, n, 7):
        kept = set(cand[i][keep[i]].tolist())
        assert kept <= set(g[i].tolist()), i
    gn = g.numpy()
    d = ((base[gn[:300]] - base[:300, None, :]) ** 2).sum(-1)
    assert (np.diff(d, axis=1) >= 0).all()
    sig = datasets.signs_for(128, 1)
    gt = builder.ground_truth(base, q, 10)
    rec = []
    for gr in (bare, g):
        cb = builder.codebook_from_graph(base, gr, sig)
        ids, _ = O.OracleIndex.from_codebook(cb).search(q, 10, 64)
        rec.append(O.recall(ids, gt, 10))
    assert rec[0] < 0.1 and rec[1] > 0.4 and rec[1] > 5 * rec[0], rec
