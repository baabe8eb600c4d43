"""Parity of the HIP search kernel with the CPU oracle (ids and per-query
work counters must be identical: integer data makes every distance exact,
and the oracle fixes the same tie and race resolution)."""
from __future__ import annotations

import os

import numpy as np
import pytest

from conftest import small_index

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("search_form")]


def _run(cb, q, K, beam, metric=0, entry=None):
    from flashgann_amd import Index
    from oracle import oracle as O
    ix = Index.from_codebook(cb, metric=metric, entry=entry)
    ids, st, cnt = ix.search(q, K, beam, counters=True)
    oix = O.OracleIndex.from_codebook(cb, use_ip=bool(metric), entry=ix.entry)
    ref_ids, ref_cnt = oix.search(q, K, beam)
    ref_cnt = ref_cnt.view(np.uint32).reshape(-1, 6)
    ix.close()
    return ids, cnt, ref_ids, ref_cnt


def _assert_equal(ids, cnt, ref_ids, ref_cnt, label):
    bad = np.nonzero((ids != ref_ids).any(1) | (cnt != ref_cnt).any(1))[0]
    assert bad.size == 0, (f"{label}: {bad.size} queries differ; first {bad[:5]}; "
                           f"gpu cnt {cnt[bad[0]]} ref cnt {ref_cnt[bad[0]]}")


@pytest.mark.parametrize("K,beam", [(10, 16), (10, 64), (100, 100), (100, 128), (100, 256),
                                    (100, 384), (100, 1000), (10, 1), (64, 32), (100, 1024),
                                    (100, 257), (100, 300), (100, 640), (100, 896), (50, 777)])
def test_search_int128_beams(gpu_available, K, beam):
    cb, q, _ = small_index()
    ids, cnt, rids, rcnt = _run(cb, q, K, beam)
    _assert_equal(ids, cnt, rids, rcnt, f"K={K} beam={beam}")


@pytest.mark.parametrize("degree", [8, 16, 48])
def test_search_degrees(gpu_available, degree):
    cb, q, _ = small_index(n=2500, degree=degree)
    ids, cnt, rids, rcnt = _run(cb, q, 100, 128)
    _assert_equal(ids, cnt, rids, rcnt, f"degree={degree}")


def test_search_float_unit_vectors(gpu_available):
    cb, q, _ = small_index(n=3000, dim=96, comps=32, kind="unit")
    ids, cnt, rids, rcnt = _run(cb, q, 10, 64)
    _assert_equal(ids, cnt, rids, rcnt, "unit96")


@pytest.mark.parametrize("degree,K,beam", [(16, 10, 64), (16, 100, 256), (16, 100, 512), (32, 100, 256),
                                           (32, 100, 512)])
def test_search_c3_shapes(gpu_available, degree, K, beam):
    """C3's shapes on float data against the oracle: 96-d unit vectors
    (padded 128) with degree-16 and degree-32 graphs, each through its
    fixed-geometry kernel, at K = 10 and K = 100 and merge-path beams."""
    cb, q, _ = small_index(n=4000, nq=32, dim=96, comps=32, degree=degree, kind="unit")
    ids, cnt, rids, rcnt = _run(cb, q, K, beam)
    _assert_equal(ids, cnt, rids, rcnt, f"unit96 degree {degree} K={K} beam={beam}")


def test_search_inner_product(gpu_available):
    cb, q, _ = small_index(n=2000, dim=96, comps=16, kind="unit", use_ip=True)
    ids, cnt, rids, rcnt = _run(cb, q, 10, 64, metric=1)
    _assert_equal(ids, cnt, rids, rcnt, "ip96")


@pytest.mark.parametrize("dim,kind,K,beam", [(128, "unit", 100, 256), (128, "unit", 100, 512), (960, "box", 100, 384)])
def test_search_inner_product_beams(gpu_available, dim, kind, K, beam):
    """Inner product on the headline's fixed 128-d kernel (both merge builds)
    and on the generic geometry at a beam over 256."""
    cb, q, _ = small_index(n=2000 if dim == 128 else 1500, nq=8, dim=dim, comps=16, kind=kind, use_ip=True)
    ids, cnt, rids, rcnt = _run(cb, q, K, beam, metric=1)
    _assert_equal(ids, cnt, rids, rcnt, f"ip{dim} beam {beam}")


def test_search_dim960(gpu_available):
    cb, q, _ = small_index(n=1500, nq=8, dim=960, comps=8, kind="box")
    ids, cnt, rids, rcnt = _run(cb, q, 100, 128)
    _assert_equal(ids, cnt, rids, rcnt, "box960")


def test_search_dim1536(gpu_available):
    """C5's row shape: 1536-d unit vectors, rotation padded to 2048 (the
    largest padded dimension the kernel takes)."""
    cb, q, _ = small_index(n=1200, nq=8, dim=1536, comps=8, kind="aniso")
    ids, cnt, rids, rcnt = _run(cb, q, 100, 128)
    _assert_equal(ids, cnt, rids, rcnt, "aniso1536")
    ids, cnt, rids, rcnt = _run(cb, q, 10, 32)
    _assert_equal(ids, cnt, rids, rcnt, "aniso1536 beam 32")


@pytest.mark.parametrize("dim,kind,n,K,beam", [(960, "box", 1500, 100, 384), (960, "box", 1500, 100, 640),
                                               (1536, "aniso", 1200, 100, 768), (300, "unit", 1200, 10, 1000)])
def test_search_generic_large_beams(gpu_available, dim, kind, n, K, beam):
    """The generic geometry's beams over 256 (its merge over segment-strided
    lanes and the wide pick), as the C4 and C5 operating points run them."""
    cb, q, _ = small_index(n=n, nq=8, dim=dim, comps=8, kind=kind)
    ids, cnt, rids, rcnt = _run(cb, q, K, beam)
    _assert_equal(ids, cnt, rids, rcnt, f"{kind}{dim} beam {beam}")


@pytest.mark.parametrize("bad", ["inf", "nan"])
def test_search_non_finite_distances(gpu_available, bad):
    """One row in twenty gets a vector that overflows (1e30: exact distances
    are inf) or is NaN, after the graph and codes were built from the real
    data, so estimates stay finite while such children's exact distances
    enter the candidate buffer and the beam as non-finite keys.  The merges
    then take the reference's bisection and full candidate network, and ids
    and counters must still equal the oracle's."""
    import dataclasses
    cb, q, _ = small_index()
    rows = cb.rows.copy()
    rng = np.random.default_rng(7)
    pick = rng.choice(cb.npoints, cb.npoints // 20, replace=False)
    pick = pick[pick != cb.entry]
    rows[pick, :cb.layout.dim] = np.float32(1e30) if bad == "inf" else np.float32(np.nan)
    cb2 = dataclasses.replace(cb, rows=rows)
    for beam in (64, 256, 512):
        ids, cnt, rids, rcnt = _run(cb2, q, 100, beam)
        _assert_equal(ids, cnt, rids, rcnt, f"{bad} beam {beam}")


def test_empty_batch(gpu_available):
    """nq = 0 is a no-op through both entry points (no launch, outputs untouched)."""
    import torch
    from flashgann_amd import Index
    cb, q, _ = small_index()
    ix = Index.from_codebook(cb)
    ids, st, cnt = ix.search(q[:0], 10, 64, counters=True)
    assert ids.shape == (0, 10) and cnt.shape == (0, 6)
    res = torch.full((4, 10), 7, dtype=torch.int32, device="cuda")
    dq = torch.as_tensor(q[:4], device="cuda")
    ix.search_device(dq.data_ptr(), 0, 10, 64, res.data_ptr())
    torch.cuda.synchronize()
    assert (res.cpu() == 7).all()
    ix.close()


def test_oversized_batch_rejected(gpu_available):
    """nq above 2^31 - 1 is FG_EINVAL before any launch (one workgroup per
    query; the grid size is a signed 32-bit count), on every search entry."""
    import ctypes as C
    import torch
    from flashgann_amd import Index, _lib
    cb, q, _ = small_index()
    ix = Index.from_codebook(cb)
    res = torch.full((4, 10), 7, dtype=torch.int32, device="cuda")
    dq = torch.as_tensor(q[:4], device="cuda")
    L = _lib.lib()
    qp, rp = C.c_void_p(dq.data_ptr()), C.c_void_p(res.data_ptr())
    assert L.fg_search_device(ix._h, qp, 2 ** 31, 10, 64, rp, None, None) == -1
    assert b"2^31" in L.fg_last_error()
    assert L.fg_search_stream(ix._h, qp, 2 ** 31, 10, 64, rp, 2 ** 31, 2, None) == -1
    torch.cuda.synchronize()
    assert (res.cpu() == 7).all()
    ix.close()


def test_search_entry_auto(gpu_available):
    from flashgann_amd import Index
    from oracle import oracle as O
    cb, q, base = small_index()
    ix = Index.from_codebook(cb, entry=0xFFFFFFFF)
    assert ix.entry == O.lib().fgo_entry_point(O.ptr(cb.rows, O.C.c_float), cb.npoints, 128,
                                               cb.layout.row_offset, 0)
    ix.close()
    ids, cnt, rids, rcnt = _run(cb, q, 10, 64, entry=0xFFFFFFFF)
    _assert_equal(ids, cnt, rids, rcnt, "entry auto")


@pytest.mark.parametrize("dim,degree,kind", [(128, 32, "int"), (96, 16, "unit"), (100, 32, "int"), (64, 32, "int")])
def test_timed_instantiation_matches_counting_one(gpu_available, dim, degree, kind):
    """The kernel built without work counters (the one bench.py times) returns
    the same ids as the counting build the parity tests compare."""
    from flashgann_amd import Index
    cb, q, _ = small_index(n=2500, dim=dim, degree=degree, kind=kind, comps=16)
    ix = Index.from_codebook(cb)
    for K, beam in [(10, 64), (100, 256)]:
        a, _, _ = ix.search(q, K, beam, counters=True)
        b, _, _ = ix.search(q, K, beam, counters=False)
        assert np.array_equal(a, b), (dim, degree, K, beam)
    ix.close()


def _degree_case(degree):
    """Degree 4 (stage-II keep rate rho2 = 0, the reference's deg <= 4 rule)
    and degree 64 (the largest the kernel takes: two 32-neighbour tiles per
    parent)."""
    cb, q, _ = small_index(n=1500, nq=16, degree=degree)
    ids, cnt, rids, rcnt = _run(cb, q, 100, 128)
    _assert_equal(ids, cnt, rids, rcnt, f"degree={degree}")


def test_search_degree_4(gpu_available):
    _degree_case(4)


def test_search_degree_64(gpu_available):
    _degree_case(64)


@pytest.mark.parametrize("degree,beam", [(80, 256), (96, 500)])
def test_search_degree_above_64(gpu_available, degree, beam):
    """Three 32-neighbour tiles per parent (three stage-II rounds per
    iteration, compaction overflow reachable), at beams where the reference's
    2048-slot visited table cannot fill."""
    cb, q, _ = small_index(n=1500, nq=12, degree=degree)
    ids, cnt, rids, rcnt = _run(cb, q, 100, beam)
    _assert_equal(ids, cnt, rids, rcnt, f"degree={degree} beam={beam}")


@pytest.mark.parametrize("degree,beam", [(96, 600), (128, 16)])
def test_search_degree_table_overflow_rejected(gpu_available, degree, beam):
    """Where the reference's visited table could fill (beam + 512 x tiles
    keys above its 2048 slots), the search is refused before any launch."""
    from flashgann_amd import FlashGannError, Index, _lib
    cb, q, _ = small_index(n=600, nq=4, degree=degree)
    ix = Index.from_codebook(cb)
    with pytest.raises(FlashGannError) as e:
        ix.search(q, 10, beam)
    ix.close()
    assert e.value.code == _lib.FG_EINVAL and "slot table" in str(e.value)


def test_search_inner_product_generic(gpu_available):
    """Inner product on the generic geometry (300-d: padded dimension 512)."""
    cb, q, _ = small_index(n=1200, nq=8, dim=300, comps=8, kind="unit", use_ip=True)
    ids, cnt, rids, rcnt = _run(cb, q, 10, 64, metric=1)
    _assert_equal(ids, cnt, rids, rcnt, "ip300")


_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
_CLIS = {
    # this build's CLI (main.cu's interface on qg_host.hpp)
    "gpu_flashgann": os.path.join(_ROOT, "flashgann_amd", "bin", "gpu_flashgann"),
    # the reference's own main.cu, unchanged, linked with this build's
    # replacement of gpu_search_adaptive.cu (built by `make -C oracle ref`
    # where the reference tree exists; the binary travels with the tree)
    "reference_main": os.path.join(_ROOT, "oracle", "_ref", "gpu_flashgann_ref"),
}


@pytest.mark.parametrize("cli_name", sorted(_CLIS))
def test_cli_end_to_end(gpu_available, tmp_path, cli_name):
    """A CLI with main.cu's interface on files written in the reference's
    formats: printed recall equals the oracle's recall of the same search,
    and the CSV row has the reference's columns."""
    import re
    import subprocess
    from flashgann_amd import builder
    from flashgann_amd.codebook import write_fvecs, write_ivecs
    from flashgann_amd.metrics import compute_recall
    from oracle import oracle as O
    cb, q, base = small_index()
    gt = builder.ground_truth(base, q, 10)
    paths = {k: str(tmp_path / k) for k in ("base.fvecs", "query.fvecs", "gt.ivecs", "cb.index", "out.csv")}
    write_fvecs(paths["base.fvecs"], base)
    write_fvecs(paths["query.fvecs"], q)
    write_ivecs(paths["gt.ivecs"], gt)
    cb.save(paths["cb.index"])
    cli = _CLIS[cli_name]
    if not os.path.exists(cli):
        pytest.skip(f"{cli} not built (the reference tree was absent at build time)")
    r = subprocess.run([cli, paths["base.fvecs"], paths["query.fvecs"], paths["gt.ivecs"], paths["cb.index"],
                        "10", "64", "32", "-csv", paths["out.csv"]], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    m = re.search(r"Recall@10: ([0-9.]+)", r.stdout)
    assert m, r.stdout
    ref_ids, _ = O.OracleIndex.from_codebook(cb).search(q, 10, 64)
    assert abs(float(m.group(1)) - 100.0 * compute_recall(ref_ids, gt, 10)) < 1e-3
    rows = open(paths["out.csv"]).read().strip().splitlines()
    assert rows[0] == "TopK,Beam_size,Runtime,Latency,Throughput,Recall"
    assert rows[1].split(",")[:2] == ["10", "64"]


@pytest.mark.parametrize("batch,nstreams", [(5, 1), (5, 2), (7, 3), (24, 2), (100, 4)])
def test_search_stream_matches_single_launch(gpu_available, batch, nstreams):
    """fg_search_stream (batches on internal streams) returns, in query order,
    the ids of one fg_search_device launch over the same queries, and the
    caller's stream sees them complete."""
    import torch
    from flashgann_amd import Index
    cb, q, _ = small_index()
    ix = Index.from_codebook(cb)
    dq = torch.as_tensor(q, device="cuda")
    ref = torch.zeros((q.shape[0], 100), dtype=torch.int32, device="cuda")
    out = torch.full((q.shape[0], 100), -1, dtype=torch.int32, device="cuda")
    s = torch.cuda.current_stream()
    ix.search_device(dq.data_ptr(), q.shape[0], 100, 128, ref.data_ptr(), 0, s.cuda_stream)
    ix.search_stream(dq.data_ptr(), q.shape[0], 100, 128, out.data_ptr(), batch, nstreams, s.cuda_stream)
    got = out.cpu()  # ordered after the batches on the caller's stream
    assert torch.equal(got, ref.cpu())
    ix.close()
    from oracle import oracle as O
    oids, _ = O.OracleIndex.from_codebook(cb).search(q, 100, 128)
    assert np.array_equal(got.numpy().view(np.uint32), oids)


@pytest.mark.parametrize("dim,degree,kind", [(128, 32, "int"), (96, 32, "unit"), (96, 16, "unit")])
def test_fixed_geometry_matches_runtime_geometry(gpu_available, dim, degree, kind, monkeypatch):
    """The kernels specialised for the benchmark shapes (32-bit row offsets,
    compile-time field offsets) return the same ids and work counters as the
    general kernels, which codebooks of 4 GiB and more use (forced here with
    FG_FORCE_RUNTIME_GEOMETRY)."""
    from flashgann_amd import Index
    cb, q, _ = small_index(n=2500, dim=dim, degree=degree, kind=kind, comps=16)
    fixed = Index.from_codebook(cb)
    monkeypatch.setenv("FG_FORCE_RUNTIME_GEOMETRY", "1")
    general = Index.from_codebook(cb)
    monkeypatch.delenv("FG_FORCE_RUNTIME_GEOMETRY")
    for K, beam in [(10, 64), (100, 256)]:
        a, _, ca = fixed.search(q, K, beam, counters=True)
        b, _, cb_ = general.search(q, K, beam, counters=True)
        assert np.array_equal(a, b) and np.array_equal(ca, cb_), (dim, degree, K, beam)
    fixed.close()
    general.close()


@pytest.mark.parametrize("dim,degree", [(33, 32), (128, 1), (128, 2), (40, 8)])
def test_search_shape_limits(gpu_available, dim, degree):
    """The smallest dimension the layout allows (33: padded 64, two code words
    per edge) and one- and two-neighbour graphs (a candidate buffer of 8 / 16,
    stage-II keep rate 0)."""
    cb, q, _ = small_index(n=800, nq=12, dim=dim, degree=degree, comps=8)
    ids, cnt, rids, rcnt = _run(cb, q, 10, 64)
    _assert_equal(ids, cnt, rids, rcnt, f"dim={dim} degree={degree}")


def test_search_waves_reports_the_form(gpu_available, monkeypatch):
    """fg_search_waves: 2 (the team form) for a batch too small to fill the
    device, 1 for one that fills it, and the environment override wins."""
    from flashgann_amd import Index
    cb, q, _ = small_index()
    ix = Index.from_codebook(cb)
    monkeypatch.delenv("FLASHGANN_TEAM", raising=False)
    assert ix.search_waves(16, 10, 64) == 2
    assert ix.search_waves(100000, 10, 64) == 1
    monkeypatch.setenv("FLASHGANN_TEAM", "0")
    assert ix.search_waves(16, 10, 64) == 1
    monkeypatch.setenv("FLASHGANN_TEAM", "1")
    assert ix.search_waves(100000, 10, 64) == 2
    ix.close()


@pytest.mark.parametrize("dim,degree,kind,K,beam,ip", [(128, 32, "int", 100, 256, False), (128, 32, "int", 10, 64, False),
                                                       (96, 16, "unit", 100, 200, False), (96, 32, "unit", 10, 32, False),
                                                       (40, 8, "int", 10, 128, False), (128, 32, "int", 100, 512, False),
                                                       (96, 16, "unit", 100, 384, False), (128, 32, "int", 100, 1000, False),
                                                       (960, 32, "box", 100, 384, False), (96, 32, "unit", 100, 256, True),
                                                       (128, 32, "unit", 100, 512, True), (960, 32, "box", 100, 384, True)])
def test_two_launch_search_equals_one_launch(gpu_available, monkeypatch, dim, degree, kind, K, beam, ip):
    """The two-launch search (every query suspended at the top of iteration
    15 with its beam, candidates, controller, counters and prepared query
    kept in HBM, then resumed in an order of its own) returns the ids and
    work counters of the one-launch search and of the oracle, with and
    without counters, for both metrics (inner-product distances are
    negative: the ordering key is the signed best distance)."""
    from flashgann_amd import Index
    from oracle import oracle as O
    cb, q, _ = small_index(n=3000, nq=300, dim=dim, degree=degree, kind=kind, comps=16, use_ip=ip)
    ix = Index.from_codebook(cb, metric=1 if ip else 0)
    monkeypatch.setenv("FLASHGANN_TEAM", "0")
    monkeypatch.setenv("FLASHGANN_SLICE", "0")
    ids1, _, cnt1 = ix.search(q, K, beam, counters=True)
    monkeypatch.setenv("FLASHGANN_SLICE", "1")
    ids2, _, cnt2 = ix.search(q, K, beam, counters=True)
    ids3, _, _ = ix.search(q, K, beam)
    ix.close()
    assert (cnt1[:, 0] > 15).any()  # some queries are suspended and resumed
    assert np.array_equal(ids2, ids1) and np.array_equal(cnt2, cnt1)
    assert np.array_equal(ids3, ids1)
    rids, rcnt = O.OracleIndex.from_codebook(cb, use_ip=ip).search(q, K, beam)
    assert np.array_equal(ids2, rids)
    assert np.array_equal(cnt2, rcnt.view(np.uint32).reshape(-1, 6))


def test_two_launch_search_device_back_to_back(gpu_available, monkeypatch):
    """Sliced device searches on one stream reuse the index's state buffer one
    after another; a second index is independent; results equal fg_search's."""
    import torch
    from flashgann_amd import Index
    cb, q, _ = small_index(n=3000, nq=300)
    monkeypatch.setenv("FLASHGANN_TEAM", "0")
    monkeypatch.setenv("FLASHGANN_SLICE", "0")
    a = Index.from_codebook(cb)
    ref = {b: a.search(q, 100, b)[0] for b in (128, 256)}
    monkeypatch.setenv("FLASHGANN_SLICE", "1")
    dq = torch.as_tensor(q, device="cuda")
    s = torch.cuda.current_stream()
    outs = []
    for b in (256, 128, 256):
        out = torch.full((q.shape[0], 100), -1, dtype=torch.int32, device="cuda")
        a.search_device(dq.data_ptr(), q.shape[0], 100, b, out.data_ptr(), 0, s.cuda_stream)
        outs.append((b, out))
    torch.cuda.synchronize()
    for b, out in outs:
        assert np.array_equal(out.cpu().numpy().view(np.uint32), ref[b]), b
    a.close()


def test_device_search_captured_in_a_graph(gpu_available, monkeypatch):
    """A device search on a stream that is being captured makes one launch
    (the two-launch search would allocate and order itself with an event);
    every replay, with eager work between replays, returns the eager ids."""
    import torch
    from flashgann_amd import Index
    cb, q, _ = small_index(n=3000, nq=300)
    monkeypatch.setenv("FLASHGANN_TEAM", "0")
    monkeypatch.setenv("FLASHGANN_SLICE", "1")
    ix = Index.from_codebook(cb)
    ref, _, _ = ix.search(q, 100, 256)
    dq = torch.as_tensor(q, device="cuda")
    out = torch.full((q.shape[0], 100), -1, dtype=torch.int32, device="cuda")
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        ix.search_device(dq.data_ptr(), q.shape[0], 100, 256, out.data_ptr(), 0, s.cuda_stream)
    for _ in range(3):
        out.fill_(-1)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy().view(np.uint32), ref)
    del g
    ix.close()


def test_search_launches_reports_the_schedule(gpu_available, monkeypatch):
    """fg_search_launches: one launch while every query of a one-wave batch
    starts at once, two for a larger batch (up to 16,384 queries), one above
    that and for the team form; the environment override wins where the form
    allows two.  The residency threshold is found by bisection and must be a
    whole number of workgroups per CU (it depends on the device's CU count
    and the kernel's occupancy, so no number is hard-coded)."""
    import torch
    from flashgann_amd import Index
    cb, q, _ = small_index()
    ix = Index.from_codebook(cb)
    monkeypatch.delenv("FLASHGANN_TEAM", raising=False)
    monkeypatch.delenv("FLASHGANN_SLICE", raising=False)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    lo, hi = 2 * cus, 16384  # (2 x CUs: the team form, one launch)
    assert ix.search_launches(lo, 100, 256) == 1
    assert ix.search_launches(hi, 100, 256) == 2
    while hi - lo > 1:  # the largest one-launch batch
        mid = (lo + hi) // 2
        if ix.search_launches(mid, 100, 256) == 1:
            lo = mid
        else:
            hi = mid
    assert lo % cus == 0 and 2 <= lo // cus <= 64, (lo, cus)
    assert all(ix.search_launches(n, 100, 256) == 2 for n in (lo + 1, lo + 1000, 16384, 16385, 100000))
    assert ix.search_launches(16, 10, 64) == 1        # the team form
    # 200,000 queries at beam 1024 would keep 1.7 GB of state: one launch
    assert ix.search_launches(200000, 100, 1024) == 1
    monkeypatch.setenv("FLASHGANN_SLICE", "0")
    assert ix.search_launches(16384, 100, 256) == 1
    monkeypatch.setenv("FLASHGANN_SLICE", "1")
    assert ix.search_launches(lo, 100, 256) == 2
    ix.close()


@pytest.mark.parametrize("nq,beam", [(4000, 256), (4000, 384), (16384, 256), (16384, 512), (16385, 256),
                                     (30000, 384)])
def test_two_launch_search_large_batches(gpu_available, monkeypatch, nq, beam):
    """Forced two-launch searches over batches that use every part of the
    order step: queries past the one-workgroup kernel's first 1,024 slots and
    at its 16,384-query maximum, then the multi-workgroup path (chunks of
    4,096, a last partial chunk).  Ids and counters equal the one-launch
    search's, and on the distinct queries the oracle's.  The batch repeats
    300 queries, so each distinct query is checked at many positions of the
    order."""
    from flashgann_amd import Index
    from oracle import oracle as O
    cb, q, _ = small_index(n=3000, nq=300)
    qq = np.ascontiguousarray(np.resize(q, (nq, q.shape[1])))
    ix = Index.from_codebook(cb)
    monkeypatch.setenv("FLASHGANN_TEAM", "0")
    monkeypatch.setenv("FLASHGANN_SLICE", "0")
    ids1, _, cnt1 = ix.search(qq, 100, beam, counters=True)
    monkeypatch.setenv("FLASHGANN_SLICE", "1")
    assert ix.search_launches(nq, 100, beam) == 2
    ids2, _, cnt2 = ix.search(qq, 100, beam, counters=True)
    ix.close()
    assert (cnt1[:, 0] > 15).any()
    assert np.array_equal(ids2, ids1) and np.array_equal(cnt2, cnt1)
    rids, rcnt = O.OracleIndex.from_codebook(cb).search(q, 100, beam)
    rep = np.arange(nq) % q.shape[0]
    assert np.array_equal(ids2, rids[rep])
    assert np.array_equal(cnt2, rcnt.view(np.uint32).reshape(-1, 6)[rep])


@pytest.mark.parametrize("team", ["0", "1"])
@pytest.mark.parametrize("beam", [64, 512])
def test_profiling_build_same_ids(gpu_available, monkeypatch, team, beam):
    """fg_search_profile (the phase-timer instantiation of the kernel, the
    one-wave and team forms) returns the ids of the ordinary search, and its
    per-query timers are sane: phase cycle sums >= 0 and start <= end."""
    import torch
    import flashgann_amd as fg
    from flashgann_amd import Index
    monkeypatch.setenv("FLASHGANN_TEAM", team)
    cb, q, _ = small_index(n=3000, nq=24, dim=128, comps=16, degree=32)
    ix = Index.from_codebook(cb)
    K = 10
    ids = ix.search(q, K, beam)[0]
    dq = torch.as_tensor(np.ascontiguousarray(q, np.float32), device="cuda")
    dres = torch.zeros((len(q), K), dtype=torch.int32, device="cuda")
    dph = torch.zeros((len(q), fg.FG_PROFILE_SLOTS), dtype=torch.int64, device="cuda")
    ix.search_profile(dq.data_ptr(), len(q), K, beam, dres.data_ptr(), dph.data_ptr(), 0)
    torch.cuda.synchronize()
    ix.close()
    assert np.array_equal(dres.cpu().numpy().view(np.uint32), ids)
    ph = dph.cpu().numpy()
    assert (ph[:, :10] >= 0).all() and (ph[:, :10].sum(1) > 0).all()
    assert (ph[:, 10] <= ph[:, 11]).all() and (ph[:, 10] > 0).all()
