"""The oracle's and this build's host-side pieces against recorded outputs of
the reference's own host code (tests/golden/ref_host_golden.npz, written by
tests/golden/make_ref_host_golden.py from the reference headers compiled into
oracle/_ref): compute_recall and compute_rabitq_entry_point
(include/common.hpp:26-66), the codebook layout as the reference's loader
computes it (include/qg.hpp:17-42, 66-73) and the dataset-path metric
inference (include/metric.hpp).  Unlike tests/test_ref_host.py these run
without the reference tree."""
from __future__ import annotations

import os

import numpy as np

from oracle import oracle as O

GOLDEN = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ref_host_golden.npz"))


def test_recall_matches_recorded_reference():
    from flashgann_amd.metrics import compute_recall
    i = 0
    while f"recall{i}_value" in GOLDEN.files:
        pred = GOLDEN[f"recall{i}_pred"].astype(np.uint32)
        gt = np.ascontiguousarray(GOLDEN[f"recall{i}_gt"].astype(np.int32))
        want = np.float32(GOLDEN[f"recall{i}_value"])
        nq, K = pred.shape
        got = O.lib().fgo_recall(O.ptr(pred, O.C.c_uint32), O.ptr(gt, O.C.c_int32), nq, K, gt.shape[1])
        assert np.float32(got) == want, i
        assert np.float32(compute_recall(pred, gt, K)) == want, i
        i += 1
    assert i >= 6


def test_entry_point_matches_recorded_reference():
    i = 0
    while f"entry{i}_value" in GOLDEN.files:
        rows = np.ascontiguousarray(GOLDEN[f"entry{i}_rows"].astype(np.float32))
        n, dim = rows.shape
        got = O.lib().fgo_entry_point(O.ptr(rows, O.C.c_float), n, dim, dim, int(GOLDEN[f"entry{i}_ip"]))
        assert got == int(GOLDEN[f"entry{i}_value"]), i
        i += 1
    assert i >= 4


def test_layout_matches_recorded_reference():
    from flashgann_amd.codebook import Layout
    lay_c = O.Layout()
    for dim, deg, code, factor, nbr, row, padded in GOLDEN["layouts"].tolist():
        lay = Layout.make(dim, deg)
        assert (lay.code_offset, lay.factor_offset, lay.neighbor_offset, lay.row_offset, lay.padded_dim) == \
            (code, factor, nbr, row, padded), (dim, deg)
        assert O.lib().fgo_compute_layout(dim, deg, O.C.byref(lay_c)) == 0
        assert (lay_c.code_offset, lay_c.factor_offset, lay_c.neighbor_offset, lay_c.row_offset,
                lay_c.padded_dim) == (code, factor, nbr, row, padded), (dim, deg)


def test_metric_inference_matches_recorded_reference():
    import flashgann_amd as fg
    for path, is_ip in zip(GOLDEN["metric_paths"].tolist(), GOLDEN["metric_is_ip"].tolist()):
        assert int(fg.infer_metric_from_dataset_path(path)) == is_ip, path


def test_entry_point_ties_match_recorded_reference():
    """Exact ties: the nearest row stored twice keeps the first index, and
    pairs c + v, c - v equally far from the true centroid c + w / 3 (v and w
    on disjoint dimensions) are decided by the float centroid, each row
    scaled by fl(1/n) and then summed (common.hpp:26-47): the recorded
    winners are mostly the first row of the pair, sometimes the second."""
    rows = np.ascontiguousarray(GOLDEN["entry_tie_rows"].astype(np.float32))
    n, dim = rows.shape
    assert np.array_equal(rows[-1], rows[int(GOLDEN["entry_tie_value"])])
    assert O.lib().fgo_entry_point(O.ptr(rows, O.C.c_float), n, dim, dim, 0) == int(GOLDEN["entry_tie_value"])
    want = GOLDEN["entry_triples_value"].tolist()
    assert set(want[:]) >= {0, 1}
    for t, w in zip(GOLDEN["entry_triples"].astype(np.float32), want):
        t = np.ascontiguousarray(t)
        assert O.lib().fgo_entry_point(O.ptr(t, O.C.c_float), 3, t.shape[1], t.shape[1], 0) == w
