"""Writes tests/golden/ref_host_golden.npz: inputs and the outputs of the
reference's own host code for them (include/common.hpp compute_recall and
compute_rabitq_entry_point, include/qg.hpp's layout as its loader reads a
codebook file, metric.hpp's metric inference), computed by the reference
headers compiled from the reference tree into oracle/_ref (make -C oracle
ref).  The committed file lets tests/test_golden_ref_host.py check the oracle
and this build's host code against those outputs where the reference tree is
absent.  Run from the repository root:

    python tests/golden/make_ref_host_golden.py
"""
from __future__ import annotations

import ctypes as C
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from flashgann_amd.codebook import Layout, write_codebook  # noqa: E402
from oracle import oracle as O  # noqa: E402

RECALL_CASES = [(10, 10), (100, 100), (10, 100), (100, 50), (1, 1), (7, 3)]
LAYOUTS = [(33, 1), (40, 8), (64, 32), (96, 16), (96, 32), (100, 24), (128, 32), (200, 48), (960, 32), (1536, 32)]
METRIC_PATHS = ["/data/sift/base.fvecs", "/x/Text2Image1M/base.fbin", "text2image1m", "TEXT2IMAGE1M_x",
                "/d/text2image1m/", "deep1m", ""]


def main() -> int:
    R = O.ref_lib()
    if R is None:
        print("oracle/_ref is not built (make -C oracle ref needs the reference tree)", file=sys.stderr)
        return 1
    rng = np.random.default_rng(20261202)
    out = {}
    for i, (K, gtk) in enumerate(RECALL_CASES):
        nq = 37
        pred = rng.integers(0, 300, (nq, K)).astype(np.uint32)  # repeats included
        gt = rng.integers(0, 300, (nq, gtk)).astype(np.int32)
        r = R.ref_compute_recall(O.ptr(pred, C.c_uint32), gt.ctypes.data_as(C.POINTER(C.c_int)), nq, K, gtk)
        out[f"recall{i}_pred"], out[f"recall{i}_gt"] = pred.astype(np.uint16), gt.astype(np.uint16)
        out[f"recall{i}_value"] = np.float32(r)
    # integer-valued rows (stored as int8; exact as float32), so that distance
    # ties occur and the reference's tie rule is part of the record
    for i, (n, dim, use_ip, lim) in enumerate([(500, 37, 0, 50), (500, 37, 1, 50), (400, 128, 0, 3),
                                               (400, 96, 1, 100)]):
        q = rng.integers(-lim, lim + 1, (n, dim)).astype(np.int8)
        rows = q.astype(np.float32)
        e = R.ref_compute_entry_point(O.ptr(rows, C.c_float), n, dim, dim, use_ip)
        out[f"entry{i}_rows"], out[f"entry{i}_ip"], out[f"entry{i}_value"] = q, np.int32(use_ip), np.uint32(e)
    # exact ties: (a) the nearest row also stored later, so the first of equal
    # distances is kept; (b) triples c + v, c - v, c + w with v and w on
    # disjoint dimensions, whose first two rows are equally far from the true
    # centroid c + w / 3: the float centroid (each row scaled by fl(1/n), then
    # summed) decides which one is nearer
    base = rng.integers(-20, 21, (300, 37)).astype(np.float32)
    e0 = R.ref_compute_entry_point(O.ptr(base, C.c_float), 300, 37, 37, 0)
    tie = np.concatenate([base, base[e0:e0 + 1]]).astype(np.int8)
    tf = tie.astype(np.float32)
    out["entry_tie_rows"] = tie
    out["entry_tie_value"] = np.uint32(R.ref_compute_entry_point(O.ptr(tf, C.c_float), 301, 37, 37, 0))
    trip = []
    for _ in range(64):
        c = rng.integers(-40, 41, 16)
        v = np.zeros(16, np.int64)
        w = np.zeros(16, np.int64)
        v[:8] = rng.integers(-3, 4, 8)  # |v|^2 < |w|^2 / 3: the pair is nearer than c + w
        w[8:] = rng.integers(-9, 10, 8)
        t = np.stack([c + v, c - v, c + w]).astype(np.float32)
        trip.append(t)
    trip = np.stack(trip)
    out["entry_triples"] = trip.astype(np.int8)
    out["entry_triples_value"] = np.asarray(
        [R.ref_compute_entry_point(O.ptr(np.ascontiguousarray(t), C.c_float), 3, 16, 16, 0) for t in trip], np.uint32)
    offs_all = []
    with tempfile.TemporaryDirectory() as td:
        for dim, deg in LAYOUTS:
            lay = Layout.make(dim, deg)
            rows = np.zeros((2, lay.row_offset), np.float32)
            signs = np.ones(lay.padded_dim, np.float32)
            p = os.path.join(td, "cb.index")
            write_codebook(p, rows, signs, 1)
            offs = (C.c_uint64 * 5)()
            entry = C.c_uint32()
            rbuf = np.zeros(rows.size, np.float32)
            sbuf = np.zeros(lay.padded_dim, np.float32)
            rc = R.ref_qg_load(p.encode(), 2, dim, deg, offs, C.byref(entry), O.ptr(rbuf, C.c_float), rbuf.size,
                               O.ptr(sbuf, C.c_float), sbuf.size)
            assert rc == 0
            offs_all.append([dim, deg] + list(offs))
    out["layouts"] = np.asarray(offs_all, np.uint64)  # dim, degree, code, factor, neighbor, row offsets, padded dim
    out["metric_paths"] = np.asarray(METRIC_PATHS)
    out["metric_is_ip"] = np.asarray([R.ref_infer_metric_is_ip(p.encode()) for p in METRIC_PATHS], np.int32)
    dst = os.path.join(HERE, "ref_host_golden.npz")
    np.savez_compressed(dst, **out)
    print(f"wrote {dst} ({os.path.getsize(dst)} bytes)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
