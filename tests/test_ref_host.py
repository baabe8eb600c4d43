"""The oracle's and the product's host-side pieces against the reference's own
host code (include/common.hpp, data_io.hpp, qg.hpp, metric.hpp compiled from
the reference tree into oracle/_ref by oracle/Makefile)."""
from __future__ import annotations

import ctypes as C
import os

import numpy as np
import pytest

from oracle import oracle as O

REF = O.ref_lib()
pytestmark = pytest.mark.skipif(REF is None, reason="oracle/_ref not built (reference tree absent)")


def test_recall_matches_reference():
    from flashgann_amd.metrics import compute_recall
    rng = np.random.default_rng(0)
    for K, gtk in [(10, 10), (100, 100), (10, 100), (100, 50)]:
        nq = 37
        pred = rng.integers(0, 300, (nq, K)).astype(np.uint32)      # duplicates included
        gt = rng.integers(0, 300, (nq, gtk)).astype(np.int32)
        r_ref = REF.ref_compute_recall(O.ptr(pred, C.c_uint32), gt.ctypes.data_as(C.POINTER(C.c_int)), nq, K, gtk)
        r_or = O.lib().fgo_recall(O.ptr(pred, C.c_uint32), O.ptr(gt, C.c_int32), nq, K, gtk)
        assert r_ref == r_or
        assert np.float32(compute_recall(pred, gt, K)) == np.float32(r_ref)


@pytest.mark.parametrize("use_ip", [0, 1])
def test_entry_point_matches_reference(use_ip):
    rng = np.random.default_rng(1 + use_ip)
    n, dim, row = 3000, 100, 356
    rows = np.zeros((n, row), np.float32)
    rows[:, :dim] = rng.standard_normal((n, dim)).astype(np.float32) * 3 + 1
    a = REF.ref_compute_entry_point(O.ptr(rows, C.c_float), n, dim, row, use_ip)
    b = O.lib().fgo_entry_point(O.ptr(rows, C.c_float), n, dim, row, use_ip)
    assert a == b


def test_vecs_loaders_match_reference(tmp_path):
    from flashgann_amd.codebook import read_fvecs, read_ivecs, write_fvecs, write_ivecs
    rng = np.random.default_rng(2)
    x = rng.standard_normal((50, 17)).astype(np.float32)
    g = rng.integers(0, 1000, (50, 9)).astype(np.int32)
    fp, ip_ = str(tmp_path / "x.fvecs"), str(tmp_path / "g.ivecs")
    write_fvecs(fp, x)
    write_ivecs(ip_, g)
    d = C.c_int()
    buf = np.zeros(50 * 17, np.float32)
    n = REF.ref_load_fvecs(fp.encode(), C.byref(d), O.ptr(buf, C.c_float), buf.size)
    assert (n, d.value) == (50, 17) and np.array_equal(buf.reshape(50, 17), x)
    gb = np.zeros(50 * 9, np.int32)
    n = REF.ref_load_ivecs(ip_.encode(), C.byref(d), gb.ctypes.data_as(C.POINTER(C.c_int)), gb.size)
    assert (n, d.value) == (50, 9) and np.array_equal(gb.reshape(50, 9), g)
    assert np.array_equal(read_fvecs(fp), x) and np.array_equal(read_ivecs(ip_), g)


@pytest.mark.parametrize("dim,deg", [(128, 32), (96, 16), (960, 32)])
def test_codebook_file_matches_reference_loader(tmp_path, dim, deg):
    from flashgann_amd.codebook import Layout, read_codebook, write_codebook
    lay = Layout.make(dim, deg)
    rng = np.random.default_rng(dim + deg)
    n = 40
    rows = rng.standard_normal((n, lay.row_offset)).astype(np.float32)
    signs = np.where(rng.random(lay.padded_dim) < 0.5, -1, 1).astype(np.float32)
    p = str(tmp_path / "cb.index")
    write_codebook(p, rows, signs, 17)
    offs = (C.c_uint64 * 5)()
    entry = C.c_uint32()
    rbuf = np.zeros(rows.size, np.float32)
    sbuf = np.zeros(lay.padded_dim, np.float32)
    REF.ref_qg_load(p.encode(), n, dim, deg, offs, C.byref(entry), O.ptr(rbuf, C.c_float), rbuf.size,
                    O.ptr(sbuf, C.c_float), sbuf.size)
    assert list(offs) == [lay.code_offset, lay.factor_offset, lay.neighbor_offset, lay.row_offset, lay.padded_dim]
    assert entry.value == 17
    assert np.array_equal(rbuf.reshape(n, -1), rows) and np.array_equal(sbuf, signs)
    cb = read_codebook(p, n, dim, deg)
    assert cb.entry == 17 and np.array_equal(cb.rows, rows) and np.array_equal(cb.signs, signs)


def test_metric_inference_matches_reference():
    import flashgann_amd as fg
    for path in ["/data/sift/base.fvecs", "/x/Text2Image1M/base.fbin", "text2image1m", "TEXT2IMAGE1M_x", ""]:
        assert fg.infer_metric_from_dataset_path(path) == REF.ref_infer_metric_is_ip(path.encode())
