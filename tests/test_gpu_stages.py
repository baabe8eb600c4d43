"""Stage-level parity: query preparation, RaBitQ estimates and exact
distances from the HIP kernels against the oracle, bit for bit."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from conftest import small_index

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("search_form")]


STAGE_CASES = [("int", 128, 1500), ("unit", 96, 1500), ("box", 960, 1500), ("aniso", 1536, 1200)]


@pytest.mark.parametrize("kind,dim,n", STAGE_CASES)
def test_query_prepare_matches_oracle(gpu_available, kind, dim, n):
    from flashgann_amd import Index
    from oracle import oracle as O
    cb, q, _ = small_index(n=n, nq=8, dim=dim, comps=8, kind=kind)
    ix = Index.from_codebook(cb)
    rot, qt, lhw, sq = ix.query_prepare(q)
    B = cb.layout.padded_dim
    for i in range(q.shape[0]):
        qf = O.query_prepare(q[i], cb.signs, dim, B)
        assert np.array_equal(rot[i], np.ctypeslib.as_array(qf.rotated)[:B])
        assert np.array_equal(qt[i], np.ctypeslib.as_array(qf.q)[:B])
        assert (lhw[i, 0], lhw[i, 1], lhw[i, 2]) == (np.float32(qf.low), np.float32(qf.high), np.float32(qf.width))
        assert sq[i] == qf.sum_q
    ix.close()


@pytest.mark.parametrize("kind,dim,n", STAGE_CASES)
def test_scores_match_oracle(gpu_available, kind, dim, n):
    from flashgann_amd import Index
    from oracle import oracle as O
    cb, q, _ = small_index(n=n, nq=8, dim=dim, comps=8, kind=kind)
    ix = Index.from_codebook(cb)
    rng = np.random.default_rng(5)
    n = 300
    qi = rng.integers(0, q.shape[0], n).astype(np.uint32)
    pa = rng.integers(0, cb.npoints, n).astype(np.uint32)
    sl = rng.integers(0, cb.layout.degree, n).astype(np.uint32)
    el, es, ex = ix.score_edges(q, qi, pa, sl)
    lay = cb.layout
    L = O.lib()
    codes = cb.codes()
    fac = cb.factors()
    nb = cb.neighbors()
    for t in range(n):
        qf = O.query_prepare(q[qi[t]], cb.signs, dim, lay.padded_dim)
        prow = cb.rows[pa[t]]
        pd = L.fgo_warp_l2(dim, O.ptr(np.ascontiguousarray(q[qi[t]]), C.c_float), O.ptr(np.ascontiguousarray(prow[:dim]), C.c_float))
        code = np.ascontiguousarray(codes[pa[t], sl[t]])
        tx, fdq, fvq = (float(fac[pa[t], j, sl[t]]) for j in range(3))
        ref_l = L.fgo_estimate_lanes(C.byref(qf), O.ptr(code, C.c_uint8), tx, fdq, fvq, pd, lay.padded_dim)
        ref_s = L.fgo_estimate_seq(C.byref(qf), O.ptr(code, C.c_uint8), tx, fdq, fvq, pd, lay.padded_dim)
        child = int(nb[pa[t], sl[t]])
        ref_x = L.fgo_warp_l2(dim, O.ptr(np.ascontiguousarray(q[qi[t]]), C.c_float),
                              O.ptr(np.ascontiguousarray(cb.rows[child, :dim]), C.c_float))
        assert np.float32(el[t]) == np.float32(ref_l), t
        assert np.float32(es[t]) == np.float32(ref_s), t
        assert np.float32(ex[t]) == np.float32(ref_x), t
    ix.close()


def _wrap_queries(signs, B, count, seed=12):
    """Queries whose rotation puts four 64s in some 4-dim chunk (the uint8
    LUT entry of that chunk wraps): z non-zero only at multiples of 4 makes
    H z constant on every chunk, and x = s * z keeps the rotation exact."""
    from oracle import oracle as O
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < count:
        z = np.zeros(B, np.float32)
        z[::4] = rng.integers(-40, 60, B // 4)
        x = (signs * z).astype(np.float32)
        qf = O.query_prepare(x, signs, B, B)
        q = np.ctypeslib.as_array(qf.q)[:B]
        if (q.reshape(-1, 4) == 64).all(1).any():
            out.append(x)
    return np.stack(out)


@pytest.mark.parametrize("dim", [64, 256, 512, 1024, 2048])
def test_wrap_chunks_scores_and_search(gpu_available, dim):
    """The popcount planes' wrap correction reproduces the uint8 LUT, for
    each code width the estimators have: 2 words (fixed geometry) and 8, 16,
    32 and 2 x 32 words (generic geometry)."""
    from flashgann_amd import Index
    from oracle import oracle as O
    cb, _, _ = small_index(n=1200, nq=4, dim=dim, comps=8)
    q = _wrap_queries(cb.signs, dim, 6)
    ix = Index.from_codebook(cb)
    rng = np.random.default_rng(3)
    n = 200
    qi = rng.integers(0, q.shape[0], n).astype(np.uint32)
    pa = rng.integers(0, cb.npoints, n).astype(np.uint32)
    sl = rng.integers(0, cb.layout.degree, n).astype(np.uint32)
    el, es, _ = ix.score_edges(q, qi, pa, sl)
    L = O.lib()
    codes, fac = cb.codes(), cb.factors()
    for t in range(n):
        qf = O.query_prepare(q[qi[t]], cb.signs, dim, dim)
        pd = L.fgo_warp_l2(dim, O.ptr(np.ascontiguousarray(q[qi[t]]), C.c_float),
                           O.ptr(np.ascontiguousarray(cb.rows[pa[t], :dim]), C.c_float))
        code = np.ascontiguousarray(codes[pa[t], sl[t]])
        args = (float(fac[pa[t], 0, sl[t]]), float(fac[pa[t], 1, sl[t]]), float(fac[pa[t], 2, sl[t]]), pd, dim)
        assert np.float32(el[t]) == np.float32(L.fgo_estimate_lanes(C.byref(qf), O.ptr(code, C.c_uint8), *args))
        assert np.float32(es[t]) == np.float32(L.fgo_estimate_seq(C.byref(qf), O.ptr(code, C.c_uint8), *args))
    ids, _, cnt = ix.search(q, 10, 64, counters=True)
    rids, rcnt = O.OracleIndex.from_codebook(cb).search(q, 10, 64)
    assert np.array_equal(ids, rids)
    assert np.array_equal(cnt, rcnt.view(np.uint32).reshape(-1, 6))
    ix.close()


@pytest.mark.parametrize("kind,dim,n", [("int", 64, 1200), ("int", 128, 1500), ("unit", 96, 1500), ("box", 960, 1500)])
def test_zero_level_query_scores_and_search(gpu_available, kind, dim, n):
    """A query whose rotation is constant (the zero vector: width 0)
    quantizes every level to 0, so the estimator's level-0 correction is the
    whole sum: scores equal the oracle's bit for bit, and so do the search's
    ids and counters, for code widths of 2, 4 and 32 words."""
    from flashgann_amd import Index
    from oracle import oracle as O
    cb, q, _ = small_index(n=n, nq=4, dim=dim, comps=8, kind=kind)
    zq = np.concatenate([np.zeros((2, dim), np.float32), q[:2]])
    ix = Index.from_codebook(cb)
    rng = np.random.default_rng(8)
    m = 120
    qi = rng.integers(0, 2, m).astype(np.uint32)
    pa = rng.integers(0, cb.npoints, m).astype(np.uint32)
    sl = rng.integers(0, cb.layout.degree, m).astype(np.uint32)
    el, es, _ = ix.score_edges(zq, qi, pa, sl)
    L = O.lib()
    codes, fac = cb.codes(), cb.factors()
    B = cb.layout.padded_dim
    for t in range(m):
        qf = O.query_prepare(zq[qi[t]], cb.signs, dim, B)
        assert np.ctypeslib.as_array(qf.q)[:B].max() == 0
        pd = L.fgo_warp_l2(dim, O.ptr(np.ascontiguousarray(zq[qi[t]]), C.c_float),
                           O.ptr(np.ascontiguousarray(cb.rows[pa[t], :dim]), C.c_float))
        code = np.ascontiguousarray(codes[pa[t], sl[t]])
        args = (float(fac[pa[t], 0, sl[t]]), float(fac[pa[t], 1, sl[t]]), float(fac[pa[t], 2, sl[t]]), pd, B)
        assert np.float32(el[t]) == np.float32(L.fgo_estimate_lanes(C.byref(qf), O.ptr(code, C.c_uint8), *args))
        assert np.float32(es[t]) == np.float32(L.fgo_estimate_seq(C.byref(qf), O.ptr(code, C.c_uint8), *args))
    ids, _, cnt = ix.search(zq, 10, 64, counters=True)
    rids, rcnt = O.OracleIndex.from_codebook(cb).search(zq, 10, 64)
    assert np.array_equal(ids, rids)
    assert np.array_equal(cnt, rcnt.view(np.uint32).reshape(-1, 6))
    ix.close()
