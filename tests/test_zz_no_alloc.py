"""fg_search_noalloc, the allocation-free form of fg_search, against
fg_search itself: ids and work counters identical on two calls in a row (the
second with fewer queries, so stale staging from the first would show), with
and without counters; a call whose staging exceeds the fixed area is rejected
before any device work."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import small_index

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("search_form")]


def test_noalloc_equals_fg_search(gpu_available):
    from flashgann_amd import Index
    cb, q, _ = small_index(nq=400)
    ix = Index.from_codebook(cb)
    try:
        for nq, K, beam in ((400, 100, 256), (37, 10, 64), (5, 100, 1000)):
            ids, _, cnt = ix.search(q[:nq], K, beam, counters=True)
            ids_na, st, cnt_na = ix.search(q[:nq], K, beam, counters=True, noalloc=True)
            assert np.array_equal(ids_na, ids), (nq, K, beam)
            assert np.array_equal(cnt_na, cnt), (nq, K, beam)
            assert st.kernel_ms > 0.0
            ids_nc, _, none = ix.search(q[:nq], K, beam, noalloc=True)
            assert none is None and np.array_equal(ids_nc, ids), (nq, K, beam)
    finally:
        ix.close()


def test_noalloc_shared_by_indices_on_one_device(gpu_available):
    """Two indices on one device use the same staging area, one call at a time."""
    from flashgann_amd import Index
    cb, q, _ = small_index(nq=400)
    cb96, q96, _ = small_index(n=2000, nq=24, dim=96, degree=16, kind="unit")
    a, b = Index.from_codebook(cb), Index.from_codebook(cb96)
    try:
        ra, _, _ = a.search(q[:64], 10, 128)
        rb, _, _ = b.search(q96, 10, 128)
        assert np.array_equal(a.search(q[:64], 10, 128, noalloc=True)[0], ra)
        assert np.array_equal(b.search(q96, 10, 128, noalloc=True)[0], rb)
        assert np.array_equal(a.search(q[:64], 10, 128, noalloc=True)[0], ra)
    finally:
        a.close()
        b.close()


def test_noalloc_rejects_staging_above_maximum(gpu_available):
    from flashgann_amd import FlashGannError, Index, _lib
    cb, q, _ = small_index(nq=400)
    ix = Index.from_codebook(cb)
    try:
        per_query = 128 * 4 + 100 * 4
        nq = _lib.FG_NOALLOC_STAGING_BYTES // per_query + 16
        big = np.resize(q, (nq, 128)).astype(np.float32)
        with pytest.raises(FlashGannError) as e:
            ix.search(big, 100, 64, noalloc=True)
        assert e.value.code == _lib.FG_EINVAL and "staging" in str(e.value)
        # the area is still usable afterwards
        ids, _, _ = ix.search(q[:8], 100, 64)
        assert np.array_equal(ix.search(q[:8], 100, 64, noalloc=True)[0], ids)
    finally:
        ix.close()
