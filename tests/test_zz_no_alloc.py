"""fg_search_noalloc, the allocation-free form of fg_search, against
fg_search itself: ids and work counters identical on two calls in a row (the
second with fewer queries, so stale staging from the first would show), with
and without counters; a call whose staging exceeds the fixed area is rejected
before any device work; the first search of a fresh index allocates no
device memory; calls from two host threads on one device take turns."""
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


def test_noalloc_first_search_on_a_fresh_index_allocates_nothing(gpu_available):
    """On an index that has never searched (so fg_search's own staging
    buffers do not exist), the first call is fg_search_noalloc: the device's
    free memory is the same before and after it, and a second call returns
    the same ids.  A search on another index first loads the kernels, whose
    code objects take device memory once per process."""
    import torch

    from flashgann_amd import Index
    cb, q, _ = small_index(nq=400)
    warm = Index.from_codebook(cb)
    warm.search(q[:64], 100, 256, counters=True, noalloc=True)
    warm.close()
    ix = Index.from_codebook(cb)
    try:
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info()[0]
        ids, _, cnt = ix.search(q[:64], 100, 256, counters=True, noalloc=True)
        torch.cuda.synchronize()
        assert torch.cuda.mem_get_info()[0] == free0
        ids2, _, cnt2 = ix.search(q[:64], 100, 256, counters=True, noalloc=True)
        assert np.array_equal(ids2, ids) and np.array_equal(cnt2, cnt)
        assert torch.cuda.mem_get_info()[0] == free0
    finally:
        ix.close()


def test_noalloc_calls_from_two_threads_take_turns(gpu_available):
    """Two host threads search two indices on one device through
    fg_search_noalloc at the same time (ctypes releases the interpreter lock
    during the call), each with its own queries: every call returns the ids
    its own serial call does, because the per-device lock keeps one call at a
    time in the shared staging area."""
    import threading

    from flashgann_amd import Index
    cb, q, _ = small_index(nq=400)
    cb96, q96, _ = small_index(n=2000, nq=24, dim=96, degree=16, kind="unit")
    a, b = Index.from_codebook(cb), Index.from_codebook(cb96)
    try:
        want_a = [a.search(q[i * 50:(i + 1) * 50], 10, 128)[0] for i in range(8)]
        want_b = b.search(q96, 10, 128)[0]
        errors = []

        def run_a():
            for rep in range(6):
                for i in range(8):
                    if not np.array_equal(a.search(q[i * 50:(i + 1) * 50], 10, 128, noalloc=True)[0], want_a[i]):
                        errors.append(("a", rep, i))

        def run_b():
            for rep in range(48):
                if not np.array_equal(b.search(q96, 10, 128, noalloc=True)[0], want_b):
                    errors.append(("b", rep))

        ts = [threading.Thread(target=run_a), threading.Thread(target=run_b)]
        for t in ts:
            t.start()
        for t in ts:
            t.join(timeout=60)
        assert not any(t.is_alive() for t in ts)
        assert not errors, errors[:5]
    finally:
        a.close()
        b.close()
