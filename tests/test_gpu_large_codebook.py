"""GPU parity on a codebook larger than 4 GiB whose reachable rows all lie
beyond byte offset 2^32.  The reference addresses a row as
size_t(node) * row_offset (src/adaptive_search.cuh:225, 338, 366, 438); the
kernels specialised for d 128 / degree 32 use 32-bit byte offsets, so a
codebook of 4 GiB or more must be served by the general kernels with 64-bit
row addresses.  A 3,000-node graph is placed at node ids 2,800,000 ..
2,802,999 of a 2,900,000-row codebook (4.45 GB at 1,536 B per row; row
2,796,203 is the first to start past 2^32 bytes); the other rows are
unreachable.  Ids and work counters must equal the oracle's, and equal the
same search on the 3,000-row codebook with the ids shifted (the search
depends on ids only through the visited set, which is exact)."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import small_index

pytestmark = pytest.mark.gpu

ROWS = 2_900_000
OFFSET = 2_800_000


def _big_codebook(cb):
    from flashgann_amd.codebook import MAX_INDEX, Codebook
    lay = cb.layout
    assert OFFSET * lay.row_offset * 4 > 1 << 32
    rows = np.zeros((ROWS, lay.row_offset), np.float32)
    rows[:, lay.neighbor_offset:].view(np.uint32)[:] = MAX_INDEX
    small = cb.rows.copy()
    ids = small[:, lay.neighbor_offset:].view(np.uint32)
    ids[ids != MAX_INDEX] += OFFSET
    rows[OFFSET:OFFSET + cb.npoints] = small
    return Codebook(rows, cb.signs, cb.entry + OFFSET, lay)


@pytest.mark.parametrize("K,beam", [(10, 64), (100, 256)])
def test_codebook_above_4gib_matches_oracle(gpu_available, K, beam):
    from flashgann_amd import Index
    from oracle import oracle as O
    cb, q, _ = small_index(n=3000, nq=48, dim=128, comps=16, degree=32)
    big = _big_codebook(cb)
    print(f"codebook above 4 GiB: {big.rows.nbytes / 1e9:.2f} GB, K={K}, beam={beam}", flush=True)
    ix = Index.from_codebook(big)
    assert ix.search_geometry() == 1  # the general kernels, 64-bit row addresses
    ids, _, cnt = ix.search(q, K, beam, counters=True)
    ix.close()
    small_ix = Index.from_codebook(cb)
    assert small_ix.search_geometry() == 0
    sids, _, scnt = small_ix.search(q, K, beam, counters=True)
    small_ix.close()
    rids, rcnt = O.OracleIndex.from_codebook(big).search(q, K, beam)
    assert (ids >= OFFSET).all() and (ids < OFFSET + cb.npoints).all()
    assert np.array_equal(ids, rids)
    assert np.array_equal(cnt, rcnt.view(np.uint32).reshape(-1, 6))
    assert np.array_equal(ids, sids + OFFSET)
    assert np.array_equal(cnt, scnt)
