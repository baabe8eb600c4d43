"""GPU parity on the hand-traced cases of tests/crafted.py: the kernel's ids
and work counters must equal the oracle's (whose traces on the same inputs
are pinned by hand in test_oracle_traces.py)."""
from __future__ import annotations

import numpy as np
import pytest

import crafted

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("search_form")]


def _both(cb, q, K, beam):
    from flashgann_amd import Index
    from oracle import oracle as O
    ix = Index.from_codebook(cb)
    ids, _, cnt = ix.search(q, K, beam, counters=True)
    ix.close()
    rids, rcnt = O.OracleIndex.from_codebook(cb).search(q, K, beam)
    return ids, cnt, rids, rcnt.view(np.uint32).reshape(-1, 6)


@pytest.mark.parametrize("beam", [931, 1000, 1024])
def test_line_search_at_iteration_cap(gpu_available, beam):
    """max_iter = (11 beam + 9)/10 exceeds 1024 here, so every query runs all
    1024 iterations and the last iteration's candidates are merged after the
    loop (adaptive_search.cuh:449-451).  They hold the best ids found, so a
    missing final merge changes every query's top-K."""
    cb, q, _ = crafted.line_index()
    ids, cnt, rids, rcnt = _both(cb, q, 10, beam)
    assert (cnt[:, 0] == 1024).all() and (rcnt[:, 0] == 1024).all()
    assert np.array_equal(cnt, rcnt)
    assert np.array_equal(ids, rids)


@pytest.mark.parametrize("beam", [100, 930])
def test_line_search_at_max_iter(gpu_available, beam):
    """Below the cap the search stops at max_iter, after that iteration's merge."""
    cb, q, _ = crafted.line_index()
    ids, cnt, rids, rcnt = _both(cb, q, 10, beam)
    assert (cnt[:, 0] == (11 * beam + 9) // 10).all()
    assert np.array_equal(cnt, rcnt) and np.array_equal(ids, rids)


@pytest.mark.parametrize("name,K,beam,want", [
    ("scenario_cutoff", 2, 3, [5, 9]),
    ("scenario_stage2", 10, 64, [0, 1, 2, 3, 4, 5, 6, 10, 12, 14]),
    ("scenario_stage2_cutoff", 8, 8, [0, 1, 2, 3, 4, 5, 6, 30]),
    ("scenario_reset", 16, 16, [36, 35, 34, 33, 32, 31, 30, 29, 29, 28, 27, 26, 25, 24, 23, 22]),
    ("scenario_short_graph", 8, 8, [1, 2, 0] + [0x7FFFFFFF] * 5),
    ("scenario_short_graph", 4, 2, [1, 2, 2, 2]),
    ("scenario_stage2_parents", 8, 8, [0, 1, 31, 2, 41, 3, 50, 51]),
    ("scenario_wide_degree", 12, 64, [0, 1, 2, 3, 4, 5, 6, 7, 8, 21, 0x7FFFFFFF, 0x7FFFFFFF]),
    ("scenario_wide_degree_codes", 12, 64, [0, 1, 2, 3, 4, 5, 6, 7, 8, 21, 0x7FFFFFFF, 0x7FFFFFFF]),
    ("scenario_task_order", 44, 64, [0] + list(range(1, 12)) + list(range(20, 52))),
    ("scenario_out_of_range_ids", 10, 64, [0, 1, 2, 3, 4, 5, 6, 11, 9, 13]),
    ("scenario_shared_child", 10, 64, [0, 1, 2, 3, 4, 5, 6, 30, 31, 32]),
])
def test_hand_traced_scenarios(gpu_available, name, K, beam, want):
    cb, q = getattr(crafted, name)()
    ids, cnt, rids, rcnt = _both(cb, q, K, beam)
    assert ids[0].tolist() == want
    assert np.array_equal(ids, rids) and np.array_equal(cnt, rcnt)


def test_complete_graph_brute_force(gpu_available):
    cb, q, base = crafted.complete_graph()
    d = ((q[:, None, :].astype(np.float64) - base[None]) ** 2).sum(-1)
    gt = np.lexsort((np.broadcast_to(np.arange(base.shape[0]), d.shape), d), axis=1)[:, :10]
    ids, cnt, rids, rcnt = _both(cb, q, 10, 64)
    assert np.array_equal(ids, gt)
    assert np.array_equal(ids, rids) and np.array_equal(cnt, rcnt)


@pytest.mark.parametrize("beam", [256, 512, 1024])
def test_random_graph_nearly_full_visited_set(gpu_available, beam):
    """Random links and K = beam: the visited set comes within a few keys of
    the worst case the table is sized for (test_oracle_search checks the fill
    on the oracle's traces); ids and work counters equal the oracle's."""
    cb, q, _ = crafted.random_graph_index()
    ids, cnt, rids, rcnt = _both(cb, q, beam, beam)
    assert np.array_equal(cnt, rcnt)
    assert np.array_equal(ids, rids)
