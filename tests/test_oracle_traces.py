"""Pins for the oracle's controller and search-loop sequencing.

The expected values below are worked out by hand from the reference's rules
(the derivation is in each docstring), not recomputed with the oracle's
formulas: the controller (src/adaptive_search_utils.cuh:32-135), the K-th
cutoff (:25-30), the loop order of src/adaptive_search.cuh:126-215 (reset and
restore, then the merge, then cutoff, controller, pick), the near count and
keep rules (:281-302, :397-404), max_iter (gpu_search_adaptive.cu:96) and the
final merge (adaptive_search.cuh:449-451).  The hand-built codebooks are in
tests/crafted.py.
"""
from __future__ import annotations

import numpy as np
import pytest

import crafted
from oracle import oracle as O

FLT_MAX = float(np.finfo(np.float32).max)
MSB = 0x80000000


def _ctl(entry):
    st = O.CtlState()
    O.lib().fgo_ctl_init(O.C.byref(st), entry)
    return st


def _step(st, beam0, rho2):
    O.lib().fgo_controller_step(O.C.byref(st), beam0, rho2)
    return st.spec_degree, st.rho, st.top1_stall_iters


def _record(st, dists):
    a = np.asarray(dists, np.float32)
    O.lib().fgo_record_expander(O.C.byref(st), O.ptr(a, O.C.c_float), len(a))
    return st.last_expander_distance, st.current_expander_distance


def test_controller_trajectory_degree32():
    """Degree 32: phase-2 rate 1 - 4/32 = 0.875, stage-I span 0.875 - 0.25 =
    0.625.  Entry distance 1000.
      step 0 (top-1 5): first update, rate 0.25, stall 0; expander at 900
      step 1 (top-1 7): progress (1000 - 900)/1000 = 0.1 -> 0.25 + 0.0625 = 0.3125
      step 2 (top-1 7, stall 1): expander 850 recorded after step 1, progress
             (900 - 850)/1000 = 0.05 -> 0.34375
      step 3 (stall 2): expander 850 again, progress 0 -> 0.34375
      step 4 (stall 3): expander 800, progress 0.05 -> 0.375
      step 5 (stall 4): stage II, theta 8, rate 0.875
      then the three expanders 100, 200, 300: the LAST one (300) is recorded
      step 6 (top-1 9): stall back to 0 but stage II sticks."""
    st = _ctl(1000.0)
    assert _step(st, 5, 0.875) == (1, 0.25, 0)
    assert _record(st, [900]) == (1000.0, 900.0)
    th, rho, stall = _step(st, 7, 0.875)
    assert (th, stall) == (1, 0) and rho == pytest.approx(0.3125, abs=1e-6)
    assert _record(st, [850]) == (900.0, 850.0)
    th, rho, stall = _step(st, 7, 0.875)
    assert (th, stall) == (1, 1) and rho == pytest.approx(0.34375, abs=1e-6)
    _record(st, [850])
    th, rho, stall = _step(st, 7 | MSB, 0.875)  # the expanded flag is masked off
    assert (th, stall) == (1, 2) and rho == pytest.approx(0.34375, abs=1e-6)
    _record(st, [800])
    th, rho, stall = _step(st, 7, 0.875)
    assert (th, stall) == (1, 3) and rho == pytest.approx(0.375, abs=1e-6)
    _record(st, [2000])
    assert _step(st, 7, 0.875) == (8, 0.875, 4)
    assert st.warmup_done == 1
    assert _record(st, [100, 200, 300]) == (2000.0, 300.0)
    assert _step(st, 9, 0.875) == (8, 0.875, 0)
    assert st.policy_iters == 7


def test_controller_small_degree_span_and_cap():
    """Degree <= 4: phase-2 rate 0 (RHO_MIN), so the span and the cap are
    RHO_MAX - RHO_MIN = 0.99.  Entry 100, expanders 100 then 40: progress
    0.6 -> 0.25 + 0.594 = 0.844; then 40 -> 0 (progress 0.4): 0.844 + 0.396
    is clamped to 0.99."""
    st = _ctl(100.0)
    _step(st, 1, 0.0)
    _record(st, [100])
    _step(st, 2, 0.0)
    _record(st, [40])
    assert _step(st, 3, 0.0)[1] == pytest.approx(0.844, abs=1e-6)
    _record(st, [0])
    assert _step(st, 4, 0.0)[1] == pytest.approx(0.99, abs=1e-7)


def test_controller_progress_guards():
    """Progress is 0 when it would be negative, and when the entry distance
    is 0 (|entry| <= 1e-20) or not finite: the rate then stays where it is.
    Entry 100, expanders 50 then 80: step 2 moves the rate by 0.625 * 0.5 to
    0.5625, step 3 (progress -0.3) keeps it.  Entries 0 and inf never move it
    from 0.25."""
    for entry, exps, r2 in ((100.0, [50, 80], 0.5625), (0.0, [0, -5], 0.25), (float("inf"), [3, 1], 0.25)):
        st = _ctl(entry)
        _step(st, 1, 0.875)
        _record(st, [exps[0]])
        assert _step(st, 2, 0.875)[1] == r2, entry
        _record(st, [exps[1]])
        assert _step(st, 3, 0.875)[1] == r2, entry


def test_kth_cutoff_position():
    """Valid only once the beam's last slot holds an id; then the distance at
    position min(K, beam) - 1."""
    L = O.lib()
    idx = np.array([3, 4, 5, 6, 0xFFFFFFFF], np.uint32)
    d = np.array([1, 2, 3, 4, FLT_MAX], np.float32)
    u32, f32 = O.C.c_uint32, O.C.c_float
    assert L.fgo_kth_cutoff(2, 5, O.ptr(idx, u32), O.ptr(d, f32)) == FLT_MAX
    assert L.fgo_kth_cutoff(2, 4, O.ptr(idx, u32), O.ptr(d, f32)) == 2.0
    assert L.fgo_kth_cutoff(3, 4, O.ptr(idx, u32), O.ptr(d, f32)) == 3.0
    assert L.fgo_kth_cutoff(10, 4, O.ptr(idx, u32), O.ptr(d, f32)) == 4.0
    idx[1] |= MSB  # expanded entries count as filled
    assert L.fgo_kth_cutoff(1, 2, O.ptr(idx, u32), O.ptr(d, f32)) == 1.0


def _trace(cb, q, K, beam):
    out, cnt, tr = O.OracleIndex.from_codebook(cb).search_one(q[0], K, beam, trace_cap=1100)
    c = tuple(getattr(cnt, f) for f, _ in O.Counters._fields_)
    recs = []
    for t in tr:
        ids = [t.cand_idx[i] for i in range(t.n_cand) if t.cand_idx[i] != 0xFFFFFFFF]
        ds = [t.cand_dist[i] for i in range(t.n_cand) if t.cand_idx[i] != 0xFFFFFFFF]
        recs.append(dict(theta=t.theta, rho=t.rho, parents=list(t.parents)[: t.n_parents],
                         top1=t.top1 & ~MSB, kth=t.kth_cutoff, cand=ids, cdist=ds, stall=t.stall,
                         last=t.last_expander_distance, cur=t.current_expander_distance,
                         restored=t.restored))
    return out.tolist(), c, recs


def test_trace_cutoff_and_near_count():
    """Degree 4 (span and cap 0.99), beam 3 (max_iter (33 + 9)/10 = 4), K 2.
      it 0: expand 0 (d 100); keep ceil(4 * 0.75) = 3 of 4 valid, so all four
            are estimated (36, 49, 64, 81) and 1, 2, 3 scored in estimate
            order.  The beam was not full: no cutoff.
      it 1: beam [1:36, 2:49, 3:64] is full, cutoff = beam[K-1] = 49.  Expand
            1; its children are estimated at 25, 49 (node 6, truly at 40), 50,
            80.  Near count (estimate <= 49) = 2, so 2 are kept: 5 and 6.
      it 2: beam [5:25, 1:36, 6:40], cutoff 36; progress (100 - 36)/100 = 0.64,
            rate 0.25 + 0.99 * 0.64 = 0.8836.  Expand 5: all its children
            are visited (the keep-all shortcut: no estimates).
      it 3: progress (36 - 25)/100 = 0.11: 0.8836 + 0.1089 is capped at 0.99;
            keep ceil(4 * 0.01) = 1.  Expand 6 (top-1 5 again: stall 1);
            children 9 (est 30) and 10 (est 45) are estimated, one kept: 9.
      it 4: the iteration limit; the final merge puts 9 at rank 2.
    Counters: 4 iterations, 4 expansions, 16 ids, 4 + 4 + 2 estimates,
    1 + 3 + 2 + 1 exact distances."""
    cb, q = crafted.scenario_cutoff()
    out, cnt, tr = _trace(cb, q, 2, 3)
    assert out == [5, 9]
    assert cnt == (4, 4, 16, 10, 7, 0xFFFFFFFF)
    assert [t["parents"] for t in tr] == [[0], [1], [5], [6]]
    assert [t["kth"] for t in tr] == [FLT_MAX, 49.0, 36.0, 36.0]
    assert [t["cand"] for t in tr] == [[1, 2, 3], [5, 6], [], [9]]
    assert [t["cdist"] for t in tr] == [[36, 49, 64], [25, 40], [], [30]]
    assert [t["top1"] for t in tr] == [0, 1, 5, 5]
    assert [t["stall"] for t in tr] == [0, 0, 0, 1]
    assert np.allclose([t["rho"] for t in tr], [0.25, 0.25, 0.8836, 0.99], atol=1e-6)
    assert [(t["last"], t["cur"]) for t in tr] == [(100, 100), (100, 36), (36, 25), (25, 40)]
    assert all(t["theta"] == 1 for t in tr)


def test_trace_stage2_switch_and_keep():
    """Degree 8 (phase-2 rate 0.5), beam 64 (never full: no cutoff), K 10.
      it 0: expand the entry 0 (d 1, top-1 for good); keep ceil(8 * 0.75) = 6
            of its 8 children (10 .. 80): 1 .. 6 are scored.
      it 1-3: expand 1, 2, 3 (dead ends); the top-1 stalls 1, 2, 3 times and
            progress is negative (expanders get farther), so the rate stays 0.25.
      it 4: fourth stall: theta 8, rate 0.5.  The unexpanded entries are 4, 5,
            6: three tasks.  Keep min(ceil(8 * 0.5), 32 / 8) = 4 per parent.
            The slots of 4 and 5 hold estimate ranks 8 1 7 2 6 3 5 4, so their
            kept lanes are 1, 3, 5, 7: 10 12 14 16 | 18 20 22 24 (distances
            base + 10 .. + 40 for bases 100, 200).  Parent 6 has 5 fresh
            children (ranks 5 1 4 2 3 in slots 0 2 4 6 7): 5 > 4, so all 5 are
            estimated and the four best kept, listed in lane order 26 27 28 29
            (310, 340, 320, 330).
      it 5: the first 8 of those 12 in beam order; it 6: the other 4 in beam
            order (26, 28, 29, 27); it 7 finds nothing to expand.
    Counters: 7 iterations, 1+1+1+1+3+8+4 = 19 expansions, 4 * 8 + 24 + 64 +
    32 = 152 ids, 8 + 8 + 8 + 5 estimates, 1 + 6 + 12 exact distances, stage
    II from iteration 4."""
    cb, q = crafted.scenario_stage2()
    out, cnt, tr = _trace(cb, q, 10, 64)
    assert out == [0, 1, 2, 3, 4, 5, 6, 10, 12, 14]
    assert cnt == (7, 19, 152, 29, 19, 4)
    assert [t["theta"] for t in tr] == [1, 1, 1, 1, 8, 8, 8]
    assert [t["stall"] for t in tr] == [0, 1, 2, 3, 4, 5, 6]
    assert np.allclose([t["rho"] for t in tr], [0.25] * 4 + [0.5] * 3)
    assert [t["parents"] for t in tr] == [[0], [1], [2], [3], [4, 5, 6],
                                         [10, 12, 14, 16, 18, 20, 22, 24], [26, 28, 29, 27]]
    assert tr[0]["cand"] == [1, 2, 3, 4, 5, 6]
    assert tr[4]["cand"] == [10, 12, 14, 16, 18, 20, 22, 24, 26, 27, 28, 29]
    assert tr[4]["cdist"] == [110, 120, 130, 140, 210, 220, 230, 240, 310, 340, 320, 330]
    assert all(t["kth"] == FLT_MAX for t in tr)
    # the last selected expander's distance is the one recorded
    assert (tr[4]["cur"], tr[5]["cur"], tr[6]["cur"]) == (60.0, 240.0, 340.0)


def test_trace_stage2_cutoff_near_count():
    """Degree 8, beam 8 (max_iter 9), K 8: the cutoff is beam[7].
      it 0: expand 0 (top-1 for good): 1 .. 6 scored (keep 6 of 8).
      it 1: beam [0 .. 6] is not full.  Expand 1: its two children 9 (500)
            and 10 (510) are both kept (2 <= 6).
      it 2: beam [0 .. 6, 9] is full: cutoff 500.  2 and 3 (it 3) are dead ends.
      it 4: fourth stall, stage II over the unexpanded 4, 5, 6, 9.  Only 4 has
            fresh children, estimated 400, 500, 600 .. 1100: near count
            (estimate <= 500) 2, so min(2, 4) = 2 are kept: 30 (400) and 31
            (estimated 500, truly 450).
      it 5: beam [0 .. 6, 30] (31 and 9 fall out), cutoff 400; expand 30, a
            dead end; it 6 finds nothing to expand.
    Counters: 6 iterations, 1+1+1+1+4+1 = 9 expansions, 4 * 8 + 4 * 8 + 8 = 72
    ids, 8 + 8 estimates, 1 + 6 + 2 + 2 exact distances."""
    cb, q = crafted.scenario_stage2_cutoff()
    out, cnt, tr = _trace(cb, q, 8, 8)
    assert out == [0, 1, 2, 3, 4, 5, 6, 30]
    assert cnt == (6, 9, 72, 16, 11, 4)
    assert [t["parents"] for t in tr] == [[0], [1], [2], [3], [4, 5, 6, 9], [30]]
    assert [t["kth"] for t in tr] == [FLT_MAX, FLT_MAX, 500.0, 500.0, 500.0, 400.0]
    assert [t["cand"] for t in tr] == [[1, 2, 3, 4, 5, 6], [9, 10], [], [], [30, 31], []]
    assert tr[4]["cdist"] == [400.0, 450.0]
    assert [t["theta"] for t in tr] == [1, 1, 1, 1, 8, 8]


def test_trace_reset_readmits_pending_sibling():
    """Degree-3 path (i -> i+1, i+2, i-1; distance 10000 - 10 i), beam 16,
    K 16: iteration k expands node 2k and scores 2k+1, 2k+2 (2k-1 is
    visited).  max_iter = (176 + 9)/10 = 18.  At iteration 15 the visited set
    is rebuilt from the beam before the merge, so 29 and 30 (scored at
    iteration 14) are not in it: expanding 30 admits 29 a second time.  The
    final beam holds 29 twice.  No estimates (keep ceil(3 (1 - rate)) = 3
    while the rate stays below 1/3), 1 + 2 * 18 + 1 exact distances."""
    cb, q = crafted.scenario_reset()
    out, cnt, tr = _trace(cb, q, 16, 16)
    assert out == [36, 35, 34, 33, 32, 31, 30, 29, 29, 28, 27, 26, 25, 24, 23, 22]
    assert cnt == (18, 18, 54, 0, 38, 0xFFFFFFFF)
    assert [t["parents"] for t in tr] == [[2 * k] for k in range(18)]
    assert [t["restored"] for t in tr] == [1 if k == 15 else 0 for k in range(18)]
    for k, t in enumerate(tr):
        want = [31, 32, 29] if k == 15 else [2 * k + 1, 2 * k + 2]
        assert t["cand"] == want, k


def test_complete_graph_beam_covers_all_is_brute_force():
    """On a complete graph with beam >= n every node is scored exactly and
    never evicted, so the result is the brute-force top-K (distinct integer
    distances).  The searches end before the first visited-set rebuild
    (iteration 15), so no node is admitted twice."""
    cb, q, base = crafted.complete_graph()
    d = ((q[:, None, :].astype(np.float64) - base[None]) ** 2).sum(-1)
    gt = np.lexsort((np.broadcast_to(np.arange(base.shape[0]), d.shape), d), axis=1)[:, :10]
    ids, cnt = O.OracleIndex.from_codebook(cb).search(q, 10, 64)
    assert (cnt["iterations"] < 15).all()
    for i in range(q.shape[0]):
        ds = np.sort(d[i])
        assert ds[9] < ds[10], "ties at the K-th place"
    assert np.array_equal(ids, gt)


@pytest.mark.parametrize("beam", [1, 16, 64, 100, 128, 256, 930, 931, 1000, 1024])
def test_line_iterations_and_final_merge(beam):
    """A search on the line never runs out of unexpanded entries, so it runs
    exactly min((11 beam + 9)/10, 1024) iterations.  Whatever stops it, the
    last iteration's candidates are merged: the result's distances are the K
    smallest of all exact distances the search computed (the beam keeps the
    best `beam` of everything merged, and K <= beam)."""
    cb, q, base = crafted.line_index()
    oix = O.OracleIndex.from_codebook(cb)
    K = min(10, beam)
    for qi in range(2):
        out, cnt, tr = oix.search_one(q[qi], K, beam, trace_cap=1100)
        assert cnt.iterations == min((11 * beam + 9) // 10, 1024)
        seen = [float(((base[0] - q[qi]) ** 2).sum())]
        for t in tr:
            seen += [t.cand_dist[i] for i in range(32) if t.cand_idx[i] != 0xFFFFFFFF]
        got = np.sort(((base[out.astype(np.int64)] - q[qi]) ** 2).sum(-1))
        assert np.array_equal(got, np.sort(np.asarray(seen, np.float32))[:K]), (beam, qi)


def test_trace_result_writer_empty_slots():
    """adaptive_search.cuh:455-464 masks the expanded flag off a beam slot
    BEFORE testing it against MAX_INDEX, so a slot that never held an id
    (0xFFFFFFFF) is written as 0x7FFFFFFF; only positions at or past the beam
    repeat the last id written.  Degree 2: cbs = 16, keep ceil(2 * 0.75) = 2
    takes both of the entry's children without estimates.
      beam 8, K 8: it 0 expands 0 and scores 1 (36), 2 (49); it 1 and 2
            expand 1 and 2 (children visited); it 3 has nothing to expand.
            The beam holds 1, 2, 0 and five empty slots.
      beam 2, K 4: the same three iterations (max_iter (22 + 9)/10 = 3); the
            beam keeps 1, 2 and positions 2, 3 repeat 2.
    Counters: 3 iterations, 3 expansions, 3 x 2 ids, no estimates, 1 + 2
    exact distances."""
    cb, q = crafted.scenario_short_graph()
    out, cnt, tr = _trace(cb, q, 8, 8)
    assert out == [1, 2, 0] + [0x7FFFFFFF] * 5
    assert cnt == (3, 3, 6, 0, 3, 0xFFFFFFFF)
    assert [t["parents"] for t in tr] == [[0], [1], [2]]
    out, cnt, tr = _trace(cb, q, 4, 2)
    assert out == [1, 2, 2, 2]
    assert cnt == (3, 3, 6, 0, 3, 0xFFFFFFFF)
    assert [t["kth"] for t in tr] == [FLT_MAX, 49.0, 49.0]


def test_trace_stage2_parent_distance_lane_tie_and_keep_all():
    """Degree 8, beam 8, K 8 (crafted.scenario_stage2_parents).
      it 0-3: as in scenario_stage2_cutoff: 1 .. 6 scored, then 9 (500) and
            10 (510); 2 and 3 are dead ends; the cutoff is 500 from it 2.
      it 4: fourth stall: stage II over 4 (40), 5 (50), 6 (60), 9 (500), keep
            min(ceil(8 * 0.5), 32 / 8) = 4 per parent.
            parent 4: no fresh child (keep-all, nothing estimated);
            parent 5: estimates from ITS distance (adaptive_search.cuh:394):
              420, 490, 505, 600 .. 1000; near count (<= 500) 2: keep 30, 31;
            parent 6: all 8 estimated above 500 (near count 0, keep
              clamp(0, 1, 4) = 1); the minimum 650 is tied between lanes 1
              (41) and 3 (43): the lower lane wins (utils.cuh:261);
            parent 9: 4 fresh children = the keep, so all four are admitted
              unestimated (`keep >= valid`, adaptive_search.cuh:387).
            Compacted in (task, lane) order: 30 31 41 50 51 52 53, scored at
            420, 15, 25, 35, 36, 37, 38.
      it 5: beam [0, 1, 31, 2, 41, 3, 50, 51], cutoff 36; the four new
            entries are dead ends.  it 6 finds nothing to expand.
    Counters: 6 iterations, 1+1+1+1+4+4 = 12 expansions, 4 x 8 + 8 x 8 = 96
    ids, 8 + 8 + 8 estimates, 1 + 6 + 2 + 7 exact distances, stage II from
    iteration 4."""
    cb, q = crafted.scenario_stage2_parents()
    out, cnt, tr = _trace(cb, q, 8, 8)
    assert out == [0, 1, 31, 2, 41, 3, 50, 51]
    assert cnt == (6, 12, 96, 24, 16, 4)
    assert [t["parents"] for t in tr] == [[0], [1], [2], [3], [4, 5, 6, 9], [31, 41, 50, 51]]
    assert [t["kth"] for t in tr] == [FLT_MAX, FLT_MAX, 500.0, 500.0, 500.0, 36.0]
    assert tr[4]["cand"] == [30, 31, 41, 50, 51, 52, 53]
    assert tr[4]["cdist"] == [420, 15, 25, 35, 36, 37, 38]
    assert tr[5]["cand"] == []


def test_trace_wide_degree_tiles():
    """Degree 40, beam 64 (never full: no cutoff), K 12
    (crafted.scenario_wide_degree).
      it 0: one expander reads min(40, cbs 32) = 32 slots
            (adaptive_search.cuh:222): 1 .. 8 are found (keep ceil(32 * 0.75)
            = 24 >= 8: all scored); node 9 in slot 35 is never read.
      it 1-3: 1, 2, 3 are dead ends; top-1 0 stalls 1, 2, 3 times.
      it 4: stage II, rate 1 - 4/40 = 0.9, parents 4 .. 8, two tiles each: 10
            tasks in two rounds.  A full tile keeps min(ceil(32 * 0.1), 4) =
            4, the 8-slot second tile min(ceil(8 * 0.1), 4) = 1
            (adaptive_search.cuh:380-382): of parent 4's fresh 20, 21, 22
            (slots 32-34, estimated 200, 150, 300) only 21 is kept.
      it 5: expand 21 (a dead end); it 6 finds nothing.
    The beam holds 10 ids: positions 10 and 11 are empty slots (0x7FFFFFFF).
    Counters: 6 iterations, 1+1+1+1+5+1 = 10 expansions, 4 x 32 + 6 x 40 =
    368 ids, 3 estimates, 1 + 8 + 1 exact distances."""
    cb, q = crafted.scenario_wide_degree()
    out, cnt, tr = _trace(cb, q, 12, 64)
    assert out == [0, 1, 2, 3, 4, 5, 6, 7, 8, 21, 0x7FFFFFFF, 0x7FFFFFFF]
    assert cnt == (6, 10, 368, 3, 10, 4)
    assert [t["parents"] for t in tr] == [[0], [1], [2], [3], [4, 5, 6, 7, 8], [21]]
    assert tr[0]["cand"] == [1, 2, 3, 4, 5, 6, 7, 8]
    assert tr[4]["cand"] == [21] and tr[4]["cdist"] == [150]
    assert np.allclose([t["rho"] for t in tr[4:]], [0.9, 0.9])


def test_trace_task_order_and_collect_cap():
    """Degree 40, beam 64, K 44 (crafted.scenario_task_order).
      it 0: the entry's 11 neighbours (keep ceil(32 * 0.75) = 24 >= 11: all).
      it 1-3: 1, 2, 3 are dead ends; top-1 0 stalls 1, 2, 3 times.
      it 4: stage II (rate 1 - 4/40 = 0.9), parents 4 .. 11, two tiles each:
            16 tasks, parent by parent (adaptive_search.cuh:351-354), in
            two rounds of 8.  A first tile keeps min(ceil(32 * 0.1), 32 / 8)
            = 4 >= its 4 children and the 8-slot second tile min(ceil(8 *
            0.1), 4) = 1 >= its 1: every child is kept, 40 in all.  The first
            task round (parents 4-7, both tiles) collects 20 .. 39, including the second
            tiles' 24, 29, 34, 39, whatever order its warps take (20 <= 32
            slots); tasks taken tile by tile would fill all 32 slots with
            first tiles in the first task round instead.  The second (parents 8-11) has 12
            slots for its 20 children: in the reference its warps race for
            them, here they go in (task, lane) order, the oracle's stated
            rule: 40 .. 49 (parents 8, 9) and the first two of parent 10's
            first tile, 50 and 51; 52 .. 59 are inserted but never scored.
      it 5-8: the 32 children, eight per iteration, all dead ends; it 9
            finds nothing to expand.
    Counters: 9 iterations, 1+1+1+1+8+32 = 44 expansions, 4 x 32 + 40 x 40
    = 1,728 ids, no estimates, 1 + 11 + 32 = 44 exact distances, stage II
    from iteration 4."""
    cb, q = crafted.scenario_task_order()
    out, cnt, tr = _trace(cb, q, 44, 64)
    assert out == [0] + list(range(1, 12)) + list(range(20, 52))
    assert cnt == (9, 44, 1728, 0, 44, 4)
    assert [t["parents"] for t in tr[:5]] == [[0], [1], [2], [3], list(range(4, 12))]
    assert [t["theta"] for t in tr] == [1, 1, 1, 1, 8, 8, 8, 8, 8]
    assert set(range(20, 40)) <= set(tr[4]["cand"])  # first task round, in any order of its warps
    assert tr[4]["cand"] == list(range(20, 52))  # second task round in (task, lane) order
    assert [t["parents"] for t in tr[5:]] == [list(range(20 + 8 * i, 28 + 8 * i)) for i in range(4)]


def test_controller_stage1_rate_capped_at_phase2_rate():
    """Degree 32 (phase-2 rate 0.875, span 0.625), entry 100, expanders 10,
    50, 10 (not monotone, as in a real search): progress 0.9 takes the rate to
    0.25 + 0.5625 = 0.8125, the rise to 50 adds nothing, the drop back to 10
    adds 0.625 * 0.4 = 0.25, and 1.0625 is clamped to the phase-2 rate 0.875
    (adaptive_search_utils.cuh:104-107), not to RHO_MAX 0.99."""
    st = _ctl(100.0)
    _step(st, 1, 0.875)
    _record(st, [10])
    assert _step(st, 2, 0.875)[1] == pytest.approx(0.8125, abs=1e-6)
    _record(st, [50])
    assert _step(st, 3, 0.875)[1] == pytest.approx(0.8125, abs=1e-6)
    _record(st, [10])
    th, rho, stall = _step(st, 4, 0.875)
    assert (th, stall) == (1, 0) and rho == np.float32(0.875)


def test_controller_unfinite_expander_distances_fall_back():
    """expander_progress (adaptive_search_utils.cuh:51-72): a current
    expander distance that is not finite (or FLT_MAX) falls back to the last
    one, and a last one that is not falls back to the entry distance;
    record_selected_expander_dist (:41-49) moves the current distance into
    `last`, or the entry distance when the current one is not finite.
    Entry 10, expanders 40 then FLT_MAX: at step 3 last = 40 and current
    falls back to 40, so progress is 0 and the rate stays 0.25 (falling back
    to the entry 10 would give progress 3 -> 1 and the rate 0.875)."""
    st = _ctl(10.0)
    _step(st, 1, 0.875)
    assert _record(st, [40]) == (10.0, 40.0)
    assert _step(st, 2, 0.875)[1] == 0.25
    assert _record(st, [FLT_MAX]) == (40.0, FLT_MAX)
    assert _step(st, 3, 0.875)[1] == 0.25
    assert (st.last_expander_distance, st.current_expander_distance) == (40.0, 40.0)
    fresh = _ctl(7.0)  # current is FLT_MAX before any step: last becomes the entry
    assert _record(fresh, [3]) == (7.0, 3.0)


def test_trace_out_of_range_ids_are_not_children():
    """Degree 8, beam 64, K 10 (crafted.scenario_out_of_range_ids; BAD_ID =
    40 with 15 nodes).
      it 0: the entry's 8 slots are read; 7 valid (BAD_ID is not: child_id
            >= npoints, adaptive_search.cuh:233), keep min(ceil(8 * 0.75),
            8) = 6 < 7: 7 estimates, 1 .. 6 kept (7 at 70 is not).
      it 1-3: 1, 2, 3 are dead ends; top-1 0 stalls 1, 2, 3 times.
      it 4: stage II, rate 1 - 4/8 = 0.5, parents 4, 5, 6.  Parent 4 lists
            BAD_ID (not valid, :372) and 8 .. 14: keep min(ceil(8 * 0.5),
            32 / 8) = 4 < 7: 7 estimates, the four smallest 11 (110), 9
            (120), 13 (130), 14 (140), listed in lane order 9, 11, 13, 14.
      it 5: parents 11, 9, 13, 14 (dead ends); it 6 finds nothing.
    Counters: 6 iterations, 1+1+1+1+3+4 = 11 expansions, 8 + 3 x 8 + 3 x 8 +
    4 x 8 = 88 ids, 7 + 7 = 14 estimates, 1 + 6 + 4 = 11 exact distances."""
    cb, q = crafted.scenario_out_of_range_ids()
    assert cb.rows.shape[0] < crafted.BAD_ID
    out, cnt, tr = _trace(cb, q, 10, 64)
    assert out == [0, 1, 2, 3, 4, 5, 6, 11, 9, 13]
    assert cnt == (6, 11, 88, 14, 11, 4)
    assert [t["parents"] for t in tr] == [[0], [1], [2], [3], [4, 5, 6], [11, 9, 13, 14]]
    assert tr[0]["cand"] == [1, 2, 3, 4, 5, 6]
    assert tr[4]["cand"] == [9, 11, 13, 14] and tr[4]["cdist"] == [120, 110, 130, 140]


def test_trace_wide_degree_estimates_read_their_own_slot():
    """crafted.scenario_wide_degree_codes: as test_trace_wide_degree_tiles,
    but parent 4's second-tile estimates come from the codes at slots 32-34
    (the code of neighbour slot nidx, adaptive_search.cuh:392-394).  By hand
    (the docstring of the scenario) they are 395.0, 5.0 and 200 for 20, 21
    and 22, so 21 is kept; an estimate read from slot l of the tile would
    give 20 the smallest (slot 0's zero code) and keep 20."""
    cb, q = crafted.scenario_wide_degree_codes()
    qf = O.query_prepare(q[0], cb.signs, 40, 64)
    assert (qf.sum_q, qf.low, qf.high) == (2048, 7.0, 13.0)
    assert list(qf.q[:4]) == [63, 1, 63, 1]
    lay = cb.layout
    codes = cb.rows[4, lay.code_offset:lay.factor_offset].view(np.uint8).reshape(lay.degree, -1)
    est = [O.lib().fgo_estimate_seq(O.C.byref(qf), O.ptr(np.ascontiguousarray(codes[s]), O.C.c_uint8),
                                     160.0, 1.0, 0.0, 40.0, 64) for s in (32, 33, 34)]
    w = np.float32(6.0) / np.float32(63.0)
    assert est == pytest.approx([200 + w * 2048, 200 - w * 2048, 200], abs=1e-3)
    out, cnt, tr = _trace(cb, q, 12, 64)
    assert out == [0, 1, 2, 3, 4, 5, 6, 7, 8, 21, 0x7FFFFFFF, 0x7FFFFFFF]
    assert cnt == (6, 10, 368, 3, 10, 4)
    assert tr[4]["cand"] == [21] and tr[4]["cdist"] == [150]


def test_trace_shared_child_first_task_keeps_it():
    """Degree 8, beam 64, K 10 (crafted.scenario_shared_child).
      it 0: the entry's 6 neighbours (keep ceil(8 * 0.75) = 6 >= 6: all).
      it 1-3: 1, 2, 3 are dead ends; top-1 0 stalls 1, 2, 3 times.
      it 4: stage II (rate 1 - 4/8 = 0.5), parents 4, 5, 6, one round.  Each
            task keeps min(ceil(8 * 0.5), 32 / 8) = 4 of its 8 valid
            children by estimate: parent 4 keeps 30 (150), 20, 21, 22, in
            lane order 20, 21, 22, 30; parent 5, which also sees 30 as
            unvisited (the set as it stood at the round's start), keeps 30,
            31 (170), 32, 33, in lane order 31, 30, 32, 33.  Inserts in
            (task, lane) order: parent 4's 30 goes in, parent 5's is a
            repeat and is dropped: candidates 20, 21, 22, 30, 31, 32, 33.
            (Seeing parent 4's inserts already would have kept 34 for
            parent 5; the later task winning would list 31, 30, ... first.)
      it 5: the seven children (dead ends); it 6 finds nothing.
    Counters: 6 iterations, 1+1+1+1+3+7 = 14 expansions, 4 x 8 + 3 x 8 +
    7 x 8 = 112 ids, 8 + 8 = 16 estimates, 1 + 6 + 7 = 14 exact distances."""
    cb, q = crafted.scenario_shared_child()
    out, cnt, tr = _trace(cb, q, 10, 64)
    assert out == [0, 1, 2, 3, 4, 5, 6, 30, 31, 32]
    assert cnt == (6, 14, 112, 16, 14, 4)
    assert [t["parents"] for t in tr[:5]] == [[0], [1], [2], [3], [4, 5, 6]]
    assert tr[4]["cand"] == [20, 21, 22, 30, 31, 32, 33]
    assert tr[5]["parents"] == [30, 31, 32, 33, 20, 21, 22]
