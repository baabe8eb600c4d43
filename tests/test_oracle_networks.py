"""Pins the oracle's sorting networks and merges.

The oracle states the reference's warp networks (include/utils.cuh:307-414) as
standard bitonic stages over positions.  Here the reference's own lane-level
procedure is replayed literally (32 lanes, per-lane shuffle rule, blocked
layout position = N*lane + i) and compared on inputs with many tied keys, so a
wrong direction bit, distance or tie rule in the restatement fails."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from oracle import oracle as O

FLT_MAX = np.float32(np.finfo(np.float32).max)
MAXI = 0xFFFFFFFF


def _shfl_swap(k, v, i, off, p):
    """swap_if_needed (utils.cuh:309-316) on item i of all 32 lanes at once."""
    nk = [row[:] for row in k]
    nv = [row[:] for row in v]
    for lane in range(32):
        k0, k1 = k[lane][i], k[lane ^ off][i]
        if k0 != k1 and ((k0 < k1) != p[lane]):
            nk[lane][i] = k1
            nv[lane][i] = v[lane ^ off][i]
    return nk, nv


def _reg_swap(k, v, lane, i, j, p):
    """swap_if_needed (utils.cuh:319-328) between items i < j of one lane."""
    if k[lane][i] != k[lane][j] and ((k[lane][i] < k[lane][j]) != p):
        k[lane][i], k[lane][j] = k[lane][j], k[lane][i]
        v[lane][i], v[lane][j] = v[lane][j], v[lane][i]


def ref_warp_merge(k, v, N, rng):
    """warp_merge_core<N> (utils.cuh:330-402), literally."""
    if N == 1:
        if rng == 1:
            return k, v
        b = rng
        c = b // 2
        while c >= 1:
            p = [bool(l & b) == bool(l & c) for l in range(32)]
            k, v = _shfl_swap(k, v, 0, c, p)
            c //= 2
        return k, v
    if N == 2:
        if rng == 1:
            for l in range(32):
                _reg_swap(k, v, l, 0, 1, (l & 1) == 0)
            return k, v
        b = rng
        c = b // 2
        while c >= 1:
            p = [bool(l & b) == bool(l & c) for l in range(32)]
            for i in range(2):
                k, v = _shfl_swap(k, v, i, c, p)
            c //= 2
        for l in range(32):
            _reg_swap(k, v, l, 0, 1, (l & b) == 0)
        return k, v
    if rng == 1:
        b = 2
        while b <= N:
            c = b // 2
            while c >= 1:
                for l in range(32):
                    for i in range(N):
                        j = i ^ c
                        if i >= j:
                            continue
                        line = i + N * l
                        _reg_swap(k, v, l, i, j, bool(line & b) == bool(line & c))
                c //= 2
            b *= 2
        return k, v
    b = rng
    c = b // 2
    while c >= 1:
        p = [bool(l & b) == bool(l & c) for l in range(32)]
        for i in range(N):
            k, v = _shfl_swap(k, v, i, c, p)
        c //= 2
    c = N // 2
    while c >= 1:
        for l in range(32):
            for i in range(N):
                j = i ^ c
                if i >= j:
                    continue
                _reg_swap(k, v, l, i, j, (l & b) == 0)
        c //= 2
    return k, v


def ref_warp_sort(k, v, N):
    rng = 1
    while rng <= 32:
        k, v = ref_warp_merge(k, v, N, rng)
        rng *= 2
    return k, v


def _blocked(keys, vals, N):
    k = [[keys[N * l + i] for i in range(N)] for l in range(32)]
    v = [[vals[N * l + i] for i in range(N)] for l in range(32)]
    return k, v


def _flat(k, v, N):
    return (np.array([k[l][i] for l in range(32) for i in range(N)], dtype=np.float32),
            np.array([v[l][i] for l in range(32) for i in range(N)], dtype=np.uint32))


def _oracle_sort(keys, vals):
    k = np.ascontiguousarray(keys, dtype=np.float32).copy()
    v = np.ascontiguousarray(vals, dtype=np.uint32).copy()
    O.lib().fgo_bitonic_sort(O.ptr(k, C.c_float), O.ptr(v, C.c_uint32), k.size)
    return k, v


@pytest.mark.parametrize("N", [1, 2, 4, 8])
@pytest.mark.parametrize("seed", range(6))
def test_warp_sort_matches_lane_replay(N, seed):
    rng = np.random.default_rng(100 * N + seed)
    n = 32 * N
    keys = rng.integers(0, 6, n).astype(np.float32)       # heavy ties
    keys[rng.random(n) < 0.2] = FLT_MAX
    vals = rng.permutation(n).astype(np.uint32)
    rk, rv = _flat(*ref_warp_sort(*_blocked(list(keys), list(vals), N), N), N)
    ok, ov = _oracle_sort(keys, vals)
    assert np.array_equal(rk, ok) and np.array_equal(rv, ov)
    assert np.all(np.diff(ok) >= 0)


def _same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


@pytest.mark.parametrize("N", [1, 2, 4])
@pytest.mark.parametrize("seed", range(4))
def test_warp_sort_with_nan_matches_lane_replay(N, seed):
    """NaN keys (rows of NaN in a codebook): each lane of a cross-lane
    compare-exchange decides on its own (utils.cuh:309-316), so a NaN can be
    dropped and its partner duplicated; the oracle must do the same."""
    rng = np.random.default_rng(500 + 10 * N + seed)
    n = 32 * N
    keys = rng.integers(0, 6, n).astype(np.float32)
    keys[rng.random(n) < 0.15] = np.nan
    keys[rng.random(n) < 0.1] = FLT_MAX
    vals = rng.permutation(n).astype(np.uint32)
    rk, rv = _flat(*ref_warp_sort(*_blocked(list(keys), list(vals), N), N), N)
    ok, ov = _oracle_sort(keys, vals)
    assert _same_bits(rk, ok) and np.array_equal(rv, ov)
    # the per-lane rule really is not a permutation here
    assert not np.array_equal(np.sort(rv), np.sort(vals)) or seed > 0


@pytest.mark.parametrize("N", [1, 2, 4])
def test_final_merge_stage_matches_lane_replay(N):
    rng = np.random.default_rng(7 + N)
    n = 32 * N
    for _ in range(5):
        half = n // 2
        a = np.sort(rng.integers(0, 8, half)).astype(np.float32)
        b = np.sort(rng.integers(0, 8, n - half))[::-1].astype(np.float32)
        keys = np.concatenate([a, b])
        vals = rng.permutation(n).astype(np.uint32)
        rk, rv = _flat(*ref_warp_merge(*_blocked(list(keys), list(vals), N), N, 32), N)
        k = keys.copy()
        v = vals.copy()
        O.lib().fgo_bitonic_stage(O.ptr(k, C.c_float), O.ptr(v, C.c_uint32), n, n)
        assert np.array_equal(rk, k) and np.array_equal(rv, v)


def _ref_small_merge(beam_d, beam_i, cand_d, cand_i, cbs, pbeam, first):
    """topk_small_by_bitonic_sort<1, pbeam/32> (utils.cuh:490-586), literally."""
    N2 = pbeam // 32
    k1 = [[float(cand_d[l]) if l < cbs else FLT_MAX] for l in range(32)]
    v1 = [[int(cand_i[l]) if l < cbs else MAXI] for l in range(32)]
    k1, v1 = ref_warp_sort(k1, v1, 1)
    cd, ci = list(cand_d), list(cand_i)
    for l in range(32):
        if l < cbs and l < pbeam:
            cd[l], ci[l] = k1[l][0], v1[l][0]
    if first:
        k2 = [[float(beam_d[l + 32 * i]) for i in range(N2)] for l in range(32)]
        v2 = [[int(beam_i[l + 32 * i]) for i in range(N2)] for l in range(32)]
        k2, v2 = ref_warp_sort(k2, v2, N2)
    else:
        k2 = [[float(beam_d[N2 * l + i]) for i in range(N2)] for l in range(32)]
        v2 = [[int(beam_i[N2 * l + i]) for i in range(N2)] for l in range(32)]
    for l in range(32):
        for i in range(N2):
            j = N2 * l + i
            kk = pbeam - 1 - j
            if kk >= pbeam or kk >= cbs:
                continue
            if k2[l][i] > cd[kk]:
                k2[l][i], v2[l][i] = cd[kk], ci[kk]
    k2, v2 = ref_warp_merge(k2, v2, N2, 32)
    return _flat(k2, v2, N2)


@pytest.mark.parametrize("pbeam", [32, 64, 128])
@pytest.mark.parametrize("first", [0, 1])
@pytest.mark.parametrize("cbs", [32, 16])
@pytest.mark.parametrize("nan", [False, True])
def test_small_merge_matches_lane_replay(pbeam, first, cbs, nan):
    rng = np.random.default_rng(pbeam + 3 * first + cbs + 7 * nan)
    L = O.lib()
    for _ in range(4):
        bd = np.sort(rng.integers(0, 10, pbeam)).astype(np.float32)
        bd[rng.random(pbeam) < 0.2] = FLT_MAX
        bd = np.sort(bd)
        if first:
            rng.shuffle(bd)
        bi = rng.permutation(1000)[:pbeam].astype(np.uint32)
        cd = rng.integers(0, 10, 32).astype(np.float32)
        if nan:
            cd[rng.random(32) < 0.2] = np.nan
            bd[rng.random(pbeam) < 0.1] = np.nan
        ci = (1000 + rng.permutation(100)[:32]).astype(np.uint32)
        rk, rv = _ref_small_merge(bd, bi, cd, ci, cbs, pbeam, first)
        b1, b2, c1, c2 = bd.copy(), bi.copy(), cd.copy(), ci.copy()
        sd = np.zeros(1024, np.float32)
        si = np.zeros(1024, np.uint32)
        L.fgo_merge_candidates(O.ptr(b1, C.c_float), O.ptr(b2, C.c_uint32), O.ptr(c1, C.c_float),
                               O.ptr(c2, C.c_uint32), cbs, pbeam, first, O.ptr(sd, C.c_float),
                               O.ptr(si, C.c_uint32))
        assert _same_bits(b1, rk) and np.array_equal(b2, rv)


def test_merge_path_distinct_keys_is_sorted_union():
    """Distinct keys: the merge-path variant returns the pbeam smallest of
    beam U candidates in order, for every reference segmentation."""
    rng = np.random.default_rng(3)
    L = O.lib()
    for pbeam in (129, 200, 256, 384, 640, 1000, 1024):
        allk = rng.permutation(5000).astype(np.float32)
        bd = np.sort(allk[:pbeam])
        cd = allk[pbeam : pbeam + 32].copy()
        bi = np.arange(pbeam, dtype=np.uint32)
        ci = np.arange(10000, 10032, dtype=np.uint32)
        ref = np.sort(np.concatenate([bd, cd]))[:pbeam]
        b1, b2 = bd.copy(), bi.copy()
        sd = np.zeros(1024, np.float32)
        si = np.zeros(1024, np.uint32)
        L.fgo_merge_candidates(O.ptr(b1, C.c_float), O.ptr(b2, C.c_uint32), O.ptr(cd, C.c_float),
                               O.ptr(ci, C.c_uint32), 32, pbeam, 0, O.ptr(sd, C.c_float),
                               O.ptr(si, C.c_uint32))
        assert np.array_equal(b1, ref)
        key_of = {**{int(i): float(k) for i, k in zip(bi, bd)}, **{int(i): float(k) for i, k in zip(ci, np.sort(cd))}}
        assert all(key_of[int(i)] == float(k) for i, k in zip(b2, b1))


@pytest.mark.parametrize("pbeam", [256, 384, 512, 1024])
def test_merge_path_ties_inside_segments_keep_beam_first(pbeam):
    """Keys tied between the beam and the candidates: the output loop takes
    the beam entry on `<=` (utils.cuh:656-661), so the result is the stable
    merge with beam entries before candidates of equal key.  At these beams
    the reference's segmentation gives every thread 4 outputs (ceil(pbeam/4)
    threads, at most 256), so each tie is placed strictly inside one group
    of 4 outputs with distinct keys on either side of every group boundary:
    the partitions at the boundaries are unique and only the `<=` decides.
    Group g of the output holds keys 10g, 10g+1, 10g+1, 10g+2; in 32 groups
    the tied pair is (beam, candidate), in the others (beam, beam), and in 8
    of the candidate groups a second beam entry shares the key (beam, beam,
    candidate over positions 1-3).  The 32 leftover beam entries sort after
    everything and drop out."""
    L = O.lib()
    groups = pbeam // 4
    cand_groups = set(range(1, groups, groups // 32))
    assert len(cand_groups) == 32
    triple = set(sorted(cand_groups)[::4])
    beam_k, cand_k, want = [], [], []  # want: (key, source) in output order
    for g in range(groups):
        k0, k1, k3 = 10 * g, 10 * g + 1, 10 * g + 2
        if g in triple:
            slots = [(k0, "b"), (k1, "b"), (k1, "b"), (k1, "c")]
        elif g in cand_groups:
            slots = [(k0, "b"), (k1, "b"), (k1, "c"), (k3, "b")]
        else:
            slots = [(k0, "b"), (k1, "b"), (k1, "b"), (k3, "b")]
        for k, src in slots:
            (beam_k if src == "b" else cand_k).append(k)
        want += slots
    beam_k += [100000 + i for i in range(pbeam - len(beam_k))]
    assert len(beam_k) == pbeam and len(cand_k) == 32
    for b in range(4, pbeam, 4):  # distinct keys across every group boundary
        assert want[b - 1][0] < want[b][0]
    bd = np.asarray(beam_k, np.float32)
    bi = np.arange(pbeam, dtype=np.uint32)
    rng = np.random.default_rng(pbeam)
    perm = rng.permutation(32)  # the candidate buffer arrives unsorted
    cd = np.asarray(cand_k, np.float32)[perm].copy()
    ci = (5000 + perm).astype(np.uint32)
    # expected ids: beam entries in beam order, candidates in key order
    nb = nc = 0
    want_ids = []
    for k, src in want:
        if src == "b":
            want_ids.append(nb)
            nb += 1
        else:
            want_ids.append(5000 + nc)
            nc += 1
    sd = np.zeros(1024, np.float32)
    si = np.zeros(1024, np.uint32)
    L.fgo_merge_candidates(O.ptr(bd, C.c_float), O.ptr(bi, C.c_uint32), O.ptr(cd, C.c_float),
                           O.ptr(ci, C.c_uint32), 32, pbeam, 0, O.ptr(sd, C.c_float), O.ptr(si, C.c_uint32))
    assert bd.tolist() == [float(k) for k, _ in want]
    assert bi.tolist() == want_ids


def _ref_partition(a, b, diag):
    """Brute force: the binary search of utils.cuh:588-616, unrolled."""
    na, nb = len(a), len(b)
    low, high = max(0, diag - nb), min(diag, na)
    while low <= high:
        ai = (low + high) >> 1
        bi = diag - ai
        al = a[ai - 1] if ai > 0 else -FLT_MAX
        ar = a[ai] if ai < na else FLT_MAX
        bl = b[bi - 1] if bi > 0 else -FLT_MAX
        br = b[bi] if bi < nb else FLT_MAX
        if al > br:
            high = ai - 1
        elif bl > ar:
            low = ai + 1
        else:
            return ai
    return low


def test_merge_path_partition_valid_split():
    rng = np.random.default_rng(11)
    L = O.lib()
    for _ in range(200):
        na = int(rng.integers(1, 300))
        a = np.sort(rng.integers(0, 20, na)).astype(np.float32)
        b = np.sort(rng.integers(0, 20, 32)).astype(np.float32)
        diag = int(rng.integers(0, na + 33))
        got = L.fgo_merge_path_partition(O.ptr(a, C.c_float), na, O.ptr(b, C.c_float), 32, diag)
        assert got == _ref_partition(list(a), list(b), diag)
        bi = diag - got
        # a valid merge split: everything left of it <= everything right of it
        left = np.concatenate([a[:got], b[:bi]])
        right = np.concatenate([a[got:], b[bi:]])
        if left.size and right.size:
            assert left.max() <= right.min()



def _ref_merge_path(bd, bi, cd, ci, pbeam, active):
    """The output loop of topk_candidate_sort_and_merge (utils.cuh:637-669)
    over `active` threads of a 256-thread block, candidates already sorted:
    thread t writes outputs [t pbeam / active, (t + 1) pbeam / active), each
    end located by the partition, the beam taken on `<=`."""
    od, oi = [0.0] * pbeam, [0] * pbeam
    for t in range(active):
        ob, oe = min(pbeam, t * pbeam // active), min(pbeam, (t + 1) * pbeam // active)
        tb, te = _ref_partition(bd, cd, ob), _ref_partition(bd, cd, oe)
        ti, c, cend = tb, ob - tb, oe - te
        for o in range(ob, oe):
            if c >= cend or (ti < te and bd[ti] <= cd[c]):
                od[o], oi[o] = bd[ti], bi[ti]
                ti += 1
            else:
                od[o], oi[o] = cd[c], ci[c]
                c += 1
    return od, oi


@pytest.mark.parametrize("pbeam", [129, 160, 200, 300, 513, 1000])
def test_merge_path_segmentation_with_boundary_ties(pbeam):
    """Keys tied between the beam and the candidates across segment
    boundaries: which thread takes which tied entry depends on where the
    segments start, so the ids' order pins the reference's segmentation,
    ceil(pbeam / 4) threads rounded up to a multiple of 32 and at most 256
    (utils.cuh:632-635).  Beam keys are integers with repeats, candidate keys
    distinct integers (so the candidate sort has no ties to place); each case
    is checked to come out differently with the unrounded thread count."""
    L = O.lib()
    rng = np.random.default_rng(pbeam)
    active = min(256, ((pbeam + 3) // 4 + 31) // 32 * 32)
    unrounded = (pbeam + 3) // 4
    assert active != unrounded
    differs = 0
    for trial in range(8):
        bd = np.sort(rng.integers(0, 60, pbeam)).astype(np.float32)
        bi = np.arange(pbeam, dtype=np.uint32)
        cs = np.sort(rng.choice(60, 32, replace=False)).astype(np.float32)
        perm = rng.permutation(32)
        cd = cs[perm].copy()
        ci = (5000 + perm).astype(np.uint32)
        want_d, want_i = _ref_merge_path(list(bd), list(bi), list(cs), list(range(5000, 5032)), pbeam, active)
        _, other_i = _ref_merge_path(list(bd), list(bi), list(cs), list(range(5000, 5032)), pbeam, unrounded)
        differs += other_i != want_i
        sd = np.zeros(1024, np.float32)
        si = np.zeros(1024, np.uint32)
        L.fgo_merge_candidates(O.ptr(bd, C.c_float), O.ptr(bi, C.c_uint32), O.ptr(cd, C.c_float),
                               O.ptr(ci, C.c_uint32), 32, pbeam, 0, O.ptr(sd, C.c_float), O.ptr(si, C.c_uint32))
        assert bd.tolist() == want_d, trial
        assert bi.tolist() == want_i, trial
    assert differs >= 1

@pytest.mark.parametrize("top", [8, 16])
def test_short_candidate_sort_equals_full_network(top):
    """A 32-entry candidate buffer whose slots from `span` on hold the reset
    pair (FLT_MAX, MAX_INDEX), with no key above FLT_MAX, sorts the same
    under the stages up to block size 8 / 16 as under the full 32-entry
    network (the kernel sorts such buffers with the shorter networks)."""
    rng = np.random.default_rng(top)
    fmax = np.finfo(np.float32).max
    for _ in range(3000):
        span = int(rng.integers(0, top + 1))
        k = np.full(32, fmax, np.float32)
        v = np.full(32, 0xFFFFFFFF, np.uint32)
        k[:span] = rng.integers(0, 5, span).astype(np.float32)  # heavy ties
        if span and rng.random() < 0.25:
            k[rng.integers(0, span)] = fmax  # a real child at exactly FLT_MAX
        v[:span] = rng.permutation(4096)[:span]
        k1, v1, k2, v2 = k.copy(), v.copy(), k.copy(), v.copy()
        O.lib().fgo_bitonic_sort(O.ptr(k1, C.c_float), O.ptr(v1, C.c_uint32), 32)
        O.lib().fgo_bitonic_sort(O.ptr(k2, C.c_float), O.ptr(v2, C.c_uint32), top)
        assert np.array_equal(k1, k2) and np.array_equal(v1, v2), (span, k, v)
    # an infinite key inside the span breaks the equivalence: the kernel
    # checks for it and falls back to the full network
    k = np.full(32, fmax, np.float32)
    v = np.full(32, 0xFFFFFFFF, np.uint32)
    k[:3] = [1.0, np.inf, 2.0]
    v[:3] = [7, 8, 9]
    k1, v1, k2, v2 = k.copy(), v.copy(), k.copy(), v.copy()
    O.lib().fgo_bitonic_sort(O.ptr(k1, C.c_float), O.ptr(v1, C.c_uint32), 32)
    O.lib().fgo_bitonic_sort(O.ptr(k2, C.c_float), O.ptr(v2, C.c_uint32), top)
    assert not (np.array_equal(k1, k2) and np.array_equal(v1, v2))


def _direct_split(a, b, d):
    """The kernel's direct split search (fg_search.hip merge_path): the last
    i in [max(d - nb, 0), min(d, na)] with a[i-1] <= b[d-i], by steps of
    32 .. 1 that test min(pos + step, hi), and whether the boundary pair
    a[r-1], b[d-r] ties below FLT_MAX."""
    na, nb = len(a), len(b)
    fa = lambda i: -FLT_MAX if i < 0 else (FLT_MAX if i >= na else a[i])
    fb = lambda j: -FLT_MAX if j < 0 else (FLT_MAX if j >= nb else b[j])
    lo0, hi = max(d - nb, 0), min(d, na)
    pos = lo0
    for step in (32, 16, 8, 4, 2, 1):
        c = min(pos + step, hi)
        assert -1 <= c - 1 < na and 0 <= d - c <= nb  # reads stay in range
        if fa(c - 1) <= fb(d - c):
            pos = c
    tie = pos > lo0 and fa(pos - 1) == fb(d - pos) and fa(pos - 1) != FLT_MAX
    return pos, tie


def _segmented_merge(ak, av, bk, bv, split):
    """topk_candidate_sort_and_merge's output loop (utils.cuh:618-680) with the
    reference block's segmentation, the split of each boundary from `split`."""
    pbeam = len(ak)
    active = min(256, ((pbeam + 3) // 4 + 31) // 32 * 32)
    ok, ov = [], []
    for t in range(active):
        ob, oe = min(pbeam, t * pbeam // active), min(pbeam, (t + 1) * pbeam // active)
        tb, te = split(ob), split(oe)
        ti, ci, ce = tb, ob - tb, oe - te
        for _ in range(ob, oe):
            if ci >= ce or (ti < te and ak[ti] <= bk[ci]):
                ok.append(ak[ti]); ov.append(av[ti]); ti += 1
            else:
                ok.append(bk[ci]); ov.append(bv[ci]); ci += 1
    return ok, ov


@pytest.mark.parametrize("pbeam", [256, 512, 1024])
def test_direct_split_search_equals_bisection(pbeam):
    """The kernel finds merge-path splits by a direct binary search and replays
    the reference's bisection only when a boundary pair ties below FLT_MAX.
    Without such a tie the merged beam must equal the reference's
    (fgo_merge_path_partition, the bisection of utils.cuh:588-616) -- also when
    empty (FLT_MAX, MAX_INDEX) entries tie, where the split index may differ.
    With ties the split can differ, so the guard is not vacuous."""
    rng = np.random.default_rng(pbeam)
    L = O.lib()
    fmax = float(FLT_MAX)
    clean = differ_when_tied = 0
    for case in range(120):
        span = [3, 40, 5000, 100000][case % 4]  # key range: heavy, some, few ties
        nfill = int(rng.integers(0, pbeam + 1))
        ak = np.full(pbeam, fmax, np.float32)
        av = np.full(pbeam, MAXI, np.uint32)
        ak[:nfill] = np.sort(rng.integers(0, span, nfill)).astype(np.float32)
        av[:nfill] = rng.permutation(1 << 20)[:nfill]
        nc = int(rng.integers(0, 33))
        bk = np.full(32, fmax, np.float32)
        bv = np.full(32, MAXI, np.uint32)
        bk[:nc] = np.sort(rng.integers(0, span, nc)).astype(np.float32)
        bv[:nc] = (1 << 21) + rng.permutation(1 << 20)[:nc]
        ref = lambda d: L.fgo_merge_path_partition(O.ptr(ak, C.c_float), pbeam, O.ptr(bk, C.c_float), 32, d)
        active = min(256, ((pbeam + 3) // 4 + 31) // 32 * 32)
        bounds = [min(pbeam, t * pbeam // active) for t in range(1, active + 1)]
        fast = {d: _direct_split(list(ak), list(bk), d) for d in bounds}
        tied = any(t for _, t in fast.values())
        got = _segmented_merge(list(ak), list(av), list(bk), list(bv),
                               lambda d: 0 if d == 0 else fast[d][0])
        want = _segmented_merge(list(ak), list(av), list(bk), list(bv), ref)
        if not tied:
            clean += 1
            assert got == want, (case, pbeam)
        elif got != want:
            differ_when_tied += 1
    assert clean > 30 and differ_when_tied > 0, (clean, differ_when_tied)
