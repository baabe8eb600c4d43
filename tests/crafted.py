"""Hand-built codebooks whose searches can be traced by hand.

Every edge u -> v carries factor_dq = factor_vq = 0 and an all-zero code, so
the search's RaBitQ estimate (include/utils.cuh:989-993)

    est = triple_x + d(q, u) + factor_dq * width * (2 raw - sum_q) + factor_vq * low

is exactly triple_x + d(q, u).  Setting triple_x = est(u -> v) - d(q, u)
gives each edge the estimate the scenario wants, independent of the query's
quantization.  Node vectors are integer points q + o with |o|^2 = the wanted
squared distance (four-square decompositions), so exact distances are exact
integers too.  Used by the CPU trace tests and, unchanged, by the GPU parity
tests.
"""
from __future__ import annotations

import functools
import math

import numpy as np

from flashgann_amd.codebook import MAX_INDEX, Codebook, Layout

DIM = 40  # padded dimension 64: the smallest layout with a code region


@functools.lru_cache(maxsize=None)
def four_squares(n: int) -> tuple[int, int, int, int]:
    """a^2 + b^2 + c^2 + d^2 == n with a >= b >= c >= d >= 0 (brute force)."""
    a = math.isqrt(n)
    while a >= 0:
        r1 = n - a * a
        b = min(a, math.isqrt(r1))
        while b >= 0:
            r2 = r1 - b * b
            c = min(b, math.isqrt(r2))
            while c >= 0:
                r3 = r2 - c * c
                d = math.isqrt(r3)
                if d * d == r3 and d <= c:
                    return a, b, c, d
                c -= 1
            b -= 1
        a -= 1
    raise ValueError(n)


def query(dim: int = DIM) -> np.ndarray:
    """(10, 3, 0, ...): its rotation is not constant, so the quantizer's width
    is nonzero (a constant rotated query is undefined in the reference)."""
    q = np.zeros(dim, np.float32)
    q[0], q[1] = 10, 3
    return q


def make(dist: dict[int, int], adj: dict[int, list[int]], est: dict[tuple[int, int], int],
         degree: int, entry: int = 0, dim: int = DIM) -> tuple[Codebook, np.ndarray]:
    """Codebook over nodes 0..max(dist) at the given squared distances from
    query(); adj[u] lists u's neighbours (padded with 0xFFFFFFFF to degree);
    est[(u, v)] is the estimate of edge u -> v (default: the exact distance)."""
    n = max(dist) + 1
    q = query(dim)
    lay = Layout.make(dim, degree)
    rows = np.zeros((n, lay.row_offset), np.float32)
    for v in range(n):
        o = np.zeros(dim, np.float32)
        o[2:6] = four_squares(dist[v])
        rows[v, :dim] = q + o
    f = rows[:, lay.factor_offset:lay.neighbor_offset].reshape(n, 3, degree)
    ids = rows[:, lay.neighbor_offset:lay.row_offset].view(np.uint32)
    ids[:] = MAX_INDEX
    f[:, 0, :] = np.float32(np.finfo(np.float32).max)  # padding edges
    for u, lst in adj.items():
        assert len(lst) <= degree
        for j, v in enumerate(lst):
            if v is None:
                continue
            ids[u, j] = v
            e = est[(u, v)] if (u, v) in est else dist[v]
            f[u, 0, j] = e - dist[u]
    signs = np.ones(lay.padded_dim, np.float32)
    return Codebook(rows, signs, entry, lay), q[None, :]


def scenario_cutoff():
    """Degree 4, beam 3, K 2: the K-th cutoff at beam[min(K, beam) - 1] and
    the near count's `<=` (an estimate equal to the cutoff), the keep-all
    shortcut, and the rho trajectory of stage I."""
    dist = {0: 100, 1: 36, 2: 49, 3: 64, 4: 81, 5: 25, 6: 40, 7: 50, 8: 80, 9: 30, 10: 45}
    adj = {0: [1, 2, 3, 4], 1: [5, 6, 7, 8], 2: [0, 1], 3: [0], 4: [0], 5: [1, 6, 0, 2],
           6: [9, 10, 1, 5], 7: [1], 8: [1], 9: [5, 6, 10, 1], 10: [6]}
    est = {(1, 6): 49}  # node 6 is at 40 but estimated at 49, the cutoff
    return make(dist, adj, est, degree=4)


def scenario_stage2():
    """Degree 8, beam 64, K 10: three dead-end stage-I expansions under a
    fixed top-1 (the entry), the switch to stage II on the fourth stall, and a
    stage-II round over three parents that keeps 4 children each (selected by
    estimate, compacted in (task, lane) order).  Parents 4 and 5 have 8 fresh
    children; parent 6 has 5 (its other slots point at visited nodes), one
    more than it keeps, so the keep-all shortcut must not apply."""
    dist = {0: 1}
    adj = {0: [1, 2, 3, 4, 5, 6, 7, 8]}
    for i in range(1, 9):
        dist[i] = 10 * i
        adj[i] = [0]
    pattern = [8, 1, 7, 2, 6, 3, 5, 4]  # estimate rank of each neighbour slot
    nxt = 9
    for p, base in ((4, 100), (5, 200)):
        kids = list(range(nxt, nxt + 8))
        nxt += 8
        adj[p] = kids
        for k, r in zip(kids, pattern):
            dist[k] = base + 10 * r
            adj[k] = [p]
    # parent 6: fresh 25..29 at ranks 5, 1, 4, 2, 3 between visited 0, 1, 2
    adj[6] = [25, 0, 26, 1, 27, 2, 28, 29]
    for k, r in zip((25, 26, 27, 28, 29), (5, 1, 4, 2, 3)):
        dist[k] = 300 + 10 * r
        adj[k] = [6]
    return make(dist, adj, {}, degree=8)


def scenario_stage2_cutoff():
    """Degree 8, beam 8, K 8: stage II with a valid cutoff (beam[7]) and an
    estimate equal to it.  Node 1's two far children (500, 510) fill the beam;
    2 and 3 are dead ends; the fourth stall switches to stage II over parents
    4, 5, 6, 9, of which only 4 has fresh children, estimated at 400, 500 (node
    31, truly at 450), 600 .. 1100 against the cutoff 500."""
    dist = {0: 1}
    adj = {0: [1, 2, 3, 4, 5, 6, 7, 8]}
    for i in range(1, 9):
        dist[i] = 10 * i
        adj[i] = [0]
    adj[1] = [9, 10, 0]
    dist[9], dist[10] = 500, 510
    adj[9], adj[10] = [1], [1]
    kids = list(range(30, 38))
    adj[4] = kids
    est = {}
    for k, e in zip(kids, (400, 500, 600, 700, 800, 900, 1000, 1100)):
        dist[k] = e
        adj[k] = [4]
    dist[31] = 450
    est[(4, 31)] = 500
    for i in range(11, 30):  # unused ids, so that 30.. exist
        dist[i] = 5000
        adj[i] = [0]
    return make(dist, adj, est, degree=8)


def scenario_reset(n: int = 40):
    """Degree 3 path: node i links to i+1, i+2, i-1 and lies at squared
    distance 10000 - 10 i, so stage I expands node 2k at iteration k.  The
    visited set is rebuilt from the beam at iteration 15, before that
    iteration's merge: node 29, scored at iteration 14, is then admitted a
    second time by its sibling 30 (the reference's quirk at
    adaptive_search.cuh:128-145)."""
    dist = {i: 10000 - 10 * i for i in range(n)}
    adj = {}
    for i in range(n):
        adj[i] = [i + 1 if i + 1 < n else None, i + 2 if i + 2 < n else None, i - 1 if i >= 1 else None]
    return make(dist, adj, {}, degree=3)


def complete_graph(n: int = 33, dim: int = 128, nq: int = 8, seed: int = 11):
    """n integer points, each linked to all others (degree n - 1) in
    (distance, id) order, with real RaBitQ codes; queries from the same
    distribution."""
    from flashgann_amd import builder, datasets
    rng = np.random.default_rng(seed)
    base = rng.integers(0, 40, size=(n, dim)).astype(np.float32)
    q = rng.integers(0, 40, size=(nq, dim)).astype(np.float32)
    d = ((base[:, None, :].astype(np.float64) - base[None, :, :]) ** 2).sum(-1)
    np.fill_diagonal(d, np.inf)
    order = np.lexsort((np.broadcast_to(np.arange(n), (n, n)), d), axis=1)[:, : n - 1]
    cb = builder.codebook_from_graph(base, order, datasets.signs_for(128, 1), entry=0)
    return cb, q, base


@functools.lru_cache(maxsize=None)
def line_index(n: int = 20000, dim: int = 64, degree: int = 32):
    """Points i e_0 (i = 0..n-1) on a line, each linked to its `degree`
    nearest by (distance, id), with real RaBitQ codes; entry point 0 and four
    queries past the far end.  Stage I walks ~16 nodes per iteration, so a
    search never runs out of unexpanded entries: it stops at max_iter =
    min((11 beam + 9) / 10, 1024) (gpu_search_adaptive.cu:96,
    adaptive_search_config.cuh:12) with candidates still arriving."""
    from flashgann_amd import builder, datasets
    base = np.zeros((n, dim), np.float32)
    base[:, 0] = np.arange(n)
    # the degree nearest of r are the window of degree + 1 points around r
    # (shifted inwards at the ends) without r, ordered by (distance, id)
    lo = np.clip(np.arange(n) - degree // 2, 0, n - 1 - degree)
    win = lo[:, None] + np.arange(degree + 1)[None, :]
    r = np.arange(n)[:, None]
    nbrs = win[win != r].reshape(n, degree)
    order = np.lexsort((nbrs, np.abs(nbrs - r)), axis=1)
    nbrs = np.take_along_axis(nbrs, order, axis=1)
    cb = builder.codebook_from_graph(base, nbrs, datasets.signs_for(64, 1), entry=0)
    q = np.zeros((4, dim), np.float32)
    q[:, 0] = [n + 10, n + 500, n + 3000, 2 * n]
    q[:, 1] = [0, 1, 2, 3]
    return cb, q, base


@functools.lru_cache(maxsize=None)
def random_graph_index(n: int = 20000, dim: int = 128, degree: int = 32, nq: int = 4, seed: int = 7):
    """Integer points in [0, 16)^dim, each linked to `degree` uniformly random
    other points; entry point 0, queries from the same distribution.  Nearly
    every child is fresh, so with K = beam each stage-II iteration inserts
    close to 32 keys into the visited table: between two resets the table
    comes within a few keys of its worst case (beam + 16 x 32 + 1 keys), which
    the kernel's table is sized to hold with one slot to spare."""
    from flashgann_amd import builder, datasets
    rng = np.random.default_rng(seed)
    base = rng.integers(0, 16, size=(n, dim)).astype(np.float32)
    q = rng.integers(0, 16, size=(nq, dim)).astype(np.float32)
    nb = rng.integers(0, n - 1, size=(n, degree))
    nb = nb + (nb >= np.arange(n)[:, None])  # no self links
    cb = builder.codebook_from_graph(base, nb, datasets.signs_for(128, 1), entry=0)
    return cb, q, base


def visited_peak(trace, beam: int) -> int:
    """Most distinct keys the visited set holds between two resets of one
    traced search: the restored beam (every merged candidate enters the beam
    until it is full, and none repeats an entry still in it) plus the
    candidates inserted over the next 16 iterations and the entry point."""
    valid = np.array([sum(1 for c in r.cand_idx if c != 0xFFFFFFFF) for r in trace])
    merged = 1 + np.cumsum(valid)
    peak = 0
    for t0 in range(15, len(trace), 16):
        peak = max(peak, min(beam, int(merged[t0 - 1])) + int(valid[t0:t0 + 16].sum()) + 1)
    return peak


def scenario_short_graph():
    """Three nodes, degree 2: the entry 0 (100) links to 1 (36) and 2 (49),
    which link back to 0.  Every search reaches three nodes, fewer than the
    beam or K asks for, so the result writer's empty slots show
    (adaptive_search.cuh:455-464): a beam slot that never held an id is
    written as 0x7FFFFFFF (its MSB masked before the MAX_INDEX test), and
    only positions past the beam repeat the last id."""
    dist = {0: 100, 1: 36, 2: 49}
    adj = {0: [1, 2], 1: [0], 2: [0]}
    return make(dist, adj, {}, degree=2)


def scenario_stage2_parents():
    """Degree 8, beam 8, K 8: one stage-II round whose outcome depends on
    three rules of adaptive_search.cuh:377-404 that the other scenarios leave
    open.  The prelude is scenario_stage2_cutoff's (1 .. 6 scored from the
    entry, 9 (500) and 10 (510) from node 1, 2 and 3 dead ends), so the
    round runs over parents 4 (40), 5 (50), 6 (60) and 9 (500) with the
    K-th cutoff 500 and a keep of 4 per parent:
      - parent 5 (not the first parent) has 8 fresh children estimated at
        420, 490, 505, 600 .. 1000 from ITS distance 50: two are within the
        cutoff.  Estimated from the first parent's distance (40) instead,
        three would be;
      - parent 6 has 8 fresh children all above the cutoff, the best two
        tied at 650 in lanes 1 and 3: the keep falls to 1 and the lower lane
        wins the tie;
      - parent 9 has exactly 4 fresh children (the keep): all are admitted
        without estimates, although their estimates (600 .. 900) lie above
        the cutoff."""
    cb_dist = {0: 1}
    adj = {0: [1, 2, 3, 4, 5, 6, 7, 8]}
    for i in range(1, 9):
        cb_dist[i] = 10 * i
        adj[i] = [0]
    adj[1] = [9, 10, 0]
    cb_dist[9], cb_dist[10] = 500, 510
    adj[10] = [1]
    est = {}
    # parent 5: estimates and true distances
    kids5 = list(range(30, 38))
    adj[5] = kids5
    for k, e in zip(kids5, (420, 490, 505, 600, 700, 800, 900, 1000)):
        cb_dist[k] = e
        est[(5, k)] = e
        adj[k] = [5]
    cb_dist[31], cb_dist[32] = 15, 16
    # parent 6: all above the cutoff, a tie at the minimum in lanes 1 and 3
    kids6 = list(range(40, 48))
    adj[6] = kids6
    for k, e in zip(kids6, (700, 650, 900, 650, 800, 750, 1000, 950)):
        cb_dist[k] = e
        est[(6, k)] = e
        adj[k] = [6]
    cb_dist[41], cb_dist[43] = 25, 26
    # parent 9: four fresh children between four visited ones
    adj[9] = [50, 51, 52, 53, 0, 1, 2, 3]
    for k, d, e in zip((50, 51, 52, 53), (35, 36, 37, 38), (600, 700, 800, 900)):
        cb_dist[k] = d
        est[(9, k)] = e
        adj[k] = [0]
    adj[31] = adj[41] = [0]
    for i in list(range(11, 30)) + list(range(38, 40)) + list(range(48, 50)):  # unused ids
        cb_dist[i] = 5000
        adj[i] = [0]
    return make(cb_dist, adj, est, degree=8)


def scenario_wide_degree():
    """Degree 40 (two 32-neighbour tiles per parent), beam 64, K 12.  With
    one expander the search reads only the first min(degree, 32) slots of a
    list (adaptive_search.cuh:222): node 9 (distance 5) sits in slot 35 of
    the entry's list and is never found.  In stage II the second tile of a
    parent holds 8 slots, so its keep is min(ceil(8 (1 - 0.9)), 32 / 8) = 1
    (adaptive_search.cuh:380-382 with rate 1 - 4/40): of parent 4's three
    fresh children in slots 32 .. 34 only the best estimate (21, 150) is
    kept.  Five parents of two tiles each make 10 tasks: two rounds."""
    dist = {0: 1, 9: 5}
    adj = {0: [1, 2, 3, 4, 5, 6, 7, 8] + [None] * 27 + [9]}
    for i in range(1, 9):
        dist[i] = 10 * i
        adj[i] = [0]
    adj[9] = [0]
    adj[4] = [0] + [None] * 31 + [20, 21, 22]
    for k, d in zip((20, 21, 22), (200, 150, 300)):
        dist[k] = d
        adj[k] = [4]
    for i in range(10, 20):  # unused ids
        dist[i] = 5000
        adj[i] = [0]
    return make(dist, adj, {}, degree=40)


def scenario_task_order():
    """Degree 40, beam 64, K 44: stage II's tasks run parent by parent
    (task t is tile t % 2 of parent t / 2, adaptive_search.cuh:351-354), eight
    to a round, and the compaction keeps at most BUFFER_BOUND = 32 kept
    children (:413-430); the ones past it are inserted into the visited set
    but never scored.  Which of a round's children take the last free slots
    is a race between the reference's warps; the oracle (and the kernel)
    take them in (task, lane) order.  The entry (distance 1) lists 1 ..
    11; 1, 2, 3 are dead ends, so stage II starts at iteration 4 with parents
    4 .. 11.  Parent p has four children in its first tile (slots 0-3) and
    one in its second (slot 32), ids 20 + 5 (p - 4) + j, at distance
    1000 + id; every child links back to its parent only."""
    dist = {0: 1}
    adj = {0: list(range(1, 12))}
    for i in range(1, 12):
        dist[i] = 10 * i
        adj[i] = [0]
    for p in range(4, 12):
        kids = [20 + 5 * (p - 4) + j for j in range(5)]
        adj[p] = kids[:4] + [None] * 28 + [kids[4]]
        for k in kids:
            dist[k] = 1000 + k
            adj[k] = [p]
    for i in range(12, 20):  # unused ids
        dist[i] = 5000
        adj[i] = [0]
    return make(dist, adj, {}, degree=40)


BAD_ID = 40  # an id past the last node of scenario_out_of_range_ids


def scenario_out_of_range_ids():
    """Degree 8, beam 64, K 10: a neighbour id that is neither a node nor
    0xFFFFFFFF (BAD_ID, past the 15 nodes) is not a valid child in either
    stage (adaptive_search.cuh:233, 372): it is read (ids counter) but never
    estimated, inserted or scored.  The entry lists 1 .. 7 with BAD_ID in
    slot 2; 1, 2, 3, 5, 6, 7 are dead ends, and parent 4 lists BAD_ID in slot
    0 before its children 8 .. 14.  BAD_ID's edges carry the estimate 10^6."""
    dist = {0: 1}
    adj = {0: [1, 2, BAD_ID, 3, 4, 5, 6, 7]}
    for i in range(1, 8):
        dist[i] = 10 * i
        adj[i] = [0]
    adj[4] = [BAD_ID] + list(range(8, 15))
    for k, r in zip(range(8, 15), (6, 2, 7, 1, 5, 3, 4)):  # estimate ranks of 8 .. 14
        dist[k] = 100 + 10 * r
        adj[k] = [4]
    est = {(0, BAD_ID): 10 ** 6, (4, BAD_ID): 10 ** 6}
    return make(dist, adj, est, degree=8)


def scenario_wide_degree_codes():
    """scenario_wide_degree with parent 4's second-tile estimates made by
    their codes: the edges 4 -> 20, 21, 22 (slots 32-34) carry triple_x 160
    (so triple_x + d(q, 4) = 200), factor_dq 1 and factor_vq 0, and the codes
    at slots 32, 33, 34 are all ones, all zeros and every other chunk set.
    The query (10, 3, 0, ...) rotates to 13 on even and 7 on odd dimensions
    of 64 (low 7, width 6/63), so it quantizes to q = 1 (odd) and 63 (even:
    6 / fl(6/63) + 0.5 falls a hair below 63.5 in float), sum_q = 2048: raw
    is 2048, 0 and 1024, and the estimates 200 + (6/63)(2 raw - 2048) =
    395.0, 5.0 and 200.  Slots 0-2 of the first tile (ids 0 and two
    empty slots) hold the codes zeros, ones, ones, so an estimate read from
    slot l of the tile instead of slot 32 + l would rank 20 first."""
    cb, q = scenario_wide_degree()
    lay = cb.layout
    codes = cb.rows[:, lay.code_offset:lay.factor_offset].view(np.uint8).reshape(cb.rows.shape[0], lay.degree, -1)
    f = cb.rows[:, lay.factor_offset:lay.neighbor_offset].reshape(cb.rows.shape[0], 3, lay.degree)
    for slot, byte in ((32, 0xFF), (33, 0x00), (34, 0x0F), (0, 0x00), (1, 0xFF), (2, 0xFF)):
        codes[4, slot, :] = byte
    for slot in (32, 33, 34):
        f[4, 0, slot] = 160.0
        f[4, 1, slot] = 1.0
        f[4, 2, slot] = 0.0
    return cb, q


def scenario_shared_child():
    """Degree 8, beam 64, K 10: two parents of one stage-II round list the
    same child (node 30).  The entry lists 1 .. 6; 1, 2, 3 are dead ends, so
    stage II starts at iteration 4 with parents 4, 5, 6.  Parent 4 lists
    20, 21, 22, 23, 30, 24, 25, 26 and parent 5 lists 31, 30, 32 .. 37; 6 is a
    dead end.  Both parents see 30 as unvisited (the visited set as it stood
    at the round's start) and both keep it among their four best; the
    inserts go in (task, lane) order, so parent 4's copy is the one kept and
    parent 5's is dropped, leaving parent 5 three children (the reference's
    warps race here: this is the rule the oracle and the kernel fix)."""
    dist = {0: 1}
    adj = {0: [1, 2, 3, 4, 5, 6, None, None]}
    for i in range(1, 7):
        dist[i] = 10 * i
        adj[i] = [0]
    adj[4] = [20, 21, 22, 23, 30, 24, 25, 26]
    adj[5] = [31, 30, 32, 33, 34, 35, 36, 37]
    for k, d in zip((20, 21, 22, 23, 24, 25, 26), (200, 210, 220, 230, 240, 250, 260)):
        dist[k] = d
        adj[k] = [4]
    for k, d in zip((31, 32, 33, 34, 35, 36, 37), (170, 180, 190, 300, 310, 320, 330)):
        dist[k] = d
        adj[k] = [5]
    dist[30] = 150
    adj[30] = [4]
    for i in list(range(7, 20)) + [27, 28, 29]:  # unused ids
        dist[i] = 5000
        adj[i] = [0]
    return make(dist, adj, {}, degree=8)
