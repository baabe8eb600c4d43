"""Codebook builder: graph construction and per-edge RaBitQ encoding.

The reference consumes a prebuilt SymphonyQG-style codebook and ships no
builder (README.md:12, include/qg.hpp:16).  This module writes one in the
reference's layout (include/qg.hpp:66-73).  It runs on whatever torch device
it is handed: the GPU for million-point indexes, the CPU for test fixtures.

Graph.  Exactly `degree` out-edges per node:
  * local edges: exact k-nearest candidates (k = 2*degree) pruned with the
    relative-neighbourhood rule (drop v if a kept w has d(w,v) < d(u,v)),
    at most degree - degree/4 of them;
  * long links: seeded uniform-random targets in every remaining slot (at
    least degree/4).  Mixture data with well-separated components has no
    between-component edges in a k-NN graph; the random links make every
    component reachable and let the beam search probe other components
    cheaply through RaBitQ estimates.  Recall is bimodal on such data (a query
    finds its component or misses it), and the miss rate falls with the number
    of random probes per expansion, so slots the RNG rule leaves empty go to
    random links rather than to backfilled near duplicates
    (fill_random=False backfills them from the k-NN candidates instead).
Neighbour lists are sorted by (distance, id); short lists (tiny N) are padded
with 0xFFFFFFFF, which the search treats as "no neighbour".

Encoding (per edge u -> v, residual r = v - u zero-padded to B, P = H_B diag(s)
the unnormalised Walsh-Hadamard rotation the search applies to the query,
include/utils.cuh:790-821):
    y = P r,  b_i = [y_i > 0],  s_i = 2 b_i - 1
  L2:  f = -2 |r|^2 / sum|y|;  factor_dq = f;  factor_vq = f * sum(s);
       triple_x = |r|^2 - f * <s, P u>
  IP:  f = -|r|^2 / sum|y|;    factor_dq = f;  factor_vq = f * sum(s);
       triple_x = 0
so that the search's estimate (include/utils.cuh:989-993)
    triple_x + d(q,u) + factor_dq*width*(2*raw - sum_q) + factor_vq*low
is the RaBitQ estimate of d(q,v) with P q ~ low + width*q_i.  Factors are
computed in float64 and rounded to float32.  A zero residual (duplicate point)
gets f = 0 and triple_x = 0.  Edges to padding get triple_x = FLT_MAX.
"""
from __future__ import annotations

import time

import numpy as np
import torch

from .codebook import MAX_INDEX, Codebook, Layout, code_bit_positions

FLT_MAX = float(np.finfo(np.float32).max)


def _sqnorm(x: torch.Tensor) -> torch.Tensor:
    return (x * x).sum(-1)


def knn(base: torch.Tensor, k: int, queries: torch.Tensor | None = None,
        exclude_self: bool = True, chunk_elems: int = 1 << 28):
    """Exact k nearest neighbours by L2 (or of `queries` against `base`).

    Returns (ids int64 [m,k], sqdist float32 [m,k]) ordered by (dist, id).
    Squared distances are |x|^2 + |y|^2 - 2 x.y in float32, exact for
    integer-valued data with |.|^2 < 2^24.  The distance block of one step
    stays at `chunk_elems` floats: on this ROCm build a float32 product whose
    output spans more than 2^31 bytes has returned wrong rows (measured: rows
    56-63 of a 107 x 10M product), so no product here is that large."""
    q = base if queries is None else queries
    n = base.shape[0]
    m = q.shape[0]
    kk = min(k, n - (1 if exclude_self and queries is None else 0))
    extra = min(16, n - kk)
    bn = _sqnorm(base)
    rows = max(1, min(m, chunk_elems // max(1, n)))
    ids_out = torch.empty((m, kk), dtype=torch.int64, device=base.device)
    d_out = torch.empty((m, kk), dtype=torch.float32, device=base.device)
    for s in range(0, m, rows):
        e = min(m, s + rows)
        qs = q[s:e]
        d = _sqnorm(qs)[:, None] + bn[None, :] - 2.0 * (qs @ base.T)
        d.clamp_(min=0.0)
        if exclude_self and queries is None:
            r = torch.arange(s, e, device=base.device)
            d[r - s, r] = float("inf")
        kc = min(n, kk + extra)
        dv, di = torch.topk(d, kc, dim=1, largest=False, sorted=True)
        # order by (dist, id): sort by id, then stable sort by dist
        o = torch.argsort(di, dim=1)
        di = torch.gather(di, 1, o)
        dv = torch.gather(dv, 1, o)
        o = torch.argsort(dv, dim=1, stable=True)
        ids_out[s:e] = torch.gather(di, 1, o)[:, :kk]
        d_out[s:e] = torch.gather(dv, 1, o)[:, :kk]
    return ids_out, d_out


def kmeans(x: torch.Tensor, cells: int, sample: int = 1 << 18, iters: int = 8, seed: int = 0x5EED,
           chunk: int = 1 << 16) -> torch.Tensor:
    """Lloyd's k-means on a seeded sample of x (float32 on x's device):
    returns (cells, dim) centroids.  Initial centroids are distinct sample
    points; a cell left empty keeps its centroid."""
    n, dim = x.shape
    g = torch.Generator().manual_seed(seed)
    m = min(n, max(sample, cells))
    pick = torch.randperm(n, generator=g)[:m].to(x.device)
    xs = x[pick]
    c = xs[torch.randperm(m, generator=g)[:cells].to(x.device)].clone()
    for _ in range(iters):
        a = _nearest_cells(xs, c, 1, chunk)[:, 0]
        sums = torch.zeros_like(c).index_add_(0, a, xs)
        cnt = torch.bincount(a, minlength=cells).to(x.dtype)
        nz = cnt > 0
        c[nz] = sums[nz] / cnt[nz, None]
    return c


def _nearest_cells(x: torch.Tensor, c: torch.Tensor, probes: int, chunk: int = 1 << 16) -> torch.Tensor:
    """(n, probes) int64: the `probes` nearest centroids of each row of x."""
    cn = _sqnorm(c)
    out = torch.empty((x.shape[0], probes), dtype=torch.int64, device=x.device)
    for s in range(0, x.shape[0], chunk):
        d = cn[None, :] - 2.0 * (x[s:s + chunk] @ c.T)
        out[s:s + chunk] = torch.topk(d, probes, dim=1, largest=False).indices
    return out


def knn_partitioned(x: torch.Tensor, k: int, cells: int | None = None, probes: int = 2, seed: int = 0x5EED,
                    verbose: bool = False, block_elems: int = 1 << 28):
    """Approximate k nearest neighbours of every row of x (excluding itself)
    for sets too large for knn(): k-means cells (about 2,500 points each),
    every point in the cell of its nearest centroid, and each point's
    neighbours searched exactly among the points of its `probes` nearest
    cells.  Returns (ids int64 [n,k], sqdist float32 [n,k]) ordered by
    (dist, id), -1 / inf where fewer than k points were searched."""
    n, dim = x.shape
    dev = x.device
    cells = cells or max(1, min(n // 2500, 1 << 16))
    probes = max(1, min(probes, cells))
    t0 = time.time()
    cen = kmeans(x, cells, seed=seed)
    near = _nearest_cells(x, cen, probes)
    del cen
    home = near[:, 0]
    order = torch.argsort(home)
    bounds = torch.zeros(cells + 1, dtype=torch.int64, device=dev)
    bounds[1:] = torch.cumsum(torch.bincount(home, minlength=cells), 0)
    qorder = torch.argsort(near.reshape(-1))
    qbounds = torch.zeros(cells + 1, dtype=torch.int64, device=dev)
    qbounds[1:] = torch.cumsum(torch.bincount(near.reshape(-1), minlength=cells), 0)
    del near
    if verbose:
        print(f"[builder] {cells} cells in {time.time() - t0:.1f}s", flush=True)
    xn = _sqnorm(x)
    # per cell up to 16 more than k, so that ties at a cell's k-th distance
    # still resolve by id after the merge (as in knn())
    kx = k + 16
    cid = torch.full((n * probes, kx), -1, dtype=torch.int32, device=dev)
    cdist = torch.full((n * probes, kx), float("inf"), dtype=torch.float32, device=dev)
    bh, qh = bounds.cpu().tolist(), qbounds.cpu().tolist()
    for c in range(cells):
        mem = order[bh[c]:bh[c + 1]]
        qry = qorder[qh[c]:qh[c + 1]]  # (point, probe) pairs as point * probes + probe
        if mem.numel() == 0 or qry.numel() == 0:
            continue
        xm, mn = x[mem], xn[mem]
        kk = min(kx, mem.numel())
        step = max(1, block_elems // mem.numel())
        for s in range(0, qry.numel(), step):
            qs = qry[s:s + step]
            qp = qs // probes
            d = xn[qp][:, None] + mn[None, :] - 2.0 * (x[qp] @ xm.T)
            d.clamp_(min=0.0)
            d.masked_fill_(qp[:, None] == mem[None, :], float("inf"))
            dv, di = torch.topk(d, kk, dim=1, largest=False, sorted=False)
            # a cell with fewer than kk other points returns the point itself
            # (at distance inf): it is no neighbour
            ids = mem[di]
            own = ids == qp[:, None]
            cid[qs, :kk] = torch.where(own, torch.full_like(ids, -1), ids).to(torch.int32)
            cdist[qs, :kk] = torch.where(own, torch.full_like(dv, float("inf")), dv)
        if verbose and (c + 1) % 1000 == 0:
            print(f"[builder] cell {c + 1}/{cells} searched ({time.time() - t0:.1f}s)", flush=True)
    del order, qorder, xn
    if verbose:
        print(f"[builder] per-cell neighbours in {time.time() - t0:.1f}s", flush=True)
    cid = cid.view(n, probes * kx)
    cdist = cdist.view(n, probes * kx)
    ids_out = torch.empty((n, k), dtype=torch.int64, device=dev)
    d_out = torch.empty((n, k), dtype=torch.float32, device=dev)
    big = torch.iinfo(torch.int64).max
    for s in range(0, n, 1 << 20):
        ci = cid[s:s + (1 << 20)].to(torch.int64)
        cd = cdist[s:s + (1 << 20)]
        cd = torch.where(ci < 0, torch.full_like(cd, float("inf")), cd)
        o = torch.argsort(torch.where(ci < 0, torch.full_like(ci, big), ci), dim=1)
        ci, cd = torch.gather(ci, 1, o), torch.gather(cd, 1, o)
        o = torch.argsort(cd, dim=1, stable=True)[:, :k]
        ids_out[s:s + (1 << 20)] = torch.gather(ci, 1, o)
        d_out[s:s + (1 << 20)] = torch.gather(cd, 1, o)
    return ids_out, d_out


def _pairwise_sq(v: torch.Tensor) -> torch.Tensor:
    """v: (m, c, d) -> (m, c, c) squared distances."""
    nv = _sqnorm(v)
    g = torch.bmm(v, v.transpose(1, 2).contiguous())
    return (nv[:, :, None] + nv[:, None, :] - 2.0 * g).clamp_(min=0.0)


def _prune(cand: torch.Tensor, cd: torch.Tensor, x: torch.Tensor, limit: int,
           alpha2: float = 1.0, chunk: int = 4096) -> torch.Tensor:
    """Greedy (alpha-)RNG pruning of ordered candidate lists.

    cand (n, c) int64 (-1 = none), cd (n, c) squared distances to the owner.
    Keeps candidate i unless an earlier kept w has alpha2 * d(w, v_i) < d(u, v_i)
    (alpha2 = 1: relative neighbourhood rule), at most `limit` kept.
    Returns a bool mask (n, c)."""
    n, c = cand.shape
    out = torch.zeros((n, c), dtype=torch.bool, device=cand.device)
    for s in range(0, n, chunk):
        e = min(n, s + chunk)
        cc = cand[s:e]
        valid = cc >= 0
        v = x[cc.clamp(min=0)]
        pd = _pairwise_sq(v)
        du = cd[s:e]
        kept = torch.zeros((e - s, c), dtype=torch.bool, device=cand.device)
        count = torch.zeros((e - s,), dtype=torch.int64, device=cand.device)
        for i in range(c):
            ok = valid[:, i] & (count < limit)
            if i > 0:
                bad = ((alpha2 * pd[:, i, :i] < du[:, i : i + 1]) & kept[:, :i]).any(1)
                ok &= ~bad
            kept[:, i] = ok
            count += ok.to(torch.int64)
        out[s:e] = kept
    return out


def _first_unique(m: torch.Tensor, width: int) -> torch.Tensor:
    """Row-wise: first `width` distinct non-negative entries of m in order,
    padded with -1."""
    rows, L = m.shape
    pos = torch.arange(L, device=m.device).expand(rows, L)
    key = torch.where(m >= 0, m, torch.full_like(m, -1))
    o = torch.argsort(key, dim=1, stable=True)
    sk = torch.gather(key, 1, o)
    dup_sorted = torch.zeros_like(sk, dtype=torch.bool)
    dup_sorted[:, 1:] = sk[:, 1:] == sk[:, :-1]
    dup = torch.zeros_like(dup_sorted)
    dup.scatter_(1, o, dup_sorted)
    drop = dup | (m < 0)
    rank = drop.to(torch.int64) * L + pos
    o2 = torch.argsort(rank, dim=1)[:, :width]
    sel = torch.gather(m, 1, o2)
    sel_drop = torch.gather(drop, 1, o2)
    sel = torch.where(sel_drop, torch.full_like(sel, -1), sel)
    if sel.shape[1] < width:
        pad = torch.full((rows, width - sel.shape[1]), -1, dtype=sel.dtype, device=sel.device)
        sel = torch.cat([sel, pad], 1)
    return sel


def hadamard_rotation(signs: np.ndarray, device) -> torch.Tensor:
    """P = H_B diag(signs) as float64 (B x B), H_B the Sylvester matrix."""
    b = signs.shape[0]
    idx = torch.arange(b, dtype=torch.int64)
    parity = torch.zeros((b, b), dtype=torch.int64)
    a = idx[:, None] & idx[None, :]
    while bool((a != 0).any()):
        parity ^= a & 1
        a = a >> 1
    h = (1 - 2 * parity).to(torch.float64)
    return (h * torch.as_tensor(signs, dtype=torch.float64)[None, :]).to(device)


def _reach(nbrs: torch.Tensor, reached: torch.Tensor, start: torch.Tensor) -> int:
    """Marks every node reachable from the `start` ids over the out-edges of
    nbrs (-1 = none) in `reached` (bool, in place; nodes already marked are
    not expanded again).  Returns the number of newly marked nodes."""
    frontier = start[~reached[start]]
    reached[frontier] = True
    added = int(frontier.numel())
    while frontier.numel():
        nb = nbrs[frontier].reshape(-1)
        nb = nb[nb >= 0]
        nb = torch.unique(nb[~reached[nb]])
        reached[nb] = True
        added += int(nb.numel())
        frontier = nb
    return added


def connect_graph(x: torch.Tensor, nbrs: torch.Tensor, fixed: torch.Tensor, entry: int,
                  verbose: bool = False) -> tuple[torch.Tensor, int]:
    """Makes every node reachable from `entry` by adding the fewest links the
    greedy repair finds, in the manner of NSG's spanning step (Fu et al.,
    VLDB 2019): while some node is unreached, the unreached node nearest the
    entry point is linked from its nearest reached node that has a free slot,
    and everything reachable from it is marked.  A free slot is one that is
    empty or holds an edge not in `fixed` (bool, same shape as nbrs: the
    RNG-pruned edges, which are never replaced); the link takes the last such
    slot.  Returns (nbrs with the links, number of links added)."""
    n = x.shape[0]
    dev = x.device
    nbrs = nbrs.clone()
    free = ~fixed | (nbrs < 0)
    reached = torch.zeros(n, dtype=torch.bool, device=dev)
    _reach(nbrs, reached, torch.tensor([entry], device=dev))
    xn = _sqnorm(x)
    de = _sqnorm(x - x[entry][None, :])  # distance of every node to the entry point
    links = 0
    t0 = time.time()
    while not bool(reached.all()):
        # the unreached node nearest the entry point
        u = int(torch.argmin(torch.where(reached, torch.full_like(de, float("inf")), de)).item())
        d = xn + xn[u] - 2.0 * (x @ x[u])
        has_free = free.any(1)
        d = torch.where(reached & has_free, d, torch.full_like(d, float("inf")))
        v = int(torch.argmin(d).item())
        if not bool(torch.isfinite(d[v])):
            raise RuntimeError("connect_graph: no reached node has a free slot")
        slot = int(torch.nonzero(free[v]).max().item())
        nbrs[v, slot] = u
        free[v, slot] = False
        links += 1
        _reach(nbrs, reached, torch.tensor([u], device=dev))
        if verbose and links % 200 == 0:
            print(f"[builder] connect: {links} links, {int(reached.sum())}/{n} reachable "
                  f"({time.time() - t0:.1f}s)", flush=True)
    return nbrs, links


def build_graph(x: torch.Tensor, degree: int, random_links: int | None = None,
                seed: int = 0x5EED, alpha: float = 1.0, candidates: int | None = None,
                fill_random: bool = True, verbose: bool = False, dist_block_elems: int = 1 << 30,
                knn_method: str = "exact", connect: bool = False, stats: dict | None = None) -> torch.Tensor:
    """Returns (n, degree) int64 neighbour ids (-1 = padding).  The final
    neighbour distances are gathered in row blocks of at most
    `dist_block_elems` floats.  knn_method "exact" takes the candidates from
    knn(), "partitioned" from knn_partitioned() (sets of millions of
    high-dimensional points, where the exact search is out of reach).
    connect=True (with random_links=0): the RNG-pruned k-NN edges are all
    kept, the slots they leave are backfilled from the k-NN candidates, and
    connect_graph() then replaces backfilled slots (or fills empty ones) with
    the links that make every node reachable from the entry point (the node
    nearest the mean); stats, if given, receives the number of links."""
    n = x.shape[0]
    dev = x.device
    kc = min(candidates or 2 * degree, n - 1)
    on_gpu = x.device.type == "cuda"
    if knn_method == "partitioned":
        cand, cd = knn_partitioned(x, kc, verbose=verbose)
    elif knn_method == "exact":
        cand, cd = knn(x, kc)
    else:
        raise ValueError(f"unknown knn_method {knn_method!r}")
    if verbose:
        print(f"[builder] knn done k={kc}", flush=True)
    nr = degree // 4 if random_links is None else random_links
    nr = min(nr, max(0, n - 1 - degree)) if n > 2 * degree else 0
    local_cap = degree - nr
    local_keep = _prune(cand, cd, x, local_cap, alpha2=alpha * alpha, chunk=32768 if on_gpu else 4096)
    if verbose:
        print("[builder] RNG prune done", flush=True)
    ar = torch.arange(kc, device=dev)[None, :]
    o = torch.argsort(torch.where(local_keep, ar, kc + ar), dim=1)
    local = torch.where(torch.gather(local_keep, 1, o), torch.gather(cand, 1, o),
                        torch.full_like(cand, -1))[:, :local_cap]
    parts = [local]
    if nr:
        g = torch.Generator().manual_seed(seed)
        # uniform targets != self: draw in [0, n-1) and skip over the owner
        nfill = degree if fill_random else nr
        r = torch.randint(0, n - 1, (n, 2 * nfill), generator=g).to(dev)
        own = torch.arange(n, device=dev)[:, None]
        r = r + (r >= own).to(r.dtype)
        parts.append(_first_unique(r, nfill))
    parts.append(cand)
    merged = _first_unique(torch.cat(parts, 1), degree)
    if connect:
        if nr:
            raise ValueError("connect=True builds on the RNG-pruned graph: use random_links=0")
        # the RNG-kept edges are the first entries of each list (local is in
        # candidate order and merged starts with it)
        fixed = torch.arange(degree, device=dev)[None, :] < local_keep.sum(1, keepdim=True).clamp(max=local_cap)
        fixed &= merged >= 0
        merged, links = connect_graph(x, merged, fixed, entry_point(x), verbose=verbose)
        if stats is not None:
            stats["connect_links"] = links
    # sort each list by (distance, id)
    big = torch.iinfo(torch.int64).max
    valid = merged >= 0
    # distances to the kept neighbours, in row blocks (the unblocked gather of
    # 1M x 32 x 960 floats alone is 123 GB)
    step = max(1, dist_block_elems // max(1, degree * x.shape[1]))
    dist = torch.empty(merged.shape, dtype=torch.float64, device=dev)
    for s in range(0, n, step):
        e = min(n, s + step)
        mv = x[merged[s:e].clamp(min=0)]
        dist[s:e] = _sqnorm(mv - x[s:e, None, :]).to(torch.float64)
        del mv
    dist = torch.where(valid, dist, torch.full_like(dist, float("inf")))
    o = torch.argsort(torch.where(valid, merged, torch.full_like(merged, big)), dim=1)
    merged = torch.gather(merged, 1, o)
    dist = torch.gather(dist, 1, o)
    o = torch.argsort(dist, dim=1, stable=True)
    return torch.gather(merged, 1, o)


def _encode_chunk(x: torch.Tensor, nb: torch.Tensor, c0: torch.Tensor, p: torch.Tensor, pos: torch.Tensor,
                  weights: torch.Tensor, b: int, use_ip: bool):
    """Codes (m, deg, B/8) uint8 and factors (m, 3, deg) float32 of the
    edges of m nodes: nb (m, deg) neighbour ids, c0 (m, dim) their vectors."""
    m, deg = nb.shape
    dim = x.shape[1]
    dev = x.device
    c = torch.zeros((m, b), dtype=torch.float64, device=dev)
    c[:, :dim] = c0.to(torch.float64)
    valid = nb >= 0
    v = torch.zeros((m, deg, b), dtype=torch.float64, device=dev)
    v[:, :, :dim] = x[nb.clamp(min=0)].to(torch.float64)
    r = v - c[:, None, :]
    del v
    y = r @ p.T
    bits = (y > 0)
    sgn = bits.to(torch.float64) * 2.0 - 1.0
    nr = (r * r).sum(-1)
    del r
    sabs = y.abs().sum(-1)
    del y
    ssum = sgn.sum(-1)
    zero = sabs <= 0
    if use_ip:
        f = torch.where(zero, torch.zeros_like(nr), -nr / torch.where(zero, torch.ones_like(sabs), sabs))
        tx = torch.zeros_like(f)
    else:
        f = torch.where(zero, torch.zeros_like(nr), -2.0 * nr / torch.where(zero, torch.ones_like(sabs), sabs))
        pc = c @ p.T
        spc = (sgn * pc[:, None, :]).sum(-1)
        tx = torch.where(zero, torch.zeros_like(nr), nr - f * spc)
    del sgn
    fvq = f * ssum
    tx = torch.where(valid, tx, torch.full_like(tx, FLT_MAX))
    f = torch.where(valid, f, torch.zeros_like(f))
    fvq = torch.where(valid, fvq, torch.zeros_like(fvq))
    factors = torch.stack([tx, f, fvq], 1).to(torch.float32)
    ordered = torch.zeros((m, deg, b), dtype=torch.int64, device=dev)
    ordered[:, :, pos] = (bits & valid[:, :, None]).to(torch.int64)
    del bits
    codes = (ordered.view(m, deg, b // 8, 8) * weights).sum(-1).to(torch.uint8)
    return codes, factors


def _encode_setup(signs: np.ndarray, dev):
    b = signs.shape[0]
    return (hadamard_rotation(signs, dev), torch.as_tensor(code_bit_positions(b), device=dev),
            2 ** torch.arange(8, device=dev, dtype=torch.int64))


def _encode_rows_per_chunk(deg: int, b: int, chunk_edges: int) -> int:
    return max(1, chunk_edges // max(1, deg * b // 128))


def encode(x: torch.Tensor, nbrs: torch.Tensor, signs: np.ndarray, use_ip: bool = False,
           chunk_edges: int = 1 << 20):
    """Per-edge codes (n, deg, B/8) uint8 and factors (n, 3, deg) float32."""
    n = x.shape[0]
    deg = nbrs.shape[1]
    b = signs.shape[0]
    p, pos, weights = _encode_setup(signs, x.device)
    codes = torch.zeros((n, deg, b // 8), dtype=torch.uint8, device=x.device)
    factors = torch.zeros((n, 3, deg), dtype=torch.float32, device=x.device)
    rows = _encode_rows_per_chunk(deg, b, chunk_edges)
    for s in range(0, n, rows):
        e = min(n, s + rows)
        codes[s:e], factors[s:e] = _encode_chunk(x, nbrs[s:e], x[s:e], p, pos, weights, b, use_ip)
    return codes, factors


def entry_point(x: torch.Tensor, chunk: int = 1 << 20) -> int:
    """The node nearest the mean vector (float64), in row chunks."""
    n = x.shape[0]
    mu = torch.zeros(x.shape[1], dtype=torch.float64, device=x.device)
    for s in range(0, n, chunk):
        mu += x[s:s + chunk].to(torch.float64).sum(0)
    mu /= n
    best, best_d = 0, float("inf")
    for s in range(0, n, chunk):
        d = _sqnorm(x[s:s + chunk].to(torch.float64) - mu[None, :])
        i = int(torch.argmin(d).item())
        if float(d[i]) < best_d:
            best, best_d = s + i, float(d[i])
    return best


def build_codebook(base, degree: int, signs: np.ndarray, use_ip: bool = False,
                   device: str | torch.device = "cpu", random_links: int | None = None,
                   alpha: float = 1.0, candidates: int | None = None, fill_random: bool = True,
                   store_entry: bool = True, verbose: bool = False, knn_method: str = "exact",
                   connect: bool = False, stats: dict | None = None) -> Codebook:
    """Builds a complete codebook in the reference layout.  `base` is a numpy
    array or a float32 tensor (already on `device` for sets too large to
    hold twice).  connect=True: the RNG-pruned graph made reachable from the
    entry point (build_graph)."""
    x = _as_device(base, device)
    nbrs = build_graph(x, degree, random_links=random_links, alpha=alpha, candidates=candidates,
                       fill_random=fill_random, verbose=verbose, knn_method=knn_method, connect=connect,
                       stats=stats)
    return codebook_from_graph(x, nbrs, signs, use_ip=use_ip, device=device, store_entry=store_entry,
                               verbose=verbose)


def _as_device(base, device) -> torch.Tensor:
    if isinstance(base, torch.Tensor):
        return base.to(device=device, dtype=torch.float32)
    return torch.as_tensor(np.ascontiguousarray(base, dtype=np.float32), device=device)


def codebook_from_graph(base, nbrs, signs: np.ndarray, use_ip: bool = False,
                        device: str | torch.device = "cpu", store_entry: bool = True,
                        entry: int | None = None, verbose: bool = False) -> Codebook:
    """Encodes a given graph ((n, degree) neighbour ids, -1 = padding) into a
    codebook in the reference layout.  `entry` overrides the stored entry
    point (default: the node nearest the mean).  The host rows are filled one
    chunk of nodes at a time, so the device never holds more than a chunk's
    codes."""
    x = _as_device(base, device)
    n, dim = x.shape
    nbrs = torch.as_tensor(np.asarray(nbrs) if not isinstance(nbrs, torch.Tensor) else nbrs,
                           dtype=torch.int64, device=device)
    degree = int(nbrs.shape[1])
    lay = Layout.make(dim, degree)
    if signs.shape[0] != lay.padded_dim:
        raise ValueError("signs must have padded_dim entries")
    b = lay.padded_dim
    p, pos, weights = _encode_setup(signs, x.device)
    rows = np.zeros((n, lay.row_offset), dtype=np.float32)
    code_bytes = rows[:, lay.code_offset : lay.factor_offset].view(np.uint8)
    ids = rows[:, lay.neighbor_offset : lay.row_offset].view(np.uint32)
    step = _encode_rows_per_chunk(degree, b, 1 << 20)
    for s in range(0, n, step):
        e = min(n, s + step)
        nb = nbrs[s:e]
        codes, factors = _encode_chunk(x, nb, x[s:e], p, pos, weights, b, use_ip)
        rows[s:e, :dim] = x[s:e].cpu().numpy()
        code_bytes[s:e] = codes.cpu().numpy().reshape(e - s, -1)
        rows[s:e, lay.factor_offset : lay.neighbor_offset] = factors.cpu().numpy().reshape(e - s, -1)
        nbh = nb.cpu().numpy()
        ids[s:e] = np.where(nbh < 0, MAX_INDEX, nbh).astype(np.uint32)
        if verbose and (s // step) % 100 == 99:
            print(f"[builder] encoded {e}/{n} nodes", flush=True)
    if entry is None:
        entry = entry_point(x) if store_entry else MAX_INDEX
    return Codebook(rows, np.asarray(signs, dtype=np.float32), int(entry), lay)


def ground_truth(base, queries, k: int, device: str | torch.device = "cpu", use_ip: bool = False,
                 chunk_elems: int = 1 << 28) -> np.ndarray:
    """Exact top-k ids (int32) by L2 (or by -<q,x> for IP), ties by id."""
    b = _as_device(base, device)
    q = _as_device(queries, device)
    if not use_ip:
        ids, _ = knn(b, k, queries=q, exclude_self=False, chunk_elems=chunk_elems)
        return ids.cpu().numpy().astype(np.int32)
    out = []
    rows = max(1, chunk_elems // max(1, b.shape[0]))
    for s in range(0, q.shape[0], rows):
        d = -(q[s : s + rows] @ b.T)
        dv, di = torch.topk(d, min(b.shape[0], k + 16), dim=1, largest=False)
        o = torch.argsort(di, dim=1)
        di, dv = torch.gather(di, 1, o), torch.gather(dv, 1, o)
        o = torch.argsort(dv, dim=1, stable=True)
        out.append(torch.gather(di, 1, o)[:, :k].cpu().numpy())
    return np.concatenate(out).astype(np.int32)


def check_ground_truth(base, queries, gt: np.ndarray, sample: int = 32, use_ip: bool = False,
                       device: str | torch.device = "cpu") -> int:
    """Recomputes `sample` evenly spaced queries' distances to every base
    point one query at a time (a matrix-vector product, independent of the
    blocked products ground_truth uses) and returns how many of them have a
    ground-truth set whose largest distance exceeds that query's true k-th
    distance (0 for a correct ground truth, ties included)."""
    b = _as_device(base, device)
    q = _as_device(queries, device)
    k = gt.shape[1]
    bn = _sqnorm(b)
    bad = 0
    for i in np.linspace(0, q.shape[0] - 1, min(sample, q.shape[0])).astype(np.int64):
        d = -(b @ q[int(i)]) if use_ip else bn - 2.0 * (b @ q[int(i)])
        kth = torch.topk(d, k, largest=False).values.max()
        got = d[torch.as_tensor(gt[int(i)], device=b.device, dtype=torch.int64)].max()
        if float(got) > float(kth) + 1e-4 * max(1.0, abs(float(kth))):
            bad += 1
    return bad


def graph_stats(nbrs: np.ndarray) -> dict:
    valid = nbrs != MAX_INDEX
    return {"mean_degree": float(valid.sum(1).mean()), "min_degree": int(valid.sum(1).min())}


__all__ = ["knn", "knn_partitioned", "kmeans", "build_graph", "encode", "build_codebook", "ground_truth",
           "check_ground_truth", "entry_point",
           "hadamard_rotation", "graph_stats"]
