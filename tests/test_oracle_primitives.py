"""Pins the oracle's scalar helpers, query preparation, estimators, hash,
expander picking and distances against closed forms and hand-computed cases."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from oracle import oracle as O

FLT_MAX = float(np.finfo(np.float32).max)


def L():
    return O.lib()


# ---------------------------------------------------------------- sizing

@pytest.mark.parametrize("dim,deg,row,B", [(128, 32, 384, 128), (96, 32, 352, 128), (96, 16, 224, 128),
                                           (960, 32, 2112, 1024), (1536, 32, 3712, 2048), (100, 32, 356, 128)])
def test_layout(dim, deg, row, B):
    lay = O.Layout()
    assert L().fgo_compute_layout(dim, deg, C.byref(lay)) == 0
    assert lay.padded_dim == B and lay.row_offset == row
    assert lay.code_offset == dim
    assert lay.factor_offset == dim + (B // 64) * 2 * deg
    assert lay.neighbor_offset == lay.factor_offset + 3 * deg
    from flashgann_amd.codebook import Layout
    py = Layout.make(dim, deg)
    assert (py.row_offset, py.factor_offset, py.neighbor_offset) == (row, lay.factor_offset, lay.neighbor_offset)


def test_sizing_helpers():
    lib = L()
    assert [lib.fgo_effective_sort_beam_size(b) for b in (1, 16, 32, 33, 64, 100, 128, 129, 384, 1024)] == \
        [32, 32, 32, 64, 64, 128, 128, 129, 384, 1024]
    # hash bitlen is 11 at every benchmark beam (pbeam 32..1024, buffer 32,
    # reset interval 16: utils.cuh:137-151)
    for pb in (32, 64, 128, 256, 512, 1024):
        assert lib.fgo_hash_bitlen(pb, 32, 16) == 11
    assert [lib.fgo_candidate_buffer_capacity(d) for d in (1, 2, 3, 4, 16, 32, 64)] == [8, 16, 24, 32, 32, 32, 32]
    assert lib.fgo_max_rho_bound(32) == pytest.approx(0.875)
    assert lib.fgo_max_rho_bound(16) == pytest.approx(0.75)
    assert lib.fgo_max_rho_bound(4) == 0.0


def test_keep_counts_hand_computed():
    lib = L()
    assert lib.fgo_keep_count_per_parent(32, 0.25) == 24
    assert lib.fgo_keep_count_per_parent(32, 0.875) == 4
    assert lib.fgo_keep_count_per_parent(32, 1.5) == 1
    assert lib.fgo_keep_count_per_parent(32, -0.5) == 32
    assert lib.fgo_keep_count_per_parent(10, 0.33) == 7          # ceil(6.7)
    # stage I: theta 1, rho 0.25 -> min(24, 32) = 24
    assert lib.fgo_keep_count_for_expander(32, 1, 0.25, 0, 0) == 24
    # stage II: theta 8 caps at 32/8 = 4
    assert lib.fgo_keep_count_for_expander(32, 8, 0.875, 0, 0) == 4
    assert lib.fgo_keep_count_for_expander(32, 8, 0.0, 0, 0) == 4
    # kth cutoff clamps to the near count, at least 1
    assert lib.fgo_keep_count_for_expander(32, 1, 0.25, 1, 3) == 3
    assert lib.fgo_keep_count_for_expander(32, 1, 0.25, 1, 0) == 1
    assert lib.fgo_keep_count_for_expander(32, 1, 0.25, 1, 99) == 24
    # a short tile (deg 40, second tile has 8) clamps to its active count
    assert lib.fgo_keep_count_for_expander(8, 8, 0.875, 0, 0) == 1
    # the per-parent budget is BUFFER_BOUND / theta rounded down
    # (adaptive_search_utils.cuh:126): 32 / 3 = 10, 32 / 5 = 6, 32 / 6 = 5
    assert lib.fgo_keep_count_for_expander(32, 3, 0.0, 0, 0) == 10
    assert lib.fgo_keep_count_for_expander(32, 5, 0.0, 0, 0) == 6
    assert lib.fgo_keep_count_for_expander(32, 6, 0.0, 0, 0) == 5


# ---------------------------------------------------------------- FWHT

def sylvester(b):
    i = np.arange(b)
    a = i[:, None] & i[None, :]
    par = np.zeros_like(a)
    while a.any():
        par ^= a & 1
        a >>= 1
    return (1 - 2 * par).astype(np.float64)


@pytest.mark.parametrize("dim,B", [(128, 128), (96, 128), (33, 64), (960, 1024)])
def test_rotation_is_hadamard_times_signs(dim, B):
    rng = np.random.default_rng(dim)
    x = rng.integers(-200, 200, dim).astype(np.float32)
    s = np.where(rng.random(B) < 0.5, -1.0, 1.0).astype(np.float32)
    out = np.zeros(B, np.float32)
    L().fgo_rotate(O.ptr(x, C.c_float), O.ptr(s, C.c_float), dim, B, O.ptr(out, C.c_float))
    xp = np.zeros(B)
    xp[:dim] = x * s[:dim]
    ref = sylvester(B) @ xp
    assert np.array_equal(out.astype(np.float64), ref)      # integers: exact


def test_rotation_float_close():
    rng = np.random.default_rng(1)
    x = rng.standard_normal(96).astype(np.float32)
    s = np.ones(128, np.float32)
    out = np.zeros(128, np.float32)
    L().fgo_rotate(O.ptr(x, C.c_float), O.ptr(s, C.c_float), 96, 128, O.ptr(out, C.c_float))
    xp = np.zeros(128)
    xp[:96] = x
    np.testing.assert_allclose(out, sylvester(128) @ xp, rtol=1e-5, atol=1e-4)


# ---------------------------------------------------------------- quantizer / LUT

def _prep(x, s, dim, B):
    return O.query_prepare(x, s, dim, B)


@pytest.mark.parametrize("seed", range(5))
@pytest.mark.parametrize("dim,B", [(128, 128), (96, 128), (40, 64)])
def test_quantizer_closed_form(seed, dim, B):
    """Range, width, levels and LUT over all B rotated entries (utils.cuh:
    840-939; the zero-padded dimensions of a d < B query are rotated too)."""
    rng = np.random.default_rng(seed)
    x = rng.integers(0, 150, dim).astype(np.float32)
    s = np.where(rng.random(B) < 0.5, -1.0, 1.0).astype(np.float32)
    qf = _prep(x, s, dim, B)
    y = np.ctypeslib.as_array(qf.rotated)[:B].astype(np.float32)
    q = np.ctypeslib.as_array(qf.q)[:B].astype(np.int64)
    lo, hi = y.min(), y.max()
    assert np.float32(qf.low) == lo and np.float32(qf.high) == hi
    width = np.float32(np.float32(hi - lo) * np.float32(1.0 / 63.0))
    assert np.float32(qf.width) == width
    inv = np.float32(np.float32(1.0) / width)
    # fma(y-lo, inv, 0.5) in float64 then rounded is the exact fused result here
    scaled = (np.float64(y - lo) * np.float64(inv) + 0.5).astype(np.float32)
    ref_q = np.floor(scaled.astype(np.float64) + 0.5).astype(np.int64)
    assert np.array_equal(q, ref_q)
    assert q.min() >= 1 and q.max() <= 64
    assert qf.sum_q == int(q.sum())
    lut = np.ctypeslib.as_array(qf.lut)[: 4 * B].reshape(B // 4, 16)
    for cb in range(B // 4):
        for m in range(16):
            tot = sum(int(q[4 * cb + j]) for j in range(4) if m & (8 >> j))
            assert lut[cb, m] == tot % 256


def test_lut_wraps_like_uint8():
    """A chunk of four 64s has full-nibble LUT entry 256 mod 256 = 0 (Q1).

    With z non-zero only at multiples of 4, H z is constant on every 4-dim
    chunk, and x = s * z makes the rotation exact (y = H z), so whole chunks
    reach the top level together."""
    B = 64
    rng = np.random.default_rng(12)
    s = np.where(rng.random(B) < 0.5, -1.0, 1.0).astype(np.float32)
    for _ in range(500):
        z = np.zeros(B, np.float32)
        z[::4] = rng.integers(-40, 60, B // 4)
        x = (s * z).astype(np.float32)
        qf = _prep(x, s, B, B)
        q = np.ctypeslib.as_array(qf.q)[:B].astype(np.int64)
        full = np.nonzero((q.reshape(-1, 4) == 64).all(1))[0]
        if full.size:
            break
    assert full.size, "no seed produced a chunk of four 64s"
    cb = int(full[0])
    lut = np.ctypeslib.as_array(qf.lut)[: 4 * B].reshape(B // 4, 16)
    assert lut[cb, 15] == 0 and lut[cb, 7] == 192
    code = np.zeros(B // 8, np.uint8)
    code[cb >> 1] = 0x0F if cb % 2 == 0 else 0xF0
    assert L().fgo_raw_lut(C.byref(qf), O.ptr(code, C.c_uint8), B) == 0
    # the bit-plane identity minus the wrap correction gives the same raw
    from flashgann_amd.codebook import unpack_codes
    bits = unpack_codes(code)
    assert int((bits * q).sum()) - 256 == 0


@pytest.mark.parametrize("B", [64, 128, 1024])
def test_raw_equals_bitplane_popcount(B):
    """raw = sum_i b_i q_i (bits in the code's nibble layout) whenever no chunk
    wraps: the identity the GPU's popcount planes rely on."""
    from flashgann_amd.codebook import pack_codes
    rng = np.random.default_rng(B)
    x = rng.standard_normal(B).astype(np.float32)
    s = np.where(rng.random(B) < 0.5, -1.0, 1.0).astype(np.float32)
    qf = _prep(x, s, B, B)
    q = np.ctypeslib.as_array(qf.q)[:B].astype(np.int64)
    for _ in range(20):
        bits = rng.integers(0, 2, B).astype(np.uint8)
        code = pack_codes(bits)
        raw = L().fgo_raw_lut(C.byref(qf), O.ptr(code, C.c_uint8), B)
        chunks = q.reshape(-1, 4)
        wraps = int(((chunks.sum(1) >= 256) & (bits.reshape(-1, 4).sum(1) == 4)).sum())
        assert raw == int((bits * q).sum()) - 256 * wraps


def test_estimator_formula_and_special_cases():
    rng = np.random.default_rng(9)
    B = 128
    x = rng.standard_normal(B).astype(np.float32)
    s = np.ones(B, np.float32)
    qf = _prep(x, s, B, B)
    code = rng.integers(0, 256, B // 8).astype(np.uint8)
    raw = L().fgo_raw_lut(C.byref(qf), O.ptr(code, C.c_uint8), B)
    tx, fdq, fvq, pd = np.float32(3.5), np.float32(-0.25), np.float32(1.5), np.float32(10.0)
    got = L().fgo_estimate_seq(C.byref(qf), O.ptr(code, C.c_uint8), tx, fdq, fvq, pd, B)
    rf = np.float32(2 * raw - qf.sum_q)
    e = np.float32(tx + pd)
    e = np.float32(np.float64(np.float32(fdq * np.float32(qf.width))) * np.float64(rf) + np.float64(e))
    e = np.float32(np.float64(fvq) * np.float64(np.float32(qf.low)) + np.float64(e))
    assert np.float32(got) == e
    assert L().fgo_estimate_lanes(C.byref(qf), O.ptr(code, C.c_uint8), FLT_MAX, fdq, fvq, pd, B) == 0.0
    assert L().fgo_estimate_seq(C.byref(qf), O.ptr(code, C.c_uint8), FLT_MAX, fdq, fvq, pd, B) == FLT_MAX


# ---------------------------------------------------------------- distances

def test_warp_distances():
    rng = np.random.default_rng(4)
    for dim in (33, 96, 128, 960, 1536):
        a = rng.standard_normal(dim).astype(np.float32)
        b = rng.standard_normal(dim).astype(np.float32)
        l2 = L().fgo_warp_l2(dim, O.ptr(a, C.c_float), O.ptr(b, C.c_float))
        ip = L().fgo_warp_ip(dim, O.ptr(a, C.c_float), O.ptr(b, C.c_float))
        ref = float(((a.astype(np.float64) - b) ** 2).sum())
        assert abs(l2 - ref) <= 1e-5 * ref
        refip = -float((a.astype(np.float64) * b).sum())
        assert abs(ip - refip) <= 1e-5 * np.abs(a.astype(np.float64) * b).sum()
        ai = rng.integers(0, 200, dim).astype(np.float32)
        bi = rng.integers(0, 200, dim).astype(np.float32)
        assert L().fgo_warp_l2(dim, O.ptr(ai, C.c_float), O.ptr(bi, C.c_float)) == float(((ai.astype(np.int64) - bi.astype(np.int64)) ** 2).sum())


def _tree32(v):
    """shfl_down tree of utils.cuh:277-281 / 292-296 over 32 float32 lane
    sums: offsets 16, 8, 4, 2, 1, lane l adding lane l + offset."""
    v = np.asarray(v, np.float32).copy()
    off = 16
    while off:
        v[:off] = v[:off] + v[off:2 * off]
        off //= 2
    return v[0]


def test_warp_distances_reduction_tree_bit_exact():
    """At d = 32 each lane holds one product, rounded once to float32 (the
    fmaf with a zero addend; float64 holds the product exactly), so the
    distance is exactly the shfl_down tree over those 32 values in float32.
    Random floats make the tree's sum differ in its last bits from other
    orders (sequential, pairwise from the other end) in most trials, so the
    order is pinned bit for bit."""
    rng = np.random.default_rng(9)
    differs = 0
    for _ in range(50):
        a = rng.standard_normal(32).astype(np.float32)
        b = rng.standard_normal(32).astype(np.float32)
        d = (a - b).astype(np.float32)
        sq = (d.astype(np.float64) ** 2).astype(np.float32)
        pr = (a.astype(np.float64) * b.astype(np.float64)).astype(np.float32)
        want_l2, want_ip = _tree32(sq), -_tree32(pr)
        assert np.float32(L().fgo_warp_l2(32, O.ptr(a, C.c_float), O.ptr(b, C.c_float))) == want_l2
        assert np.float32(L().fgo_warp_ip(32, O.ptr(a, C.c_float), O.ptr(b, C.c_float))) == want_ip
        seq = np.float32(0)
        for x in sq:
            seq = np.float32(seq + x)
        differs += seq != want_l2
    assert differs >= 10


# ---------------------------------------------------------------- hash / pick

def test_hash_set_semantics():
    rng = np.random.default_rng(2)
    bitlen = 11
    t = np.full(1 << bitlen, 0xFFFFFFFF, np.uint32)
    seen = set()
    for key in rng.integers(0, 5000, 1400):
        key = int(key)
        new = L().fgo_hash_insert(O.ptr(t, C.c_uint32), bitlen, key)
        assert new == (key not in seen)
        seen.add(key)
    for key in range(0, 6000, 7):
        assert L().fgo_hash_contains(O.ptr(t, C.c_uint32), bitlen, key) == (key in seen)
    # slot of a key is (k ^ (k >> bitlen)) & mask when free
    t2 = np.full(1 << bitlen, 0xFFFFFFFF, np.uint32)
    L().fgo_hash_insert(O.ptr(t2, C.c_uint32), bitlen, 123456)
    assert t2[(123456 ^ (123456 >> bitlen)) & ((1 << bitlen) - 1)] == 123456


def test_pick_expanders():
    beam = np.array([5, 7 | 0x80000000, 9, 11, 0xFFFFFFFF, 13], dtype=np.uint32)
    out = np.zeros(8, np.uint32)
    n = L().fgo_pick_expanders(2, O.ptr(out, C.c_uint32), 6, O.ptr(beam, C.c_uint32))
    assert n == 2 and list(out[:2]) == [0, 2]
    assert beam[0] & 0x80000000 and beam[2] & 0x80000000 and not beam[3] & 0x80000000
    n = L().fgo_pick_expanders(8, O.ptr(out, C.c_uint32), 6, O.ptr(beam, C.c_uint32))
    assert n == 2 and list(out[:2]) == [3, 5]
    n = L().fgo_pick_expanders(8, O.ptr(out, C.c_uint32), 6, O.ptr(beam, C.c_uint32))
    assert n == 0
    # more than 32 entries: chunks of 32, order preserved
    big = np.arange(100, dtype=np.uint32)
    big[:40] |= 0x80000000
    n = L().fgo_pick_expanders(3, O.ptr(out, C.c_uint32), 100, O.ptr(big, C.c_uint32))
    assert n == 3 and list(out[:3]) == [40, 41, 42]


def test_keep_topk_single_keep_over_a_tie_takes_the_lower_lane():
    """warp_keep_topk_smallest_f32 (utils.cuh:251-267) ranks a lane by the
    valid lanes with a smaller value or an equal value in a lower lane: with
    keep 1 over equal minima in lanes 5 and 17 (lane 9, also at the minimum,
    is invalid), only lane 5 is kept; with keep 2 lanes 5 and 17."""
    vals = np.full(32, 50.0, np.float32)
    vals[[5, 9, 17]] = 7.0
    vals[30] = 8.0
    valid = np.ones(32, np.int32)
    valid[9] = 0
    keep = np.zeros(32, np.int32)
    call = lambda k: L().fgo_warp_keep_topk(O.ptr(vals, C.c_float), valid.ctypes.data_as(C.POINTER(C.c_int)), k,
                                            keep.ctypes.data_as(C.POINTER(C.c_int)))
    assert call(1) == 1 and list(np.nonzero(keep)[0]) == [5]
    assert call(2) == 2 and list(np.nonzero(keep)[0]) == [5, 17]
    assert call(3) == 3 and list(np.nonzero(keep)[0]) == [5, 17, 30]


def test_keep_topk_rank_ties_by_lane():
    vals = np.array([3, 1, 1, 2] + [9] * 28, np.float32)
    valid = np.array([1, 1, 1, 1] + [0] * 28, np.int32)
    keep = np.zeros(32, np.int32)
    n = L().fgo_warp_keep_topk(O.ptr(vals, C.c_float), valid.ctypes.data_as(C.POINTER(C.c_int)), 2,
                               keep.ctypes.data_as(C.POINTER(C.c_int)))
    assert n == 2 and list(np.nonzero(keep)[0]) == [1, 2]
    n = L().fgo_warp_keep_topk(O.ptr(vals, C.c_float), valid.ctypes.data_as(C.POINTER(C.c_int)), 3,
                               keep.ctypes.data_as(C.POINTER(C.c_int)))
    assert list(np.nonzero(keep)[0]) == [1, 2, 3]
