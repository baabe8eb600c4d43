"""ctypes binding of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker.  The product package never
imports it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# FG_ORACLE_LIB names another build of fg_oracle.c (the mutation tests load
# deliberately broken copies through it)
LIB_PATH = os.environ.get("FG_ORACLE_LIB") or os.path.join(HERE, "liboracle.so")
REF_LIB_PATH = os.path.join(HERE, "_ref", "libfg_ref_host.so")

MAX_INDEX = 0xFFFFFFFF
MAX_PADDED_DIM = 2048


class Layout(C.Structure):
    _fields_ = [("dim", C.c_uint32), ("padded_dim", C.c_uint32), ("degree", C.c_uint32),
                ("code_offset", C.c_uint64), ("factor_offset", C.c_uint64),
                ("neighbor_offset", C.c_uint64), ("row_offset", C.c_uint64)]


class Index(C.Structure):
    _fields_ = [("data", C.POINTER(C.c_float)), ("signs", C.POINTER(C.c_float)),
                ("npoints", C.c_uint64), ("lay", Layout), ("entry", C.c_uint32),
                ("use_ip", C.c_int)]


class QueryFactors(C.Structure):
    _fields_ = [("rotated", C.c_float * MAX_PADDED_DIM), ("q", C.c_uint8 * MAX_PADDED_DIM),
                ("lut", C.c_uint8 * (4 * MAX_PADDED_DIM)), ("low", C.c_float),
                ("high", C.c_float), ("width", C.c_float), ("sum_q", C.c_int32)]


class Counters(C.Structure):
    _fields_ = [("iterations", C.c_uint32), ("expansions", C.c_uint32), ("ids_read", C.c_uint32),
                ("estimates", C.c_uint32), ("exact", C.c_uint32), ("stage2_iter", C.c_uint32)]


class TraceRec(C.Structure):
    _fields_ = [("iter", C.c_uint32), ("theta", C.c_uint32), ("rho", C.c_float),
                ("n_parents", C.c_uint32), ("parents", C.c_uint32 * 8), ("top1", C.c_uint32),
                ("top1_dist", C.c_float), ("kth_cutoff", C.c_float), ("n_cand", C.c_uint32),
                ("cand_idx", C.c_uint32 * 32), ("cand_dist", C.c_float * 32),
                ("stall", C.c_int32), ("last_expander_distance", C.c_float),
                ("current_expander_distance", C.c_float), ("restored", C.c_uint32)]


class CtlState(C.Structure):
    _fields_ = [("spec_degree", C.c_int), ("rho", C.c_float), ("policy_iters", C.c_int),
                ("top1_node", C.c_uint32), ("top1_stall_iters", C.c_int), ("warmup_done", C.c_int),
                ("entry_distance", C.c_float), ("last_expander_distance", C.c_float),
                ("current_expander_distance", C.c_float)]


COUNTER_DTYPE = np.dtype([(n, np.uint32) for n, _ in Counters._fields_])

_lib = None
_ref = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE, "all"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        f32p, u32p, u8p = C.POINTER(C.c_float), C.POINTER(C.c_uint32), C.POINTER(C.c_uint8)
        L.fgo_compute_layout.argtypes = [C.c_uint32, C.c_uint32, C.POINTER(Layout)]
        L.fgo_round_up_pow2.argtypes = [C.c_uint32]
        L.fgo_round_up_pow2.restype = C.c_uint32
        L.fgo_effective_sort_beam_size.argtypes = [C.c_uint32]
        L.fgo_effective_sort_beam_size.restype = C.c_uint32
        L.fgo_hash_bitlen.argtypes = [C.c_uint32] * 3
        L.fgo_hash_bitlen.restype = C.c_uint32
        L.fgo_candidate_buffer_capacity.argtypes = [C.c_uint32]
        L.fgo_candidate_buffer_capacity.restype = C.c_uint32
        L.fgo_max_rho_bound.argtypes = [C.c_uint32]
        L.fgo_max_rho_bound.restype = C.c_float
        L.fgo_keep_count_per_parent.argtypes = [C.c_uint32, C.c_float]
        L.fgo_keep_count_per_parent.restype = C.c_uint32
        L.fgo_keep_count_for_expander.argtypes = [C.c_uint32, C.c_int, C.c_float, C.c_int, C.c_uint32]
        L.fgo_keep_count_for_expander.restype = C.c_int
        L.fgo_rotate.argtypes = [f32p, f32p, C.c_int, C.c_int, f32p]
        L.fgo_query_prepare.argtypes = [f32p, f32p, C.c_int, C.c_int, C.POINTER(QueryFactors)]
        L.fgo_raw_lut.argtypes = [C.POINTER(QueryFactors), u8p, C.c_int]
        L.fgo_raw_lut.restype = C.c_uint32
        for name in ("fgo_estimate_lanes", "fgo_estimate_seq"):
            fn = getattr(L, name)
            fn.argtypes = [C.POINTER(QueryFactors), u8p, C.c_float, C.c_float, C.c_float, C.c_float, C.c_int]
            fn.restype = C.c_float
        for name in ("fgo_warp_l2", "fgo_warp_ip", "fgo_scalar_l2", "fgo_scalar_ip"):
            fn = getattr(L, name)
            fn.argtypes = [C.c_int, f32p, f32p]
            fn.restype = C.c_float
        L.fgo_bitonic_sort.argtypes = [f32p, u32p, C.c_uint32]
        L.fgo_bitonic_stage.argtypes = [f32p, u32p, C.c_uint32, C.c_uint32]
        L.fgo_merge_candidates.argtypes = [f32p, u32p, f32p, u32p, C.c_uint32, C.c_uint32, C.c_int, f32p, u32p]
        L.fgo_merge_path_partition.argtypes = [f32p, C.c_int, f32p, C.c_int, C.c_int]
        L.fgo_merge_path_partition.restype = C.c_int
        L.fgo_hash_insert.argtypes = [u32p, C.c_uint, C.c_uint32]
        L.fgo_hash_insert.restype = C.c_uint32
        L.fgo_hash_contains.argtypes = [u32p, C.c_uint, C.c_uint32]
        L.fgo_hash_contains.restype = C.c_uint32
        L.fgo_pick_expanders.argtypes = [C.c_int, u32p, C.c_int, u32p]
        L.fgo_pick_expanders.restype = C.c_uint32
        L.fgo_warp_keep_topk.argtypes = [f32p, C.POINTER(C.c_int), C.c_int, C.POINTER(C.c_int)]
        L.fgo_warp_keep_topk.restype = C.c_int
        L.fgo_ctl_init.argtypes = [C.POINTER(CtlState), C.c_float]
        L.fgo_controller_step.argtypes = [C.POINTER(CtlState), C.c_uint32, C.c_float]
        L.fgo_record_expander.argtypes = [C.POINTER(CtlState), f32p, C.c_uint32]
        L.fgo_kth_cutoff.argtypes = [C.c_int, C.c_int, u32p, f32p]
        L.fgo_kth_cutoff.restype = C.c_float
        L.fgo_search_one.argtypes = [C.POINTER(Index), f32p, C.c_int, C.c_int, u32p, C.POINTER(Counters),
                                     C.POINTER(TraceRec), C.c_uint32, u32p]
        L.fgo_search_one.restype = C.c_int
        L.fgo_search_batch.argtypes = [C.POINTER(Index), f32p, C.c_uint64, C.c_int, C.c_int, u32p,
                                       C.c_void_p, C.c_int]
        L.fgo_search_batch.restype = C.c_int
        L.fgo_entry_point.argtypes = [f32p, C.c_uint64, C.c_uint32, C.c_uint64, C.c_int]
        L.fgo_entry_point.restype = C.c_uint32
        L.fgo_recall.argtypes = [u32p, C.POINTER(C.c_int32), C.c_uint64, C.c_int, C.c_int]
        L.fgo_recall.restype = C.c_float
        _lib = L
    return _lib


def ref_lib():
    """The reference's own host helpers, or None where they were not built."""
    global _ref
    if _ref is None and os.path.exists(REF_LIB_PATH):
        R = C.CDLL(REF_LIB_PATH)
        R.ref_compute_recall.argtypes = [C.POINTER(C.c_uint32), C.POINTER(C.c_int), C.c_uint64, C.c_int, C.c_int]
        R.ref_compute_recall.restype = C.c_float
        R.ref_compute_entry_point.argtypes = [C.POINTER(C.c_float), C.c_uint64, C.c_uint64, C.c_uint64, C.c_int]
        R.ref_compute_entry_point.restype = C.c_uint32
        R.ref_infer_metric_is_ip.argtypes = [C.c_char_p]
        R.ref_infer_metric_is_ip.restype = C.c_int
        R.ref_load_fvecs.argtypes = [C.c_char_p, C.POINTER(C.c_int), C.POINTER(C.c_float), C.c_uint64]
        R.ref_load_fvecs.restype = C.c_uint64
        R.ref_load_ivecs.argtypes = [C.c_char_p, C.POINTER(C.c_int), C.POINTER(C.c_int), C.c_uint64]
        R.ref_load_ivecs.restype = C.c_uint64
        R.ref_qg_load.argtypes = [C.c_char_p, C.c_uint64, C.c_uint64, C.c_int, C.POINTER(C.c_uint64),
                                  C.POINTER(C.c_uint32), C.POINTER(C.c_float), C.c_uint64,
                                  C.POINTER(C.c_float), C.c_uint64]
        R.ref_qg_load.restype = C.c_int
        _ref = R
    return _ref


def ptr(a: np.ndarray, ctype):
    return a.ctypes.data_as(C.POINTER(ctype))


class OracleIndex:
    """Holds numpy buffers alive for an fgo_index."""

    def __init__(self, rows: np.ndarray, signs: np.ndarray, dim: int, degree: int, entry: int,
                 use_ip: bool = False):
        self.rows = np.ascontiguousarray(rows, dtype=np.float32)
        self.signs = np.ascontiguousarray(signs, dtype=np.float32)
        lay = Layout()
        if lib().fgo_compute_layout(dim, degree, C.byref(lay)) != 0:
            raise ValueError("bad layout")
        if self.rows.shape[1] != lay.row_offset:
            raise ValueError("row width does not match layout")
        self.ix = Index(ptr(self.rows, C.c_float), ptr(self.signs, C.c_float), self.rows.shape[0],
                        lay, entry, 1 if use_ip else 0)

    @classmethod
    def from_codebook(cls, cb, use_ip: bool = False, entry: int | None = None):
        e = cb.entry if entry is None else entry
        return cls(cb.rows, cb.signs, cb.layout.dim, cb.layout.degree, e, use_ip)

    def search_one(self, query: np.ndarray, K: int, beam: int, trace_cap: int = 0):
        q = np.ascontiguousarray(query, dtype=np.float32)
        out = np.zeros(K, dtype=np.uint32)
        cnt = Counters()
        tr = (TraceRec * trace_cap)() if trace_cap else None
        tl = C.c_uint32(0)
        rc = lib().fgo_search_one(C.byref(self.ix), ptr(q, C.c_float), K, beam, ptr(out, C.c_uint32),
                                  C.byref(cnt), tr, trace_cap, C.byref(tl))
        if rc != 0:
            raise ValueError(f"oracle search failed: {rc}")
        return out, cnt, (list(tr)[: tl.value] if tr is not None else None)

    def search(self, queries: np.ndarray, K: int, beam: int, threads: int = 0):
        q = np.ascontiguousarray(queries, dtype=np.float32)
        nq = q.shape[0]
        out = np.zeros((nq, K), dtype=np.uint32)
        cnt = np.zeros(nq, dtype=COUNTER_DTYPE)
        threads = threads or os.cpu_count() or 1
        rc = lib().fgo_search_batch(C.byref(self.ix), ptr(q, C.c_float), nq, K, beam,
                                    ptr(out, C.c_uint32), cnt.ctypes.data_as(C.c_void_p), threads)
        if rc != 0:
            raise ValueError(f"oracle batch search failed: {rc}")
        return out, cnt


def query_prepare(query: np.ndarray, signs: np.ndarray, dim: int, padded_dim: int) -> QueryFactors:
    qf = QueryFactors()
    q = np.ascontiguousarray(query, dtype=np.float32)
    s = np.ascontiguousarray(signs, dtype=np.float32)
    lib().fgo_query_prepare(ptr(q, C.c_float), ptr(s, C.c_float), dim, padded_dim, C.byref(qf))
    return qf


def recall(pred: np.ndarray, gt: np.ndarray, K: int) -> float:
    p = np.ascontiguousarray(pred, dtype=np.uint32)
    g = np.ascontiguousarray(gt, dtype=np.int32)
    return float(lib().fgo_recall(ptr(p, C.c_uint32), ptr(g, C.c_int32), p.shape[0], K, g.shape[1]))
