"""flashgann_amd -- FlashGANN's adaptive graph beam search on MI355X.

Host-side mirror of the reference's search interface:
  QuantizationGraph(num_node, dim, degree, codebook_path)   include/qg.hpp:17-42
  .set_metric / .get_metric                                 include/qg.hpp:53-54
  .gpu_search_adaptive(nq, queries, K, result_idx, beam_sz) gpu_search_adaptive.cu:12-114
      -> elapsed seconds (the reference returns it through `double &elapsed`)
plus `Index`, a handle that keeps the codebook resident on the GPU across
calls, and `search_device` for torch tensors already in HBM.
All compute goes through libflashgann.so (HIP, gfx950).
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from . import _lib
from ._lib import (FG_COUNTERS_PER_QUERY, FG_ENTRY_AUTO, FG_METRIC_IP, FG_METRIC_L2,
                   FG_PROFILE_SLOTS, FlashGannError, IndexInfo, Stats, check, lib)
from .codebook import Codebook, Layout, read_codebook

METRIC_L2 = FG_METRIC_L2
METRIC_IP = FG_METRIC_IP
COUNTER_FIELDS = ("iterations", "expansions", "ids_read", "estimates", "exact", "stage2_iter")

__all__ = ["Index", "QuantizationGraph", "FlashGannError", "METRIC_L2", "METRIC_IP",
           "infer_metric_from_dataset_path", "metric_name", "lds_bytes", "COUNTER_FIELDS"]


def _fptr(a: np.ndarray):
    return a.ctypes.data_as(C.POINTER(C.c_float))


def _uptr(a: np.ndarray):
    return a.ctypes.data_as(C.POINTER(C.c_uint32))


def infer_metric_from_dataset_path(path: str) -> int:
    """include/metric.hpp:13-28: IP iff the lower-cased path contains
    "text2image1m"."""
    return METRIC_IP if "text2image1m" in (path or "").lower() else METRIC_L2


def metric_name(metric: int) -> str:
    """include/metric.hpp:30-32"""
    return "ip" if metric == METRIC_IP else "l2"


def lds_bytes(dim: int, beam: int, degree: int) -> int:
    return int(lib().fg_lds_bytes(dim, beam, degree))


class Index:
    """A codebook resident in device memory (fg_index_create / fg_index_load)."""

    def __init__(self, handle: C.c_void_p):
        self._h = handle
        info = IndexInfo()
        check(lib().fg_index_get_info(self._h, C.byref(info)))
        self.info = info

    @classmethod
    def from_rows(cls, rows: np.ndarray, signs: np.ndarray, dim: int, degree: int,
                  entry: int = FG_ENTRY_AUTO, metric: int = METRIC_L2) -> "Index":
        rows = np.ascontiguousarray(rows, dtype=np.float32)
        signs = np.ascontiguousarray(signs, dtype=np.float32)
        h = C.c_void_p()
        check(lib().fg_index_create(_fptr(rows), rows.shape[0], dim, degree, _fptr(signs),
                                    entry & 0xFFFFFFFF, metric, C.byref(h)))
        return cls(h)

    @classmethod
    def from_codebook(cls, cb: Codebook, metric: int = METRIC_L2, entry: int | None = None) -> "Index":
        return cls.from_rows(cb.rows, cb.signs, cb.layout.dim, cb.layout.degree,
                             cb.entry if entry is None else entry, metric)

    @classmethod
    def load(cls, path: str, npoints: int, dim: int, degree: int, metric: int = METRIC_L2) -> "Index":
        h = C.c_void_p()
        check(lib().fg_index_load(path.encode(), npoints, dim, degree, metric, C.byref(h)))
        return cls(h)

    def close(self) -> None:
        if self._h:
            lib().fg_index_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def entry(self) -> int:
        return int(self.info.entry)

    def _host_queries(self, queries) -> np.ndarray:
        """(nq, dim) float32 C-contiguous; a single 1-D query becomes (1, dim)."""
        q = np.ascontiguousarray(queries, dtype=np.float32)
        if q.ndim == 1:
            q = q.reshape(1, -1)
        if q.ndim != 2 or q.shape[1] != int(self.info.dim):
            raise ValueError(f"queries must have shape (nq, {int(self.info.dim)}), got {tuple(np.shape(queries))}")
        return q

    def search(self, queries: np.ndarray, K: int, beam: int, counters: bool = False, noalloc: bool = False):
        """Host queries in, host ids out.  Returns (ids, Stats, counters|None).
        noalloc=True calls fg_search_noalloc (staging in the library's fixed
        per-device area, no device allocation; at most
        FG_NOALLOC_STAGING_BYTES of staging per call)."""
        q = self._host_queries(queries)
        nq = q.shape[0]
        out = np.zeros((nq, K), dtype=np.uint32)
        cnt = np.zeros((nq, FG_COUNTERS_PER_QUERY), dtype=np.uint32) if counters else None
        st = Stats()
        fn = lib().fg_search_noalloc if noalloc else lib().fg_search
        check(fn(self._h, _fptr(q), nq, K, beam, _uptr(out), _uptr(cnt) if cnt is not None else None,
                 C.byref(st)))
        return out, st, cnt

    def search_device(self, queries_ptr: int, nq: int, K: int, beam: int, results_ptr: int,
                      counters_ptr: int = 0, stream: int = 0) -> None:
        """Device pointers (e.g. torch tensor .data_ptr()); async on `stream`."""
        check(lib().fg_search_device(self._h, C.c_void_p(queries_ptr), nq, K, beam,
                                     C.c_void_p(results_ptr), C.c_void_p(counters_ptr or None),
                                     C.c_void_p(stream or None)))

    def search_waves(self, nq: int, K: int, beam: int) -> int:
        """Waves per query (1, or 2 for the kernel's team form) that a search
        of nq queries at this K and beam launches (fg_search_waves)."""
        w = lib().fg_search_waves(self._h, nq, K, beam)
        check(w if w < 0 else 0)
        return w

    def search_launches(self, nq: int, K: int, beam: int) -> int:
        """Kernel launches (1, or 2 for the two-launch schedule: every query
        to iteration 15, then the unfinished ones resumed longest-expected
        first) that a search of nq queries at this K and beam makes
        (fg_search_launches)."""
        n = lib().fg_search_launches(self._h, nq, K, beam)
        check(n if n < 0 else 0)
        return n

    def search_geometry(self) -> int:
        """0 when the kernels specialised for this shape (32-bit row offsets)
        serve searches on this index, 1 for the general kernels (runtime
        offsets, 64-bit row addresses) (fg_search_geometry)."""
        g = lib().fg_search_geometry(self._h)
        check(g if g < 0 else 0)
        return g

    def search_stream(self, queries_ptr: int, nq: int, K: int, beam: int, results_ptr: int,
                      batch: int, nstreams: int = 2, stream: int = 0) -> None:
        """Device pointers; the nq queries searched as batches of `batch` on
        `nstreams` internal streams (fg_search_stream), ordered after prior
        work on `stream` and before its later work."""
        check(lib().fg_search_stream(self._h, C.c_void_p(queries_ptr), nq, K, beam, C.c_void_p(results_ptr),
                                     batch, nstreams, C.c_void_p(stream or None)))

    def search_profile(self, queries_ptr: int, nq: int, K: int, beam: int, results_ptr: int,
                       phase_ptr: int, stream: int = 0) -> None:
        """Profiling build of the search: per query, 10 uint64 phase-cycle sums
        followed by the start and end time on the 100 MHz device clock
        (FG_PROFILE_SLOTS values)."""
        check(lib().fg_search_profile(self._h, C.c_void_p(queries_ptr), nq, K, beam,
                                      C.c_void_p(results_ptr), C.c_void_p(phase_ptr),
                                      C.c_void_p(stream or None)))

    def query_prepare(self, queries: np.ndarray):
        q = self._host_queries(queries)
        nq, b = q.shape[0], int(self.info.padded_dim)
        rot = np.zeros((nq, b), dtype=np.float32)
        qt = np.zeros((nq, b), dtype=np.uint8)
        lhw = np.zeros((nq, 3), dtype=np.float32)
        sq = np.zeros(nq, dtype=np.int32)
        check(lib().fg_query_prepare(self._h, _fptr(q), nq, _fptr(rot),
                                     qt.ctypes.data_as(C.POINTER(C.c_uint8)), _fptr(lhw),
                                     sq.ctypes.data_as(C.POINTER(C.c_int32))))
        return rot, qt, lhw, sq

    def score_edges(self, queries: np.ndarray, query_ix, parents, slots):
        q = self._host_queries(queries)
        qi = np.ascontiguousarray(query_ix, dtype=np.uint32)
        pa = np.ascontiguousarray(parents, dtype=np.uint32)
        sl = np.ascontiguousarray(slots, dtype=np.uint32)
        n = qi.shape[0]
        el, es, ex = (np.zeros(n, dtype=np.float32) for _ in range(3))
        check(lib().fg_score_edges(self._h, _fptr(q), q.shape[0], _uptr(qi), _uptr(pa), _uptr(sl),
                                   n, _fptr(el), _fptr(es), _fptr(ex)))
        return el, es, ex


class QuantizationGraph:
    """Mirror of the reference's QuantizationGraph (include/qg.hpp:14-89).

    The constructor reads the codebook file into host memory like qg.hpp:17-42
    (but rejects a truncated file); gpu_search_adaptive uploads it on first use
    and keeps it resident for later calls; the timed region is the kernel
    only, as in gpu_search_adaptive.cu:98-107."""

    def __init__(self, num_node: int, dim: int, degree: int, codebook_path: str):
        self.num_nodes = int(num_node)
        self.dim = int(dim)
        self.degree = int(degree)
        self.layout = Layout.make(self.dim, self.degree)
        try:
            self.codebook = read_codebook(codebook_path, self.num_nodes, self.dim, self.degree)
        except FileNotFoundError:
            raise RuntimeError("Cannot open codebook file: " + codebook_path)
        self._metric = METRIC_L2
        self._index: Index | None = None
        self._index_metric = None

    # accessors (qg.hpp:49-60)
    def get_entry_point(self) -> int:
        return self.codebook.entry

    def get_row_offset(self) -> int:
        return self.layout.row_offset

    def get_code_offset(self) -> int:
        return self.layout.code_offset

    def get_factor_offset(self) -> int:
        return self.layout.factor_offset

    def get_neighbor_offset(self) -> int:
        return self.layout.neighbor_offset

    def get_data_bytes(self) -> int:
        return self.num_nodes * self.layout.row_offset * 4

    def get_signs_bytes(self) -> int:
        return self.layout.padded_dim * 4

    def set_metric(self, metric: int) -> None:
        self._metric = metric

    def get_metric(self) -> int:
        return self._metric

    def index(self) -> Index:
        if self._index is None or self._index_metric != self._metric:
            if self._index is not None:
                self._index.close()
            self._index = Index.from_codebook(self.codebook, metric=self._metric)
            self._index_metric = self._metric
        return self._index

    def gpu_search_adaptive(self, nq: int, queries: np.ndarray, K: int, result_idx: np.ndarray,
                            beam_sz: int) -> float:
        q = np.ascontiguousarray(queries, dtype=np.float32).reshape(-1, self.dim)[:nq]
        ids, st, _ = self.index().search(q, K, beam_sz)
        result_idx.reshape(-1)[: nq * K] = ids.reshape(-1)
        return float(st.elapsed_s)
