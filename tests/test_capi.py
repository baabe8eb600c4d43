"""The C-ABI library loads and exports every symbol include/flashgann.h
declares; argument checks fail before any device call."""
from __future__ import annotations

import ctypes as C
import os
import re

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "flashgann.h")).read()
    return sorted(set(re.findall(r"^\w[\w\s\*]*?\b(fg_\w+)\s*\(", text, re.M)))


def test_header_symbols_exported():
    from flashgann_amd import _lib
    L = C.CDLL(_lib.LIB_PATH)
    syms = declared_symbols()
    assert len(syms) >= 10, syms
    for s in syms:
        assert hasattr(L, s), f"{s} declared in include/flashgann.h but not exported"
    assert set(syms) == set(_lib.EXPORTED)


def test_shape_checks_before_device_use():
    from flashgann_amd import _lib
    L = _lib.lib()
    rows = np.zeros((4, 400), dtype=np.float32)
    signs = np.ones(32, dtype=np.float32)
    h = C.c_void_p()
    rc = L.fg_index_create(rows.ctypes.data_as(C.POINTER(C.c_float)), 4, 16, 4,
                           signs.ctypes.data_as(C.POINTER(C.c_float)), 0, 0, C.byref(h))
    assert rc == _lib.FG_EINVAL
    assert b"dim" in L.fg_last_error()
    rc = L.fg_index_create(rows.ctypes.data_as(C.POINTER(C.c_float)), 4, 128, 1025,
                           signs.ctypes.data_as(C.POINTER(C.c_float)), 0, 0, C.byref(h))
    assert rc == _lib.FG_EINVAL and b"degree" in L.fg_last_error()


def test_lds_bytes_host_only():
    from flashgann_amd import lds_bytes
    small = lds_bytes(128, 128, 32)
    big = lds_bytes(128, 1024, 32)
    assert 4096 < small < big < 64 * 1024


def test_header_constants_match_binding():
    from flashgann_amd import _lib
    text = open(os.path.join(ROOT, "include", "flashgann.h")).read()
    defs = {k: int(v.rstrip("u"), 0) for k, v in re.findall(r"^#define (FG_\w+)\s+(-?\w+)", text, re.M)}
    for name in ("FG_OK", "FG_EINVAL", "FG_ENOMEM", "FG_EDEVICE", "FG_EIO", "FG_METRIC_L2", "FG_METRIC_IP",
                 "FG_ENTRY_AUTO", "FG_COUNTERS_PER_QUERY", "FG_PROFILE_SLOTS"):
        assert defs[name] == getattr(_lib, name), name


def test_search_stream_rejects_null_index():
    from flashgann_amd import _lib
    L = _lib.lib()
    rc = L.fg_search_stream(None, None, 0, 10, 64, None, 16, 2, None)
    assert rc == _lib.FG_EINVAL and b"NULL" in L.fg_last_error()


def test_index_query_shape_checks():
    """Host queries must be (nq, dim); one 1-D query becomes (1, dim).  The
    check runs before any library call (a wrong shape would otherwise make
    fg_search read past the host buffer)."""
    import pytest
    from flashgann_amd import Index
    from flashgann_amd._lib import IndexInfo
    ix = Index.__new__(Index)
    ix._h = None
    ix.info = IndexInfo(dim=128)
    assert ix._host_queries(np.zeros(128, np.float32)).shape == (1, 128)
    assert ix._host_queries(np.zeros((3, 128), np.float64)).dtype == np.float32
    for bad in (np.zeros(96, np.float32), np.zeros((3, 64), np.float32), np.zeros((2, 3, 128), np.float32)):
        with pytest.raises(ValueError):
            ix._host_queries(bad)
