"""ctypes binding of libflashgann.so (the C ABI in include/flashgann.h).

Loading fails loudly: there is no CPU fallback for the search path.
"""
from __future__ import annotations

import ctypes as C
import os

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "libflashgann.so")

FG_OK = 0
FG_EINVAL = -1
FG_ENOMEM = -2
FG_EDEVICE = -3
FG_EIO = -4
FG_METRIC_L2 = 0
FG_METRIC_IP = 1
FG_ENTRY_AUTO = 0xFFFFFFFF
FG_COUNTERS_PER_QUERY = 6
FG_PROFILE_SLOTS = 12
FG_NOALLOC_STAGING_BYTES = 16 << 20

EXPORTED = (
    "fg_index_create", "fg_index_load", "fg_index_destroy", "fg_index_get_info", "fg_search", "fg_search_noalloc",
    "fg_search_device", "fg_search_stream", "fg_search_profile", "fg_lds_bytes", "fg_search_waves", "fg_search_launches", "fg_search_geometry", "fg_query_prepare", "fg_score_edges", "fg_last_error",
    "fg_version",
)


class IndexInfo(C.Structure):
    _fields_ = [("dim", C.c_uint32), ("padded_dim", C.c_uint32), ("degree", C.c_uint32),
                ("entry", C.c_uint32), ("npoints", C.c_uint64), ("code_offset", C.c_uint64),
                ("factor_offset", C.c_uint64), ("neighbor_offset", C.c_uint64),
                ("row_offset", C.c_uint64), ("metric", C.c_int)]


class Stats(C.Structure):
    _fields_ = [("elapsed_s", C.c_double), ("kernel_ms", C.c_float), ("lds_bytes", C.c_uint32),
                ("visited_slots", C.c_uint32)]


class FlashGannError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"flashgann error {code}: {msg}")
        self.code = code


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                "(or make -C flashgann_amd/csrc); the search has no CPU fallback")
        L = C.CDLL(LIB_PATH)
        f32p, u32p, u8p, i32p = (C.POINTER(C.c_float), C.POINTER(C.c_uint32),
                                 C.POINTER(C.c_uint8), C.POINTER(C.c_int32))
        vp = C.c_void_p
        L.fg_index_create.argtypes = [f32p, C.c_uint64, C.c_uint32, C.c_uint32, f32p, C.c_uint32,
                                      C.c_int, C.POINTER(vp)]
        L.fg_index_load.argtypes = [C.c_char_p, C.c_uint64, C.c_uint32, C.c_uint32, C.c_int,
                                    C.POINTER(vp)]
        L.fg_index_destroy.argtypes = [vp]
        L.fg_index_destroy.restype = None
        L.fg_index_get_info.argtypes = [vp, C.POINTER(IndexInfo)]
        L.fg_search.argtypes = [vp, f32p, C.c_uint32, C.c_uint32, C.c_uint32, u32p, u32p,
                                C.POINTER(Stats)]
        L.fg_search_noalloc.argtypes = L.fg_search.argtypes
        L.fg_search_device.argtypes = [vp, vp, C.c_uint32, C.c_uint32, C.c_uint32, vp, vp, vp]
        L.fg_search_profile.argtypes = [vp, vp, C.c_uint32, C.c_uint32, C.c_uint32, vp, vp, vp]
        L.fg_search_stream.argtypes = [vp, vp, C.c_uint32, C.c_uint32, C.c_uint32, vp, C.c_uint32, C.c_uint32, vp]
        L.fg_lds_bytes.argtypes = [C.c_uint32, C.c_uint32, C.c_uint32]
        L.fg_lds_bytes.restype = C.c_uint32
        L.fg_search_waves.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32, C.c_uint32]
        L.fg_search_waves.restype = C.c_int
        L.fg_search_launches.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32, C.c_uint32]
        L.fg_search_launches.restype = C.c_int
        L.fg_search_geometry.argtypes = [C.c_void_p]
        L.fg_search_geometry.restype = C.c_int
        L.fg_query_prepare.argtypes = [vp, f32p, C.c_uint32, f32p, u8p, f32p, i32p]
        L.fg_score_edges.argtypes = [vp, f32p, C.c_uint32, u32p, u32p, u32p, C.c_uint32, f32p,
                                     f32p, f32p]
        L.fg_last_error.restype = C.c_char_p
        L.fg_version.restype = C.c_char_p
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != FG_OK:
        raise FlashGannError(rc, lib().fg_last_error().decode())
