"""Codebook layout, file format and fvecs/ivecs I/O.

The codebook is the reference's SymphonyQG-style file (include/qg.hpp:17-42,
66-73):

    uint32 entry_point                       (0xFFFFFFFF = compute at load)
    N rows of row_offset float32 each:
        [vector: dim][codes: deg * B/8 bytes][triple_x: deg][factor_dq: deg]
        [factor_vq: deg][neighbour ids: deg uint32]
    B float32 signs (the +-1 diagonal applied before the FWHT)

with B = padded_dim = next power of two >= dim.  Within the code region the
edges of a node are contiguous; each edge holds B/8 bytes, and 4-dim chunk cb
sits in the low nibble of byte cb>>1 (even cb) or its high nibble (odd cb),
dim 4cb+0 in bit 3 of the nibble ... dim 4cb+3 in bit 0
(include/utils.cuh:823-838, 909-917).
"""
from __future__ import annotations

import os
from dataclasses import dataclass

import numpy as np

MAX_INDEX = 0xFFFFFFFF


def padded_dim_for(dim: int) -> int:
    """Power-of-two round-up (qg.hpp:67 computes 1 << ceil(log2(dim)))."""
    b = 1
    while b < dim:
        b <<= 1
    return b


@dataclass(frozen=True)
class Layout:
    """Row layout in float units (qg.hpp:66-73)."""

    dim: int
    degree: int
    padded_dim: int
    code_offset: int
    factor_offset: int
    neighbor_offset: int
    row_offset: int

    @staticmethod
    def make(dim: int, degree: int) -> "Layout":
        b = padded_dim_for(dim)
        code = dim
        factor = code + (b // 64) * 2 * degree
        nbr = factor + 3 * degree
        row = nbr + degree
        return Layout(dim, degree, b, code, factor, nbr, row)

    @property
    def code_bytes_per_edge(self) -> int:
        return self.padded_dim // 8

    @property
    def row_bytes(self) -> int:
        return self.row_offset * 4


@dataclass
class Codebook:
    """An in-memory codebook: rows (N x row_offset float32), signs, entry."""

    rows: np.ndarray
    signs: np.ndarray
    entry: int
    layout: Layout

    @property
    def npoints(self) -> int:
        return int(self.rows.shape[0])

    def vectors(self) -> np.ndarray:
        return self.rows[:, : self.layout.dim]

    def neighbors(self) -> np.ndarray:
        lay = self.layout
        return self.rows[:, lay.neighbor_offset : lay.row_offset].view(np.uint32)

    def factors(self) -> np.ndarray:
        lay = self.layout
        return self.rows[:, lay.factor_offset : lay.neighbor_offset].reshape(
            self.npoints, 3, lay.degree
        )

    def codes(self) -> np.ndarray:
        lay = self.layout
        raw = self.rows[:, lay.code_offset : lay.factor_offset].view(np.uint8)
        return raw.reshape(self.npoints, lay.degree, lay.code_bytes_per_edge)

    def save(self, path: str) -> None:
        write_codebook(path, self.rows, self.signs, self.entry)


def write_codebook(path: str, rows: np.ndarray, signs: np.ndarray, entry: int) -> None:
    rows = np.ascontiguousarray(rows, dtype=np.float32)
    signs = np.ascontiguousarray(signs, dtype=np.float32)
    with open(path, "wb") as f:
        np.array([entry], dtype=np.uint32).tofile(f)
        rows.tofile(f)
        signs.tofile(f)


def read_codebook(path: str, npoints: int, dim: int, degree: int) -> Codebook:
    """Reads a codebook; unlike qg.hpp:33-36 a short file is an error."""
    lay = Layout.make(dim, degree)
    need = 4 + npoints * lay.row_offset * 4 + lay.padded_dim * 4
    size = os.path.getsize(path)
    if size < need:
        raise ValueError(f"codebook {path} is truncated: {size} bytes, expected {need}")
    with open(path, "rb") as f:
        entry = int(np.fromfile(f, dtype=np.uint32, count=1)[0])
        rows = np.fromfile(f, dtype=np.float32, count=npoints * lay.row_offset)
        signs = np.fromfile(f, dtype=np.float32, count=lay.padded_dim)
    return Codebook(rows.reshape(npoints, lay.row_offset), signs, entry, lay)


def write_fvecs(path: str, x: np.ndarray) -> None:
    x = np.ascontiguousarray(x, dtype=np.float32)
    n, d = x.shape
    out = np.empty((n, d + 1), dtype=np.float32)
    out[:, 0] = np.array([d], dtype=np.int32).view(np.float32)[0]
    out[:, 1:] = x
    out.tofile(path)


def write_ivecs(path: str, x: np.ndarray) -> None:
    x = np.ascontiguousarray(x, dtype=np.int32)
    n, d = x.shape
    out = np.empty((n, d + 1), dtype=np.int32)
    out[:, 0] = d
    out[:, 1:] = x
    out.tofile(path)


def _read_vecs(path: str, dtype) -> np.ndarray:
    """data_io.hpp:18-77: count = file_size / (4 + 4*dim); every row's leading
    int must equal the first one."""
    raw = np.fromfile(path, dtype=np.int32)
    if raw.size == 0:
        return np.zeros((0, 0), dtype=dtype)
    d = int(raw[0])
    n = raw.size // (d + 1)
    raw = raw[: n * (d + 1)].reshape(n, d + 1)
    if not np.all(raw[:, 0] == d):
        raise ValueError(f"{path}: inconsistent row dimensions")
    return raw[:, 1:].copy().view(dtype)


def read_fvecs(path: str) -> np.ndarray:
    return _read_vecs(path, np.float32)


def read_ivecs(path: str) -> np.ndarray:
    return _read_vecs(path, np.int32)


def code_bit_positions(padded_dim: int) -> np.ndarray:
    """Bit index (within one edge's B/8-byte code) holding dim i:
    4*(i >> 2) + 3 - (i & 3)."""
    i = np.arange(padded_dim)
    return 4 * (i >> 2) + 3 - (i & 3)


def pack_codes(bits: np.ndarray) -> np.ndarray:
    """bits: (..., B) {0,1} in dim order -> (..., B/8) uint8 in code order."""
    b = bits.shape[-1]
    ordered = np.zeros(bits.shape, dtype=np.uint8)
    ordered[..., code_bit_positions(b)] = bits
    return np.packbits(ordered, axis=-1, bitorder="little")


def unpack_codes(codes: np.ndarray) -> np.ndarray:
    """Inverse of pack_codes: (..., B/8) uint8 -> (..., B) bits in dim order."""
    ordered = np.unpackbits(codes, axis=-1, bitorder="little")
    return ordered[..., code_bit_positions(ordered.shape[-1])]
