"""Neighbor-list oracle (TEST INFRASTRUCTURE ONLY): ctypes wrapper of nlist_oracle.c.

Restates molix::get_neighbor_pairs (reference
src/molix/op/src/neighbors/get_neighbor_pairs.cpp:28-77) bit for bit.
Pinned by: tests/golden/nlist_golden.npz (outputs of the reference op itself,
compiled from its sources), and the brute-force / cell-list variants agreeing.
"""

from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "_ref", "liboracle.so")
_lib = None


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            subprocess.run(["make", "-C", HERE, "oracle"], check=True, capture_output=True)
        lib = C.CDLL(LIB)
        for name in ("half", "cells"):
            for t in ("float", "double"):
                fn = getattr(lib, f"oracle_nlist_{name}_{t}")
                fn.restype = C.c_int64
                fn.argtypes = [C.c_void_p, C.c_int64, C.c_double, C.c_void_p, C.c_int64] + [C.c_void_p] * 4
        _lib = lib
    return _lib


def half_pairs(pos: np.ndarray, cutoff: float, box: np.ndarray | None, cells: bool = False):
    """All half pairs (row > col) in the reference's (row, col) order.

    Returns (rows int32, cols int32, deltas, distances) in pos's dtype.
    """
    lib = load()
    dt = pos.dtype
    assert dt in (np.float32, np.float64)
    p = np.ascontiguousarray(pos)
    b = None if box is None or box.size == 0 else np.ascontiguousarray(box, dtype=dt)
    tname = "float" if dt == np.float32 else "double"
    fn = getattr(lib, f"oracle_nlist_{'cells' if cells else 'half'}_{tname}")
    n = p.shape[0]
    bp = None if b is None else b.ctypes.data
    cnt = fn(p.ctypes.data, n, cutoff, bp, 0, None, None, None, None)
    rows = np.empty(cnt, np.int32)
    cols = np.empty(cnt, np.int32)
    d = np.empty((cnt, 3), dt)
    dist = np.empty(cnt, dt)
    fn(p.ctypes.data, n, cutoff, bp, cnt, rows.ctypes.data, cols.ctypes.data, d.ctypes.data, dist.ctypes.data)
    return rows, cols, d, dist


def get_neighbor_pairs(pos: np.ndarray, cutoff: float, max_num_pairs: int, box: np.ndarray | None):
    """The reference op's outputs (neighbors (2, W), deltas, distances, num_pairs).

    Width semantics of the reference CPU path (.cpp:55-73): -1 -> N(N-1)/2 slots
    at the triangular index; M -> the found pairs padded to M (all found pairs
    when there are more than M).
    """
    rows, cols, d, dist = half_pairs(pos, cutoff, box)
    n = pos.shape[0]
    found = rows.shape[0]
    if max_num_pairs == -1:
        width = n * (n - 1) // 2
        slot = rows.astype(np.int64) * (rows.astype(np.int64) - 1) // 2 + cols
    else:
        width = max(max_num_pairs, found)
        slot = np.arange(found)
    nb = np.full((2, width), -1, np.int32)
    dd = np.full((width, 3), np.nan, pos.dtype)
    ds = np.full(width, np.nan, pos.dtype)
    nb[0, slot], nb[1, slot], dd[slot], ds[slot] = rows, cols, d, dist
    return nb, dd, ds, np.array([found], np.int32)


def directed_pairs(pos: np.ndarray, cutoff: float, box: np.ndarray | None, cells: bool = True):
    """All ordered pairs (i, j), i != j, sorted by (i, j), with the reference geometry:
    deltas[i, j] = the half-list delta of (max, min), negated when i < j.
    """
    rows, cols, d, dist = half_pairs(pos, cutoff, box, cells=cells)
    i = np.concatenate([rows, cols])
    j = np.concatenate([cols, rows])
    dd = np.concatenate([d, -d])
    ds = np.concatenate([dist, dist])
    order = np.lexsort((j, i))
    return i[order], j[order], dd[order], ds[order]
