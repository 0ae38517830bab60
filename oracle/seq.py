"""numpy/ctypes front end of the sequential C oracle (``oracle/bevpool_seq.c``).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).  The shared object is
built by ``oracle/Makefile`` (``make -C oracle``) into
``oracle/_build/liboracle_seq.so``; ``__graft_entry__.build()`` runs it.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

_LIB_PATH = Path(__file__).resolve().parent / '_build' / 'liboracle_seq.so'
_lib = None

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags='C_CONTIGUOUS')
_i64p = np.ctypeslib.ndpointer(dtype=np.int64, flags='C_CONTIGUOUS')
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags='C_CONTIGUOUS')
_u32p = np.ctypeslib.ndpointer(dtype=np.uint32, flags='C_CONTIGUOUS')
_i64 = ctypes.c_int64


def lib():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            raise FileNotFoundError(f'{_LIB_PATH} missing: run `make -C oracle`')
        L = ctypes.CDLL(str(_LIB_PATH))
        L.oracle_quantize_geom.argtypes = [_f32p, _i64, _i64, _f32p, _f32p, _i64p, _i64p]
        L.oracle_quantize_geom.restype = None
        L.oracle_coord_ranks.argtypes = [_i64p, _i64, _i64, _i64, _i64, _i64, _i64p]
        L.oracle_coord_ranks.restype = _i64
        L.oracle_stable_sort.argtypes = [_i64p, _i64, _i64, _i64p, _i64p]
        L.oracle_stable_sort.restype = _i64
        L.oracle_intervals.argtypes = [_i64p, _i64, _i32p, _i32p]
        L.oracle_intervals.restype = _i64
        L.oracle_forward.argtypes = [_f32p, _i64, _i64, _i64p, _i64, _i64, _f32p]
        L.oracle_forward.restype = None
        L.oracle_backward.argtypes = [_u32p, _i64, _i64p, _i64, _u32p]
        L.oracle_backward.restype = None
        _lib = L
    return _lib


def quantize_geom(geom: np.ndarray, points_per_batch: int, offset, dx, nx) -> np.ndarray:
    """rank per point (-1 dropped); geom is (N_all, 3) fp32 in point order."""
    g = np.ascontiguousarray(geom, dtype=np.float32).reshape(-1, 3)
    rank = np.empty(g.shape[0], dtype=np.int64)
    lib().oracle_quantize_geom(
        g,
        g.shape[0],
        int(points_per_batch),
        np.asarray(offset, dtype=np.float32),
        np.asarray(dx, dtype=np.float32),
        np.asarray(nx, dtype=np.int64),
        rank,
    )
    return rank


def coord_ranks(coords: np.ndarray, B, D, H, W):
    c = np.ascontiguousarray(coords, dtype=np.int64).reshape(-1, 4)
    rank = np.empty(c.shape[0], dtype=np.int64)
    bad = lib().oracle_coord_ranks(c, c.shape[0], int(B), int(D), int(H), int(W), rank)
    return rank, int(bad)


def stable_sort(rank: np.ndarray, n_cells: int):
    r = np.ascontiguousarray(rank, dtype=np.int64)
    perm = np.empty(r.shape[0], dtype=np.int64)
    srt = np.empty(r.shape[0], dtype=np.int64)
    k = lib().oracle_stable_sort(r, r.shape[0], int(n_cells), perm, srt)
    if k < 0:
        raise MemoryError('oracle_stable_sort allocation failed')
    return perm[:k].copy(), srt[:k].copy()


def intervals(sorted_rank: np.ndarray):
    s = np.ascontiguousarray(sorted_rank, dtype=np.int64)
    starts = np.empty(max(1, s.shape[0]), dtype=np.int32)
    lengths = np.empty(max(1, s.shape[0]), dtype=np.int32)
    m = lib().oracle_intervals(s, s.shape[0], starts, lengths)
    return starts[:m].copy(), lengths[:m].copy()


def forward_rows(x: np.ndarray, rank: np.ndarray, n_cells: int) -> np.ndarray:
    """Cell-major sums (n_cells, C), point order, fp32 from +0.0."""
    xx = np.ascontiguousarray(x, dtype=np.float32)
    n, C = xx.shape
    out = np.empty((n_cells, C), dtype=np.float32)
    lib().oracle_forward(xx, C, C, np.ascontiguousarray(rank, dtype=np.int64), n, n_cells, out)
    return out


def backward_rows(grad_rows_bits: np.ndarray, rank: np.ndarray) -> np.ndarray:
    """x_grad bits (N, C) uint32 from cell-major grad rows (n_cells, C) uint32."""
    g = np.ascontiguousarray(grad_rows_bits, dtype=np.uint32)
    C = g.shape[1]
    r = np.ascontiguousarray(rank, dtype=np.int64)
    out = np.empty((r.shape[0], C), dtype=np.uint32)
    lib().oracle_backward(g, C, r, r.shape[0], out)
    return out
