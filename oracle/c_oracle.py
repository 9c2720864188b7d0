"""ctypes wrapper of liboracle_shortlist.so (test infrastructure only)."""
from __future__ import annotations

import ctypes
from typing import Optional

import numpy as np

from .build_oracle import LIB, build

_lib = None


def load():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        _lib = ctypes.CDLL(str(LIB))
        _lib.oracle_shortlist_build.restype = ctypes.c_int
    return _lib


def shortlist_build(rows: np.ndarray, row_batch: Optional[np.ndarray], T: int, L: int, local_w: int, stride: int,
                    slots: int, scores: Optional[np.ndarray], K: int):
    """rows int32 (N,), row_batch int32 (N,) or None, scores f32 (B, Ts) or
    None.  Returns (cand int32 (N, L), lengths int32 (N,))."""
    lib = load()
    rows = np.ascontiguousarray(rows, dtype=np.int32)
    N = rows.size
    cand = np.empty((N, L), dtype=np.int32)
    lens = np.empty((N,), dtype=np.int32)
    rb = None if row_batch is None else np.ascontiguousarray(row_batch, dtype=np.int32)
    if scores is not None:
        sc = np.ascontiguousarray(scores, dtype=np.float32)
        if sc.ndim == 1:
            sc = sc[None, :]
        B, Ts = sc.shape
        sp = sc.ctypes.data_as(ctypes.c_void_p)
    else:
        B, Ts, sp, K = 1, 0, None, 0
    rc = lib.oracle_shortlist_build(
        rows.ctypes.data_as(ctypes.c_void_p), None if rb is None else rb.ctypes.data_as(ctypes.c_void_p),
        ctypes.c_int64(N), ctypes.c_int64(T), ctypes.c_int(L), ctypes.c_int(local_w), ctypes.c_int(stride),
        ctypes.c_int(slots), sp, ctypes.c_int(B), ctypes.c_int64(Ts), ctypes.c_int(K),
        cand.ctypes.data_as(ctypes.c_void_p), lens.ctypes.data_as(ctypes.c_void_p))
    if rc != 0:
        raise RuntimeError("oracle_shortlist_build failed")
    return cand, lens
