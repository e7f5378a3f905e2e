"""ctypes access to oracle/lib/liboracle_ref.so (test/baseline infrastructure)."""

from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "lib" / "liboracle_ref.so"
_lib = None


def load():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            from .build import build
            build()
        lib = C.CDLL(str(LIB_PATH))
        fp = C.POINTER(C.c_float)
        lib.ref_forward_matvec_rows.restype = C.c_int
        lib.ref_forward_matvec_rows.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int64, fp, fp,
                                                C.c_float, fp, C.c_int, C.c_int64, C.c_int64, fp]
        lib.ref_num_threads.restype = C.c_int
        _lib = lib
    return _lib


def _fp(a):
    return a.ctypes.data_as(C.POINTER(C.c_float))


def forward_matvec_rows(kind: int, ard: bool, X, params, noise: float, V, row0: int,
                        nrows: int) -> np.ndarray:
    """fp32 reference-order (K + noise I) V restricted to rows [row0, row0+nrows)."""
    lib = load()
    X = np.ascontiguousarray(X, dtype=np.float32)
    V = np.ascontiguousarray(np.atleast_2d(V), dtype=np.float32)
    params = np.ascontiguousarray(params, dtype=np.float32)
    n, d = X.shape
    out = np.empty((V.shape[0], nrows), dtype=np.float32)
    rc = lib.ref_forward_matvec_rows(int(kind), int(ard), d, n, _fp(X), _fp(params),
                                     float(noise), _fp(V), V.shape[0], int(row0),
                                     int(nrows), _fp(out))
    if rc != 0:
        raise ValueError("ref_forward_matvec_rows rejected its arguments")
    return out


def num_threads() -> int:
    return int(load().ref_num_threads())
