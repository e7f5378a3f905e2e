"""ctypes binding of the gfx950 C-ABI library ``libmojogp_amd.so``.

The library is built in-tree by ``mojogp_amd.build`` and located through, in
order, the ``MOJOGP_AMD_LIB`` environment variable and
``mojogp_amd/lib/libmojogp_amd.so``.  There is no fallback: if the library is
missing every entry point raises ``NativeLibraryError``.
"""

from __future__ import annotations

import ctypes as C
import os
import threading
from pathlib import Path

import numpy as np

LIB_ENV = "MOJOGP_AMD_LIB"
DEFAULT_LIB = Path(__file__).resolve().parent / "lib" / "libmojogp_amd.so"

c_float_p = C.POINTER(C.c_float)
c_double_p = C.POINTER(C.c_double)
c_int64_p = C.POINTER(C.c_int64)
c_int_p = C.POINTER(C.c_int)
c_void_pp = C.POINTER(C.c_void_p)


class NativeLibraryError(RuntimeError):
    """The native gfx950 library is missing or failed to load."""


class NativeCallError(RuntimeError):
    """A native entry point returned a non-zero status."""

    def __init__(self, name: str, status: int, message: str):
        super().__init__(f"{name} failed (status {status}): {message}")
        self.status = status


# name -> (restype, argtypes).  Every entry returns an int status except the
# few informational calls.
_SIGNATURES = {
    "mgp_last_error": (C.c_int, [C.c_char_p, C.c_size_t]),
    "mgp_version": (C.c_char_p, []),
    "mgp_device_count": (C.c_int, [c_int_p]),
    "mgp_init_provider": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int64, c_float_p,
                                    c_float_p, C.c_int, C.c_float, c_void_pp]),
    "mgp_destroy_provider": (C.c_int, [C.c_void_p]),
    "mgp_update_params": (C.c_int, [C.c_void_p, c_float_p, C.c_int]),
    "mgp_update_noise": (C.c_int, [C.c_void_p, C.c_float]),
    "mgp_get_noise": (C.c_int, [C.c_void_p, c_float_p]),
    "mgp_get_diagonal_value": (C.c_int, [C.c_void_p, c_float_p]),
    "mgp_provider_info": (C.c_int, [C.c_void_p, c_int64_p, c_int_p, c_int_p, c_int_p,
                                    c_int_p]),
    "mgp_forward_matvec": (C.c_int, [C.c_void_p, c_float_p, C.c_int, c_float_p]),
    "mgp_forward_matvec_device": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int,
                                            C.c_void_p]),
    "mgp_direct_matvec": (C.c_int, [C.c_void_p, c_float_p, C.c_int, c_float_p]),
    "mgp_cross_matvec": (C.c_int, [C.c_void_p, c_float_p, C.c_int64, c_float_p,
                                   C.c_int, c_float_p]),
    "mgp_extract_diagonal": (C.c_int, [C.c_void_p, c_float_p]),
    "mgp_extract_diagonal_test": (C.c_int, [C.c_void_p, c_float_p, C.c_int64,
                                            c_float_p]),
    "mgp_benchmark_provider_ops": (C.c_int, [C.c_void_p, c_float_p, C.c_int, C.c_int,
                                             C.c_int, C.c_int, c_double_p, c_double_p,
                                             c_float_p]),
    "mgp_calibration_copy": (C.c_int, [C.c_int64, C.c_int, c_double_p]),
}

_lock = threading.Lock()
_lib: C.CDLL | None = None


def library_path() -> Path:
    env = os.environ.get(LIB_ENV)
    return Path(env) if env else DEFAULT_LIB


def exported_symbols() -> list[str]:
    """Names of every entry point this binding declares."""
    return sorted(_SIGNATURES)


def load() -> C.CDLL:
    """Load (once) and return the native library, with signatures applied."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = library_path()
        if not path.exists():
            raise NativeLibraryError(
                f"native library not found at {path}; build it with "
                "`python -m mojogp_amd.build` (hipcc, gfx950)")
        try:
            lib = C.CDLL(str(path))
        except OSError as exc:  # pragma: no cover - environment specific
            raise NativeLibraryError(f"failed to load {path}: {exc}") from exc
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def last_error() -> str:
    lib = load()
    buf = C.create_string_buffer(4096)
    lib.mgp_last_error(buf, len(buf))
    return buf.value.decode("utf-8", "replace")


def call(name: str, *args) -> None:
    """Call a status-returning entry point; raise NativeCallError on failure."""
    lib = load()
    status = getattr(lib, name)(*args)
    if status != 0:
        raise NativeCallError(name, status, last_error())


def fptr(a: np.ndarray):
    """float32 pointer of a C-contiguous float32 array."""
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(c_float_p)


def dptr(a: np.ndarray):
    assert a.dtype == np.float64 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(c_double_p)


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)
