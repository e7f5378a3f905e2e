"""The C-ABI library loads and exports every symbol include/mojogp_amd.h declares
(no compute calls: this runs on machines without a GPU)."""

import ctypes
import re
from pathlib import Path

import pytest

from mojogp_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "mojogp_amd.h"


def _declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"MGP_API\s+[\w\s\*]+?\b(mgp_\w+)\s*\(", text)))


def test_header_declares_entry_points():
    names = _declared()
    assert "mgp_init_provider" in names and "mgp_forward_matvec" in names
    assert len(names) >= 15


def test_library_exports_every_declared_symbol():
    if not _lib.library_path().exists():
        pytest.fail(f"native library missing at {_lib.library_path()}; run __graft_entry__.build()")
    lib = ctypes.CDLL(str(_lib.library_path()))
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"


def test_binding_covers_header():
    assert set(_declared()) == set(_lib.exported_symbols())


def test_error_path_reports_message():
    # Argument validation happens before any device work, so this is safe
    # without a GPU.
    import numpy as np
    X = np.zeros((4, 2), dtype=np.float32)
    params = np.ones(5, dtype=np.float32)  # wrong count for ARD d=2
    with pytest.raises(_lib.NativeCallError, match="expected 3"):
        _lib.call("mgp_init_provider", 0, 1, 2, 4, _lib.fptr(X), _lib.fptr(params), 5,
                  0.1, ctypes.byref(ctypes.c_void_p()))


def test_fn_pointer_exports_report_on_dead_handles():
    """The reference-signature fn pointers (the provider dict's update_noise,
    get_noise, get_noise_mode, get_noise_vector_ptr, get_diagonal_value) take
    the provider_ptr value and return no status: on a handle that is no live
    provider they record the error and return their sentinels, before any
    device work (safe without a GPU)."""
    import math
    upd = ctypes.CFUNCTYPE(None, ctypes.c_ssize_t, ctypes.c_float)(
        _lib.fn_address("mgp_fn_update_noise"))
    upd(0, 0.5)
    assert "null provider handle" in _lib.last_error()
    get_f = ctypes.CFUNCTYPE(ctypes.c_float, ctypes.c_ssize_t)
    get_i = ctypes.CFUNCTYPE(ctypes.c_ssize_t, ctypes.c_ssize_t)
    get_p = ctypes.CFUNCTYPE(ctypes.c_void_p, ctypes.c_ssize_t)
    bogus = 0x1000
    assert math.isnan(get_f(_lib.fn_address("mgp_fn_get_noise"))(bogus))
    assert "unknown or destroyed provider handle" in _lib.last_error()
    assert math.isnan(get_f(_lib.fn_address("mgp_fn_get_diagonal_value"))(bogus))
    assert get_i(_lib.fn_address("mgp_fn_get_noise_mode"))(bogus) == -1
    assert get_p(_lib.fn_address("mgp_fn_get_noise_vector_ptr"))(bogus) is None
