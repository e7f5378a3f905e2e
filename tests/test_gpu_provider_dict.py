"""The provider dict's fn-pointer entries, called through ctypes exactly as the
reference's Python calls them: update_noise as
CFUNCTYPE(None, c_ssize_t, c_float)(info["update_noise"])(info["provider_ptr"],
noise) (mojogp/_multi_output_backend.py:166-183), and the other non-raising
provider pointers with their signatures (erased_provider.mojo:43-50,
fn_ptr_module.py:666-696)."""

import ctypes as C

import numpy as np
import pytest

from mojogp_amd import _engine, _lib
from oracle import kernels as ok

pytestmark = pytest.mark.gpu

_UPDATE = C.CFUNCTYPE(None, C.c_ssize_t, C.c_float)
_GET_F = C.CFUNCTYPE(C.c_float, C.c_ssize_t)
_GET_I = C.CFUNCTYPE(C.c_ssize_t, C.c_ssize_t)
_GET_P = C.CFUNCTYPE(C.c_void_p, C.c_ssize_t)


def _rel(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / np.linalg.norm(b))


def test_update_noise_fn_pointer_as_the_reference_calls_it():
    rng = np.random.default_rng(21)
    n, d, t = 1500, 3, 4
    X = rng.uniform(-2, 2, size=(n, d)).astype(np.float32)
    V = rng.normal(size=(t, n)).astype(np.float32)
    params = np.array([0.8, 1.1, 0.9, 1.4], np.float32)
    km = _engine.load_kernel_module("rbf", True, d)
    info = km.init_provider(X, params, 0.1)
    ptr = info["provider_ptr"]
    print(f"provider dict fn pointers: provider_ptr {ptr:#x}", flush=True)
    try:
        _UPDATE(info["update_noise"])(ptr, 0.37)
        assert _GET_F(info["get_noise"])(ptr) == np.float32(0.37)
        assert _GET_I(info["get_noise_mode"])(ptr) == 0
        assert _GET_P(info["get_noise_vector_ptr"])(ptr) is None
        assert _GET_F(info["get_diagonal_value"])(ptr) == np.float32(1.4)
        # the product sees the noise set through the pointer
        got = info["_provider"].forward_matvec(V)
        ref = ok.forward_matvec(ok.RBF, X, V, params, 0.37, True)
        print(f"  product after update_noise(0.37): relerr {_rel(got, ref):.2e}", flush=True)
        assert _rel(got, ref) <= 1e-5
        # an invalid noise is refused (recorded, noise unchanged): no status
        # can cross this signature
        _UPDATE(info["update_noise"])(ptr, -1.0)
        assert "noise must be finite" in _lib.last_error()
        assert _GET_F(info["get_noise"])(ptr) == np.float32(0.37)
    finally:
        km.destroy_provider(info)
    # a destroyed provider: the pointers report and return their sentinels
    _UPDATE(info["update_noise"])(ptr, 0.2)
    assert "unknown or destroyed provider handle" in _lib.last_error()
    assert np.isnan(_GET_F(info["get_noise"])(ptr))
    assert _GET_I(info["get_noise_mode"])(ptr) == -1


def test_noise_vector_mode_fn_pointers():
    """Noise mode 1 (fixed per-point vector): get_noise reports the reference's
    1e-6 floor, get_noise_mode 1, get_noise_vector_ptr the device array."""
    rng = np.random.default_rng(22)
    n, d = 800, 2
    X = rng.uniform(-1, 1, size=(n, d)).astype(np.float32)
    nv = rng.uniform(0.05, 0.2, size=n).astype(np.float32)
    km = _engine.load_kernel_module("matern52", False, d)
    info = km.init_provider(X, np.array([0.7, 1.2], np.float32), 0.1, observation_noise=nv)
    ptr = info["provider_ptr"]
    try:
        assert info["noise_mode"] == 1
        assert _GET_I(info["get_noise_mode"])(ptr) == 1
        assert _GET_F(info["get_noise"])(ptr) == np.float32(1e-6)
        assert _GET_P(info["get_noise_vector_ptr"])(ptr) is not None
    finally:
        km.destroy_provider(info)
