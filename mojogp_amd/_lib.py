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


class TrainOpts(C.Structure):
    """mgp_train_opts_t"""
    _fields_ = [
        ("max_iterations", C.c_int), ("learning_rate", C.c_float), ("num_probes", C.c_int),
        ("max_cg_iter", C.c_int), ("cg_tol", C.c_float), ("precond_rank", C.c_int),
        ("verbose", C.c_int), ("use_cosine_lr", C.c_int), ("use_preconditioner", C.c_int),
        ("max_tridiag_iter", C.c_int), ("precond_rebuild_threshold", C.c_float),
        ("precond_method", C.c_int), ("init_mean", C.c_float),
        ("enable_early_stopping", C.c_int), ("early_stop_patience", C.c_int),
        ("early_stop_tol", C.c_float), ("learn_noise", C.c_int), ("noise_floor", C.c_float),
        ("noise_regularization", C.c_float), ("progress_interval", C.c_int),
        ("nan_inject_mask", C.c_ulonglong),
    ]


class Progress(C.Structure):
    """mgp_progress_t"""
    _fields_ = [
        ("phase", C.c_char_p), ("current", C.c_int), ("total", C.c_int), ("nll", C.c_double),
        ("best_nll", C.c_double), ("cg_iter", C.c_int), ("iter_ms", C.c_double),
        ("noise", C.c_double), ("mean", C.c_double), ("precond_rank", C.c_int),
        ("precond_rebuild_count", C.c_int), ("converged", C.c_int),
    ]


PROGRESS_CB = C.CFUNCTYPE(None, C.POINTER(Progress), C.c_void_p)


class TrainResult(C.Structure):
    """mgp_train_result_t"""
    _fields_ = [
        ("params", c_float_p), ("nll_history", c_float_p), ("iter_times_ms", c_double_p),
        ("cg_iterations_history", c_int_p), ("precond_rank_history", c_int_p),
        ("precond_rebuild_steps", c_int_p), ("cached_alpha", c_float_p),
        ("final_nll", C.c_float), ("noise", C.c_float), ("mean", C.c_float),
        ("iterations", C.c_int), ("converged", C.c_int), ("history_len", C.c_int),
        ("cg_history_len", C.c_int), ("rank_history_len", C.c_int),
        ("rebuild_steps_len", C.c_int), ("precond_build_count", C.c_int),
        ("precond_build_total_ms", C.c_double), ("has_alpha", C.c_int),
        ("learned_noise", c_float_p), ("noise_fn_params", c_float_p),
        ("has_learned_noise", C.c_int), ("noise_fn_len", C.c_int),
    ]


class PredictOpts(C.Structure):
    """mgp_predict_opts_t"""
    _fields_ = [
        ("mean", C.c_float), ("variance_method", C.c_int), ("max_cg_iter", C.c_int),
        ("cg_tol", C.c_float), ("precond_rank", C.c_int), ("lanczos_rank", C.c_int),
        ("exact_block_cols", C.c_int),
    ]


class PredictInfo(C.Structure):
    """mgp_predict_info_t"""
    _fields_ = [
        ("alpha_time_s", C.c_double), ("mean_time_s", C.c_double),
        ("variance_time_s", C.c_double), ("total_time_s", C.c_double),
        ("love_root_time_s", C.c_double), ("alpha_cache_used", C.c_int),
        ("love_root_cache_used", C.c_int), ("alpha_cg_iterations", C.c_int),
        ("exact_block_cols", C.c_int), ("exact_cg_block_count", C.c_int),
        ("exact_cg_total_iterations", C.c_int), ("exact_cg_max_iterations", C.c_int),
        ("exact_precond_rank", C.c_int),
    ]


class LMCTrainOpts(C.Structure):
    """mgp_lmc_train_opts_t"""
    _fields_ = [
        ("max_iterations", C.c_int), ("learning_rate", C.c_float), ("num_probes", C.c_int),
        ("max_cg_iter", C.c_int), ("cg_tol", C.c_float), ("precond_rank", C.c_int),
        ("precond_method", C.c_int), ("precond_rebuild_threshold", C.c_float),
        ("max_tridiag_iter", C.c_int), ("early_stop_tol", C.c_float),
        ("early_stop_patience", C.c_int),
    ]


class LMCTrainResult(C.Structure):
    """mgp_lmc_train_result_t"""
    _fields_ = [
        ("params", c_float_p), ("A", c_float_p), ("L", c_float_p), ("var_diag", c_float_p),
        ("noise", c_float_p), ("mean", c_float_p), ("alpha", c_float_p),
        ("nll_history", c_float_p), ("iter_times_ms", c_double_p), ("history_len", C.c_int),
        ("final_nll", C.c_float), ("iterations", C.c_int), ("converged", C.c_int),
        ("precond_rebuild_count", C.c_int),
    ]


class ICMTrainOpts(C.Structure):
    """mgp_icm_train_opts_t"""
    _fields_ = [
        ("max_iterations", C.c_int), ("learning_rate", C.c_float), ("task_rank", C.c_int),
        ("num_probes", C.c_int), ("max_cg_iter", C.c_int), ("cg_tol", C.c_float),
        ("precond_rank", C.c_int), ("precond_method", C.c_int),
        ("precond_rebuild_threshold", C.c_float), ("max_tridiag_iter", C.c_int),
        ("early_stop_patience", C.c_int), ("early_stop_tol", C.c_float),
        ("use_cosine_lr", C.c_int), ("progress_interval", C.c_int),
    ]


class ICMTrainResult(C.Structure):
    """mgp_icm_train_result_t"""
    _fields_ = [
        ("params", c_float_p), ("noise", c_float_p), ("mean", c_float_p), ("B", c_float_p),
        ("alpha", c_float_p), ("nll_history", c_float_p), ("cg_iterations_history", c_int_p),
        ("iter_times_ms", c_double_p), ("history_len", C.c_int), ("outputscale", C.c_float),
        ("final_nll", C.c_float), ("iterations", C.c_int), ("converged", C.c_int),
        ("task_rank", C.c_int), ("precond_rebuild_count", C.c_int),
    ]


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
    "mgp_init_provider_tree": (C.c_int, [C.POINTER(C.c_int), C.c_int, C.c_int, C.c_int64,
                                         c_float_p, c_float_p, C.c_int, C.c_float, c_void_pp]),
    "mgp_destroy_provider": (C.c_int, [C.c_void_p]),
    "mgp_set_categorical_tables": (C.c_int, [C.c_void_p, c_float_p, C.c_int]),
    "mgp_set_categorical_params": (C.c_int, [C.c_void_p, C.POINTER(C.c_int), C.c_int,
                                             c_float_p, C.c_int]),
    "mgp_set_learned_noise": (C.c_int, [C.c_void_p, C.c_int, C.POINTER(C.c_int), C.c_int]),
    "mgp_materialize": (C.c_int, [C.c_void_p]),
    "mgp_update_params": (C.c_int, [C.c_void_p, c_float_p, C.c_int]),
    "mgp_update_noise": (C.c_int, [C.c_void_p, C.c_float]),
    "mgp_set_noise_vector": (C.c_int, [C.c_void_p, c_float_p]),
    "mgp_get_noise": (C.c_int, [C.c_void_p, c_float_p]),
    "mgp_get_diagonal_value": (C.c_int, [C.c_void_p, c_float_p]),
    "mgp_provider_info": (C.c_int, [C.c_void_p, c_int64_p, c_int_p, c_int_p, c_int_p,
                                    c_int_p]),
    "mgp_forward_matvec": (C.c_int, [C.c_void_p, c_float_p, C.c_int, c_float_p]),
    "mgp_forward_matvec_device": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int,
                                            C.c_void_p]),
    "mgp_forward_matvec_device_noalloc": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int,
                                                    C.c_void_p]),
    "mgp_direct_matvec": (C.c_int, [C.c_void_p, c_float_p, C.c_int, c_float_p]),
    "mgp_cross_matvec": (C.c_int, [C.c_void_p, c_float_p, C.c_int64, c_float_p,
                                   C.c_int, c_float_p]),
    "mgp_extract_diagonal": (C.c_int, [C.c_void_p, c_float_p]),
    "mgp_extract_diagonal_test": (C.c_int, [C.c_void_p, c_float_p, C.c_int64,
                                            c_float_p]),
    "mgp_gradient_matvec": (C.c_int, [C.c_void_p, c_float_p, C.c_int, c_float_p]),
    "mgp_gradient_trace": (C.c_int, [C.c_void_p, c_float_p, c_float_p, C.c_int, c_double_p]),
    # fn-pointer exports with the reference's provider signatures (no status)
    "mgp_fn_update_noise": (None, [C.c_ssize_t, C.c_float]),
    "mgp_fn_get_noise": (C.c_float, [C.c_ssize_t]),
    "mgp_fn_get_noise_mode": (C.c_ssize_t, [C.c_ssize_t]),
    "mgp_fn_get_noise_vector_ptr": (C.c_void_p, [C.c_ssize_t]),
    "mgp_fn_get_diagonal_value": (C.c_float, [C.c_ssize_t]),
    "mgp_benchmark_provider_ops": (C.c_int, [C.c_void_p, c_float_p, C.c_int, C.c_int,
                                             C.c_int, C.c_int, c_double_p, c_double_p,
                                             c_float_p]),
    "mgp_calibration_copy": (C.c_int, [C.c_int64, C.c_int, c_double_p]),
    "mgp_pipe_probe": (C.c_int, [c_double_p, C.c_int]),
    "mgp_train": (C.c_int, [C.c_void_p, c_float_p, c_float_p, C.c_int, C.c_float,
                            C.POINTER(TrainOpts), PROGRESS_CB, C.c_void_p,
                            C.POINTER(TrainResult)]),
    "mgp_train_mixed": (C.c_int, [C.c_void_p, c_float_p, c_float_p, C.c_int, C.c_float,
                                  C.POINTER(C.c_int), C.c_int, c_float_p, C.c_int,
                                  C.POINTER(TrainOpts), PROGRESS_CB, C.c_void_p,
                                  C.POINTER(TrainResult), c_float_p]),
    "mgp_predict": (C.c_int, [C.c_void_p, c_float_p, c_float_p, C.c_int64,
                              C.POINTER(PredictOpts), c_float_p, c_float_p, c_float_p,
                              c_float_p, c_float_p, c_float_p, C.POINTER(PredictInfo)]),
    "mgp_prepare_prediction_cache": (C.c_int, [C.c_void_p, c_float_p, C.POINTER(PredictOpts),
                                               c_float_p, c_void_pp, C.POINTER(PredictInfo)]),
    "mgp_predict_with_cache": (C.c_int, [C.c_void_p, C.c_void_p, c_float_p, C.c_int64, C.c_int,
                                         c_float_p, c_float_p, C.POINTER(PredictInfo)]),
    "mgp_destroy_prediction_cache": (C.c_int, [C.c_void_p]),
    "mgp_bbmm_eval": (C.c_int, [C.c_void_p, c_float_p, C.c_float, C.c_int, C.c_int, C.c_int,
                                C.c_float, C.c_int, C.c_int, c_float_p, c_float_p, c_float_p,
                                c_float_p, c_int_p, c_float_p, c_double_p]),
    "mgp_gaussian": (C.c_int, [C.c_int64, C.c_uint64, c_float_p]),
    "mgp_pivoted_cholesky": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_float, C.c_float,
                                       C.c_uint64, c_float_p, c_int_p, c_float_p]),
    "mgp_lmc_forward_matvec": (C.c_int, [c_void_pp, C.c_int, C.c_int, c_float_p, c_float_p,
                                         c_float_p, c_float_p, C.c_int, c_float_p]),
    "mgp_lmc_train": (C.c_int, [c_void_pp, C.c_int, C.c_int, c_float_p, c_float_p, c_int_p,
                                c_float_p, c_float_p, c_float_p, C.POINTER(LMCTrainOpts),
                                C.POINTER(LMCTrainResult)]),
    "mgp_lmc_train_mixed": (C.c_int, [c_void_pp, C.c_int, C.c_int, c_float_p, c_float_p,
                                      c_float_p, c_float_p, c_float_p, c_int_p, c_int_p,
                                      c_float_p, C.c_int, C.POINTER(LMCTrainOpts),
                                      C.POINTER(LMCTrainResult), c_float_p, c_float_p]),
    "mgp_lmc_bbmm_eval": (C.c_int, [c_void_pp, C.c_int, C.c_int, c_float_p, c_float_p,
                                    c_float_p, c_float_p, C.c_int, C.c_int, C.c_int, C.c_float,
                                    C.c_int, C.c_int, C.c_int, c_float_p, c_float_p, c_float_p,
                                    c_float_p, c_float_p, c_float_p, c_float_p, c_int_p,
                                    c_float_p, c_double_p]),
    "mgp_lmc_benchmark_forward": (C.c_int, [c_void_pp, C.c_int, C.c_int, c_float_p, c_float_p,
                                            c_float_p, C.c_int, C.c_int, C.c_int, c_double_p,
                                            c_float_p]),
    "mgp_lmc_predict": (C.c_int, [c_void_pp, C.c_int, C.c_int, c_float_p, c_float_p, c_float_p,
                                  c_float_p, c_float_p, C.c_int64, C.c_int, C.c_int, C.c_float,
                                  C.c_int, C.c_int, c_float_p, c_float_p, c_float_p]),
    "mgp_lmc_exact_variance": (C.c_int, [c_void_pp, C.c_int, C.c_int, c_float_p, c_float_p,
                                         c_float_p, c_float_p, C.c_int64, C.c_int, C.c_float,
                                         C.c_int, c_float_p, c_int_p]),
    "mgp_lmc_pathwise_correction": (C.c_int, [c_void_pp, C.c_int, C.c_int, c_float_p,
                                              c_float_p, c_float_p, c_float_p, C.c_int,
                                              c_float_p, C.c_int64, C.c_int, C.c_float,
                                              c_float_p, c_int_p]),
    "mgp_icm_train": (C.c_int, [C.c_void_p, C.c_int, c_float_p, c_float_p, c_int_p, c_float_p,
                                C.c_float, c_float_p, c_float_p, C.POINTER(ICMTrainOpts),
                                PROGRESS_CB, C.c_void_p, C.POINTER(ICMTrainResult)]),
    "mgp_icm_train_mixed": (C.c_int, [C.c_void_p, C.c_int, c_float_p, c_float_p, c_float_p,
                                      C.c_float, c_float_p, c_int_p, C.c_int, c_float_p,
                                      C.c_int, C.POINTER(ICMTrainOpts), PROGRESS_CB,
                                      C.c_void_p, C.POINTER(ICMTrainResult), c_float_p]),
    "mgp_icm_predict": (C.c_int, [C.c_void_p, C.c_int, c_float_p, c_float_p, c_float_p,
                                  c_float_p, C.c_int64, C.c_float, C.c_int, C.c_int, C.c_float,
                                  C.c_int, C.c_int, c_float_p, c_float_p]),
    "mgp_icm_bbmm_eval": (C.c_int, [C.c_void_p, C.c_int, C.c_float, c_float_p, c_float_p,
                                    c_float_p, c_float_p, C.c_int, C.c_int, C.c_int, C.c_float,
                                    C.c_int, C.c_int, C.c_int, c_float_p, c_float_p, c_float_p,
                                    c_float_p, c_float_p, c_float_p, c_float_p, c_float_p,
                                    c_int_p, c_float_p]),
    "mgp_kron_precond": (C.c_int, [C.c_void_p, C.c_int, C.c_float, c_float_p, c_float_p,
                                   C.c_int, C.c_int, c_float_p, C.c_int, c_float_p, C.c_int,
                                   C.c_uint64, c_float_p, c_float_p, c_int_p]),
    "mgp_icm_task_covariance_init": (C.c_int, [C.c_int, C.c_int, C.c_int, c_float_p]),
    "mgp_rff_prior_values": (C.c_int, [c_float_p, C.c_int64, C.c_int, c_double_p, c_double_p,
                                       c_double_p, C.c_int, C.c_double, c_double_p, C.c_int,
                                       c_float_p]),
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


def fn_address(name: str) -> int:
    """Address of an exported entry point (the provider dict's fn-pointer
    values)."""
    return int(C.cast(getattr(load(), name), C.c_void_p).value)


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


def ofptr(a):
    """fptr, or NULL for None."""
    return None if a is None else fptr(a)


def handles(providers) -> C.Array:
    """void*[R] array of provider handles."""
    arr = (C.c_void_p * len(providers))()
    for i, p in enumerate(providers):
        arr[i] = p.handle.value
    return arr


def dptr(a: np.ndarray):
    assert a.dtype == np.float64 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(c_double_p)


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)
