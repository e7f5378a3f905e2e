"""Python shims with the reference's native-module surface.

``KernelModule`` stands where the reference's generated fn-ptr kernel module
stands (``init_provider / materialize / destroy_provider``,
mojogp/codegen_engine/emit/fn_ptr_module.py:998-1211) and ``Engine`` where
``mojogp_jit_engine`` stands (``train / predict / prepare_prediction_cache /
predict_with_cache / destroy_prediction_cache / benchmark_provider_ops``,
mojogp/kernels/jit/jit_engine_bindings.mojo:1750-1775): same positional
arguments, same return-dict keys.  Every call goes to libmojogp_amd.so; there is
no CPU fallback.
"""

from __future__ import annotations

import ctypes as C
from typing import Any

import numpy as np

from . import _lib
from ._provider import TREE_KIND, NativeProvider, kind_code

_DEFAULT_PREDICT_LANCZOS_RANK = 100
_DEFAULT_ARD_PREDICT_LANCZOS_RANK = 200


def _exact_keys(inf, vm: int) -> dict[str, Any]:
    """Exact-variance diagnostics with the reference's result keys
    (jit_engine_bindings.mojo:1187-1196); cross mode 1 = direct fill."""
    if vm != 2:
        return {}
    return {"exact_block_cols": int(inf.exact_block_cols), "exact_cross_mode": 1,
            "exact_cg_block_count": int(inf.exact_cg_block_count),
            "exact_cg_total_iterations": int(inf.exact_cg_total_iterations),
            "exact_cg_max_iterations": int(inf.exact_cg_max_iterations),
            "exact_precond_rank": int(inf.exact_precond_rank)}


class KernelModule:
    """Kernel module for one (kernel family, ARD, input dimension), or for one
    composite kernel tree (``tree_spec``, ``KernelNode.to_tree_spec``)."""

    def __init__(self, kind, ard: bool, dim: int, tree_spec=None):
        self.tree_spec = None if tree_spec is None else [int(v) for v in tree_spec]
        self.kind = TREE_KIND if tree_spec is not None else kind_code(kind)
        self.ard = bool(ard) and tree_spec is None
        self.dim = int(dim)

    def init_provider(self, X, params, noise, observation_noise=None, noise_mode=None,
                      noise_group_train=None, num_noise_groups=None) -> dict[str, Any]:
        """Noise modes (fn_ptr_module.py:297-327): 0 scalar; 1 fixed per-point
        vector (observation_noise [n]); 2 learned per-point, 3 learned per
        group (noise_group_train [n], num_noise_groups), 4 learned linear
        function of the inputs — observation_noise holds the initial vector."""
        mode = 0 if noise_mode is None and observation_noise is None else (
            1 if noise_mode is None else int(noise_mode))
        if mode not in (0, 1, 2, 3, 4):
            raise ValueError(f"noise_mode must be 0-4, got {mode}")
        if mode >= 1 and observation_noise is None:
            raise ValueError(f"noise mode {mode} needs observation_noise")
        X = _lib.f32(X)
        if X.ndim != 2 or X.shape[1] != self.dim:
            raise ValueError(f"X must have shape (n, {self.dim})")
        prov = NativeProvider(self.kind, self.ard, X, params, noise, tree_spec=self.tree_spec)
        if mode >= 1:
            try:
                prov.set_noise_vector(observation_noise)
                if mode >= 2:
                    prov.set_learned_noise(mode, noise_group_train, num_noise_groups)
            except Exception:
                prov.close()
                raise
        return {
            "provider_ptr": int(prov.handle.value),
            "n": int(X.shape[0]),
            "dim": self.dim,
            "num_gradient_params": prov.nparams,
            "supports_fused_gradient": True,
            "supports_fused_ls_os": False,
            "supports_fused_3param": False,
            "x_ptr": 0,
            "is_ard": self.ard,
            "materialization_mode": 0,
            "noise_mode": mode,
            "has_observation_noise_vector": mode >= 1,
            "noise_group_ptr": 0,
            "num_noise_groups": 0,
            # the non-raising fn pointers, C-callable with the reference's
            # signatures (fn_ptr_module.py:1120-1166; the raising ones are
            # Mojo-ABI entry points only its engine calls, so they have no
            # counterpart here)
            "update_noise": _lib.fn_address("mgp_fn_update_noise"),
            "get_noise": _lib.fn_address("mgp_fn_get_noise"),
            "get_noise_mode": _lib.fn_address("mgp_fn_get_noise_mode"),
            "get_noise_vector_ptr": _lib.fn_address("mgp_fn_get_noise_vector_ptr"),
            "get_diagonal_value": _lib.fn_address("mgp_fn_get_diagonal_value"),
            "_provider": prov,
        }

    def materialize(self, info: dict) -> bool:
        """Select the materialized route: dense K on the device as a scaled
        two-term fp16 split, refilled on every parameter update, products on
        the hand-written fp16 matrix-core kernels (materialize /
        _do_materialize, fn_ptr_module.py:363-384, 1168-1181)."""
        _provider(info).materialize()
        info["materialization_mode"] = 1
        return True

    def destroy_provider(self, info: dict) -> bool:
        prov = info.get("_provider")
        if prov is not None:
            prov.close()
        info["provider_ptr"] = 0
        info["x_ptr"] = 0
        info["materialization_mode"] = 0
        info["_provider"] = None
        return True


def _provider(info: dict) -> NativeProvider:
    prov = info.get("_provider")
    if prov is None or not info.get("provider_ptr"):
        raise RuntimeError("provider_info does not hold a live provider")
    return prov


def _resolve_lanczos_rank(info: dict, requested: int) -> int:
    """jit_engine_binding_helpers.mojo:23-45 (single-output, non-mixed)."""
    if requested > 0:
        return int(requested)
    rank = _DEFAULT_PREDICT_LANCZOS_RANK
    if info.get("is_ard"):
        rank = max(rank, _DEFAULT_ARD_PREDICT_LANCZOS_RANK)
    return rank


def _progress_bridge(callback, model: str = "single_output"):
    if callback is None:
        null = _lib.PROGRESS_CB()  # NULL function pointer
        return null, null

    def _cb(ev_ptr, _user):
        ev = ev_ptr.contents
        stats = {"nll": float(ev.nll), "best_nll": float(ev.best_nll)}
        if ev.cg_iter >= 0:
            stats["cg_iter"] = int(ev.cg_iter)
        if ev.iter_ms >= 0:
            stats["iter_ms"] = float(ev.iter_ms)
        if ev.noise >= 0:
            stats["noise"] = float(ev.noise)
        stats["mean"] = float(ev.mean)
        if ev.precond_rank >= 0:
            stats["precond_rank"] = int(ev.precond_rank)
        if ev.precond_rebuild_count >= 0:
            stats["precond_rebuild_count"] = int(ev.precond_rebuild_count)
        event = {
            "operation": "train", "model": model, "route": "unknown",
            "phase": ev.phase.decode(), "current": int(ev.current), "total": int(ev.total),
            "converged": bool(ev.converged), "stats": stats,
        }
        callback(event)

    cfun = _lib.PROGRESS_CB(_cb)
    return cfun, cfun


class Engine:
    """Engine module: training and prediction entry points."""

    # ------------------------------------------------------------ train
    def train(self, *args, nan_inject_mask: int = 0) -> dict[str, Any]:
        """train_python (jit_engine_bindings.mojo:123-432).  ``nan_inject_mask``
        (keyword only, tests): bit i treats the NLL of iteration i as NaN so
        the recovery path runs."""
        if len(args) < 17 or len(args) > 25:
            raise ValueError("train() expects between 17 and 25 positional arguments")
        info, y, params, init_noise = args[0], args[1], args[2], float(args[3])
        prov = _provider(info)
        o = _lib.TrainOpts()
        o.max_iterations = int(args[4])
        o.learning_rate = float(args[5])
        o.num_probes = int(args[6])
        o.max_cg_iter = int(args[7])
        o.cg_tol = float(args[8])
        o.precond_rank = int(args[9])
        o.verbose = int(bool(args[10]))
        o.use_cosine_lr = int(bool(args[11]))
        o.use_preconditioner = int(bool(args[12]))
        o.max_tridiag_iter = int(args[13])
        o.precond_rebuild_threshold = float(args[14])
        o.precond_method = int(args[15])
        o.init_mean = float(args[16])
        o.enable_early_stopping = int(bool(args[17])) if len(args) > 17 else 0
        o.early_stop_patience = int(args[18]) if len(args) > 18 else 10
        o.early_stop_tol = float(args[19]) if len(args) > 19 else 1e-4
        o.learn_noise = int(bool(args[20])) if len(args) > 20 else 1
        o.noise_floor = float(args[21]) if len(args) > 21 else 1e-6
        o.noise_regularization = float(args[22]) if len(args) > 22 else 0.01
        callback = args[23] if len(args) > 23 else None
        o.progress_interval = int(args[24]) if len(args) > 24 else 1
        o.nan_inject_mask = int(nan_inject_mask)
        if o.max_iterations <= 0:
            raise ValueError("max_iterations must be > 0")

        y = _lib.f32(y).ravel()
        params = _lib.f32(params).ravel()
        n, P, T = prov.n, prov.nparams, o.max_iterations
        out_params = np.zeros(P, np.float32)
        nll_h = np.zeros(T, np.float32)
        times = np.zeros(T, np.float64)
        cg_h = np.zeros(T, np.int32)
        rank_h = np.zeros(T, np.int32)
        rebuild = np.zeros(T, np.int32)
        alpha = np.zeros(n, np.float32)
        learned = np.zeros(n, np.float32)
        fnp = np.zeros(prov.d + 1, np.float32)
        res = _lib.TrainResult()
        res.learned_noise = _lib.fptr(learned)
        res.noise_fn_params = _lib.fptr(fnp)
        res.params = _lib.fptr(out_params)
        res.nll_history = _lib.fptr(nll_h)
        res.iter_times_ms = _lib.dptr(times)
        res.cg_iterations_history = cg_h.ctypes.data_as(_lib.c_int_p)
        res.precond_rank_history = rank_h.ctypes.data_as(_lib.c_int_p)
        res.precond_rebuild_steps = rebuild.ctypes.data_as(_lib.c_int_p)
        res.cached_alpha = _lib.fptr(alpha)
        cfun, _keep = _progress_bridge(callback)
        _lib.call("mgp_train", prov.handle, _lib.fptr(y), _lib.fptr(params), P, init_noise,
                  C.byref(o), cfun, None, C.byref(res))
        # The native loop left the provider at its last evaluated state.
        hl = res.history_len
        out = {
            "final_nll": float(res.final_nll),
            "noise": float(res.noise),
            "mean": float(res.mean),
            "iterations": int(res.iterations),
            "converged": bool(res.converged),
            "training_route": "materialized" if info.get("materialization_mode") == 1 else "matrix_free",
            "materialization_mode": int(info.get("materialization_mode", 0)),
            "is_ard": bool(info.get("is_ard", False)),
            "precond_method": int(o.precond_method),
            "precond_rank": int(o.precond_rank),
            "max_tridiag_iter": int(o.max_tridiag_iter),
            "precond_rebuild_threshold": float(o.precond_rebuild_threshold),
            "use_preconditioner": bool(o.use_preconditioner),
            "learn_noise": bool(o.learn_noise),
            "noise_floor": float(o.noise_floor),
            "noise_regularization": float(o.noise_regularization),
            "enable_early_stopping": bool(o.enable_early_stopping),
            "early_stop_patience": int(o.early_stop_patience),
            "early_stop_tol": float(o.early_stop_tol),
            "params": [float(v) for v in out_params],
            "iter_times_ms": [float(v) for v in times[:hl]],
            "nll_history": [float(v) for v in nll_h[:hl]],
            "cg_iterations_history": [int(v) for v in cg_h[:res.cg_history_len]],
            "precond_rank_history": [int(v) for v in rank_h[:res.rank_history_len]],
            "precond_rebuild_steps": [int(v) for v in rebuild[:res.rebuild_steps_len]],
            "precond_build_count": int(res.precond_build_count),
            "precond_rebuild_count": max(0, int(res.precond_build_count) - 1),
            "precond_build_total_ms": float(res.precond_build_total_ms),
            "actual_precond_rank": int(rank_h[res.rank_history_len - 1]) if res.rank_history_len else 0,
        }
        if res.has_alpha:
            out["cached_alpha"] = alpha
        if res.has_learned_noise:
            out["learned_observation_noise"] = learned
        if res.noise_fn_len:
            out["learned_noise_function_params"] = fnp[:res.noise_fn_len].copy()
        return out

    # ------------------------------------------------------------ mixed
    _CAT_KIND = {"gd": 0, "cr": 1, "ehh": 2, "hh": 3, "fe": 4}

    def train_mixed(self, *args) -> dict[str, Any]:
        """train_mixed (jit_engine_bindings.mojo:1241-1460): args = info, y,
        continuous params, noise, C [n, ncat] int32, cat_specs
        ({"levels", "kernel_type"} per categorical leaf in tree order), raw
        categorical params, then max_iterations, learning_rate, num_probes,
        max_cg_iter, cg_tol, precond_rank, verbose, method, precond_method,
        enable_early_stopping, early_stop_patience, early_stop_tol, callback,
        progress_interval.  The binding's loop defaults hold: cosine rate,
        mean from 0, 30 Lanczos steps, rebuild threshold 0.5.  The provider
        reads each leaf's levels from its input column (C must match it)."""
        if len(args) < 7 or len(args) > 21:
            raise ValueError("train_mixed() expects between 7 and 21 positional arguments")
        info, y, params, init_noise, Cmat, specs, cat_init = args[:7]
        prov = _provider(info)
        Cmat = np.asarray(Cmat)
        if Cmat.ndim != 2 or Cmat.shape[0] != prov.n or Cmat.shape[1] != len(specs):
            raise ValueError("cat_data must have shape (n, number of categorical leaves)")
        o = _lib.TrainOpts()
        o.max_iterations = int(args[7]) if len(args) > 7 else 100
        o.learning_rate = float(args[8]) if len(args) > 8 else 0.01
        o.num_probes = int(args[9]) if len(args) > 9 else 10
        o.max_cg_iter = int(args[10]) if len(args) > 10 else 100
        o.cg_tol = float(args[11]) if len(args) > 11 else 1e-2
        o.precond_rank = int(args[12]) if len(args) > 12 else 10
        o.verbose = int(bool(args[13])) if len(args) > 13 else 0
        method = int(args[14]) if len(args) > 14 else 0
        o.precond_method = int(args[15]) if len(args) > 15 else 0
        o.enable_early_stopping = int(bool(args[16])) if len(args) > 16 else 0
        o.early_stop_patience = int(args[17]) if len(args) > 17 else 10
        o.early_stop_tol = float(args[18]) if len(args) > 18 else 1e-4
        callback = args[19] if len(args) > 19 else None
        o.progress_interval = int(args[20]) if len(args) > 20 else 1
        o.use_cosine_lr, o.use_preconditioner, o.max_tridiag_iter = 1, 1, 30
        o.precond_rebuild_threshold, o.init_mean, o.learn_noise = 0.5, 0.0, 1
        o.noise_floor, o.noise_regularization = 1e-6, 0.0
        if o.max_iterations <= 0:
            raise ValueError("max_iterations must be > 0")
        kinds = np.array([self._CAT_KIND[str(s["kernel_type"]).lower()] for s in specs],
                         np.int32)
        cat_init = _lib.f32(cat_init).ravel()
        y = _lib.f32(y).ravel()
        params = _lib.f32(params).ravel()
        P, T = prov.nparams, o.max_iterations
        out_params = np.zeros(P, np.float32)
        nll_h = np.zeros(T, np.float32)
        times = np.zeros(T, np.float64)
        cg_h = np.zeros(T, np.int32)
        cat_out = np.zeros(max(cat_init.size, 1), np.float32)
        res = _lib.TrainResult()
        res.params = _lib.fptr(out_params)
        res.nll_history = _lib.fptr(nll_h)
        res.iter_times_ms = _lib.dptr(times)
        res.cg_iterations_history = cg_h.ctypes.data_as(_lib.c_int_p)
        cfun, _keep = _progress_bridge(callback)
        _lib.call("mgp_train_mixed", prov.handle, _lib.fptr(y), _lib.fptr(params), P,
                  float(init_noise), kinds.ctypes.data_as(C.POINTER(C.c_int)), int(kinds.size),
                  _lib.fptr(cat_init), int(cat_init.size), C.byref(o), cfun, None, C.byref(res),
                  _lib.fptr(cat_out))
        prov.cat_kinds, prov.cat_raw = kinds, cat_out[:cat_init.size].copy()
        hl = res.history_len
        return {
            "status": "trained", "num_cat_vars": int(kinds.size),
            "total_cat_params": int(cat_init.size), "num_cont_params": P,
            "nll": float(res.final_nll), "noise": float(res.noise), "mean": float(res.mean),
            "iterations": int(res.iterations), "converged": bool(res.converged),
            "training_route": "materialized" if method == 1 else "matrix_free",
            "materialization_mode": method, "precond_method": int(o.precond_method),
            "precond_rank": int(o.precond_rank),
            "enable_early_stopping": bool(o.enable_early_stopping),
            "early_stop_patience": int(o.early_stop_patience),
            "early_stop_tol": float(o.early_stop_tol),
            "params": [float(v) for v in out_params],
            "cat_params": cat_out[:cat_init.size].copy(),
            "iter_times_ms": [float(v) for v in times[:hl]],
            "nll_history": [float(v) for v in nll_h[:hl]],
            "cg_iterations_history": [int(v) for v in cg_h[:res.cg_history_len]],
        }

    # ------------------------------------------------------------ predict
    def predict(self, *args) -> dict[str, Any]:
        if len(args) < 7 or len(args) > 16:
            raise ValueError("predict() expects 7 to 16 positional arguments")
        info, y, Xs, params = args[0], args[1], args[2], args[3]
        noise, mean, vm = float(args[4]), float(args[5]), int(args[6])
        max_cg = int(args[7]) if len(args) > 7 else 100
        tol = float(args[8]) if len(args) > 8 else 1e-2
        precond_rank = int(args[9]) if len(args) > 9 else 10
        lanczos_rank = int(args[10]) if len(args) > 10 else 0
        state_current = bool(args[11]) if len(args) > 11 else False
        exact_cols = int(args[12]) if len(args) > 12 else 0
        alpha_in = _lib.f32(args[13]).ravel() if len(args) > 13 and args[13] is not None else None
        root_in = _lib.f32(args[14]).ravel() if len(args) > 14 and args[14] is not None else None
        prov = _provider(info)
        lanczos_rank = _resolve_lanczos_rank(info, lanczos_rank)
        if not state_current:
            prov.update_params(params)
            prov.update_noise(noise)
        Xs = _lib.f32(Xs)
        m = Xs.shape[0]
        y = _lib.f32(y).ravel()
        if root_in is not None and root_in.size != prov.n * lanczos_rank:
            root_in = None
        o = _lib.PredictOpts(mean, vm, max_cg, tol, precond_rank, lanczos_rank, exact_cols)
        mean_out = np.zeros(m, np.float32)
        var_out = np.zeros(m, np.float32)
        alpha_out = np.zeros(prov.n, np.float32)
        root_out = np.zeros(prov.n * lanczos_rank, np.float32) if vm == 1 and root_in is None else None
        inf = _lib.PredictInfo()
        _lib.call("mgp_predict", prov.handle, _lib.fptr(y), _lib.fptr(Xs), m, C.byref(o),
                  None if alpha_in is None else _lib.fptr(alpha_in),
                  None if root_in is None else _lib.fptr(root_in),
                  _lib.fptr(mean_out), _lib.fptr(var_out), _lib.fptr(alpha_out),
                  None if root_out is None else _lib.fptr(root_out), C.byref(inf))
        out = {
            "mean": mean_out,
            "variance": var_out if vm != 0 else np.zeros(m, np.float32),
            "std": np.sqrt(var_out) if vm != 0 else np.zeros(m, np.float32),
            "alpha_time_s": inf.alpha_time_s,
            "mean_time_s": inf.mean_time_s,
            "variance_time_s": inf.variance_time_s,
            "total_time_s": inf.total_time_s,
            "love_root_time_s": inf.love_root_time_s,
            "provider_state_update_skipped": state_current,
            "alpha_cache_used": bool(inf.alpha_cache_used),
            "love_root_cache_used": bool(inf.love_root_cache_used),
            "alpha_cg_iterations": int(inf.alpha_cg_iterations),
        }
        out.update(_exact_keys(inf, vm))
        if alpha_in is None:
            out["cached_alpha"] = alpha_out
        if root_out is not None:
            out["cached_lanczos_root"] = root_out
        return out

    # ------------------------------------------------------------ cache
    def prepare_prediction_cache(self, *args) -> dict[str, Any]:
        if len(args) < 11 or len(args) > 13:
            raise ValueError("prepare_prediction_cache() expects 11 to 13 positional arguments")
        info, y, params = args[0], args[1], args[2]
        noise, mean, vm = float(args[3]), float(args[4]), int(args[5])
        max_cg, tol, precond_rank = int(args[6]), float(args[7]), int(args[8])
        lanczos_rank = _resolve_lanczos_rank(info, int(args[9]))
        state_current = bool(args[10])
        alpha_in = _lib.f32(args[11]).ravel() if len(args) > 11 and args[11] is not None else None
        prov = _provider(info)
        if not state_current:
            prov.update_params(params)
            prov.update_noise(noise)
        y = _lib.f32(y).ravel()
        o = _lib.PredictOpts(mean, vm, max_cg, tol, precond_rank, lanczos_rank, 0)
        h = C.c_void_p()
        inf = _lib.PredictInfo()
        _lib.call("mgp_prepare_prediction_cache", prov.handle, _lib.fptr(y), C.byref(o),
                  None if alpha_in is None else _lib.fptr(alpha_in), C.byref(h), C.byref(inf))
        return {"cache_handle": int(h.value), "variance_method": vm,
                "lanczos_rank": lanczos_rank, "alpha_time_s": inf.alpha_time_s,
                "love_root_time_s": inf.love_root_time_s,
                "alpha_cache_used": bool(inf.alpha_cache_used)}

    def predict_with_cache(self, *args) -> dict[str, Any]:
        info, handle, Xs = args[0], int(args[1]), _lib.f32(args[2])
        vm = int(args[6]) if len(args) > 6 else 1
        prov = _provider(info)
        m = Xs.shape[0]
        mean_out = np.zeros(m, np.float32)
        var_out = np.zeros(m, np.float32)
        inf = _lib.PredictInfo()
        _lib.call("mgp_predict_with_cache", prov.handle, C.c_void_p(handle), _lib.fptr(Xs), m, vm,
                  _lib.fptr(mean_out), _lib.fptr(var_out), C.byref(inf))
        out = {"mean": mean_out,
               "variance": var_out if vm != 0 else np.zeros(m, np.float32),
               "std": np.sqrt(var_out) if vm != 0 else np.zeros(m, np.float32),
               "total_time_s": inf.total_time_s, "alpha_cache_used": True,
               "love_root_cache_used": bool(inf.love_root_cache_used)}
        out.update(_exact_keys(inf, vm))
        return out

    def destroy_prediction_cache(self, handle) -> bool:
        if handle:
            _lib.call("mgp_destroy_prediction_cache", C.c_void_p(int(handle)))
        return True

    # ------------------------------------------------------------ bench
    def benchmark_provider_ops(self, info, rhs, num_cols, op_code, repeats, warmup) -> dict:
        """jit_engine_bindings.mojo:439-572: op 0 forward, 1 fused gradient,
        2 fused gradient + dots, 3 dots only after one gradient pass."""
        op = int(op_code)
        if op < 0 or op > 3:
            raise ValueError("op_code must be one of 0, 1, 2, 3")
        prov = _provider(info)
        V = _lib.f32(rhs)
        if V.size != prov.n * int(num_cols):
            raise ValueError("rhs size does not match n * num_cols")
        V = V.reshape(int(num_cols), prov.n)
        times, tile_ms, out = prov.benchmark_op(V, op, int(repeats), int(warmup))
        res = {"n": prov.n, "num_cols": int(num_cols), "num_params": prov.nparams,
               "op_code": op, "repeats": int(repeats), "warmup": int(warmup),
               "times_ms": [float(t) for t in times], "tile_kernel_ms": tile_ms}
        if op == 0:
            res["output_column_major"] = out.ravel()
        return res

    # ------------------------------------------------------------ LMC
    def train_lmc(self, *args) -> dict[str, Any]:
        """train_lmc(provider_infos, init_params_per_latent, trainable_masks, Y [n, T],
        num_tasks, max_iters, lr, verbose, num_probes, max_cg_iter, cg_tol,
        precond_rank, precond_method, precond_rebuild_threshold, max_tridiag_iter,
        init_noise [T], fixed_noise [n, T], has_fixed_noise, init_mean [T]
        [, progress_callback, progress_interval])
        (train_lmc_python, jit_engine_lmc_bindings.mojo:365-597)."""
        if len(args) < 19 or len(args) > 21:
            raise ValueError("train_lmc() expects 19 to 21 positional arguments")
        infos = list(args[0])
        provs = [_provider(i) for i in infos]
        R = len(provs)
        Y = _lib.f32(args[3])
        T = int(args[4])
        if Y.ndim != 2 or Y.shape[1] != T:
            raise ValueError("Y must have shape (n, num_tasks)")
        n = Y.shape[0]
        init_params, masks = [], []
        for s, prov in enumerate(provs):
            p = _lib.f32(args[1][s]).ravel()
            m = np.ascontiguousarray(args[2][s], dtype=bool).ravel()
            if p.shape[0] != prov.nparams:
                raise ValueError("train_lmc() initial params length does not match provider "
                                 "gradient params")
            if m.shape[0] != prov.nparams:
                raise ValueError("train_lmc() trainable mask length does not match provider "
                                 "gradient params")
            init_params.append(p)
            masks.append(m)
        o = _lib.LMCTrainOpts()
        o.max_iterations = int(args[5])
        o.learning_rate = float(args[6])
        o.num_probes = int(args[8])
        o.max_cg_iter = int(args[9])
        o.cg_tol = float(args[10])
        o.precond_rank = int(args[11])
        o.precond_method = int(args[12])
        o.precond_rebuild_threshold = float(args[13])
        o.max_tridiag_iter = int(args[14])
        o.early_stop_tol = 1e-4
        o.early_stop_patience = 15
        if o.max_iterations <= 0:
            raise ValueError("max_iterations must be > 0")
        noise0 = _lib.f32(args[15]).ravel()
        fixed = None
        if bool(args[17]):
            fn = _lib.f32(args[16])
            if fn.shape != (n, T):
                raise ValueError("train_lmc() fixed observation noise must have shape [n, T]")
            fixed = np.ascontiguousarray(fn.T)
        mean0 = _lib.f32(args[18]).ravel()
        y_blocked = np.ascontiguousarray(Y.T)
        flat_p = np.concatenate(init_params).astype(np.float32)
        flat_m = np.concatenate(masks).astype(np.int32)
        it_max = o.max_iterations
        out_params = np.zeros_like(flat_p)
        A = np.zeros((R, T, T), np.float32)
        L = np.zeros((R, T, T), np.float32)
        vd = np.zeros((R, T), np.float32)
        noise = np.zeros(T, np.float32)
        mean = np.zeros(T, np.float32)
        alpha = np.zeros(n * T, np.float32)
        hist = np.zeros(it_max, np.float32)
        times = np.zeros(it_max, np.float64)
        res = _lib.LMCTrainResult()
        res.params, res.A, res.L = _lib.fptr(out_params), _lib.fptr(A), _lib.fptr(L)
        res.var_diag, res.noise, res.mean = _lib.fptr(vd), _lib.fptr(noise), _lib.fptr(mean)
        res.alpha, res.nll_history = _lib.fptr(alpha), _lib.fptr(hist)
        res.iter_times_ms = _lib.dptr(times)
        _lib.call("mgp_lmc_train", _lib.handles(provs), R, T, _lib.fptr(y_blocked),
                  _lib.fptr(flat_p), flat_m.ctypes.data_as(_lib.c_int_p), _lib.fptr(noise0),
                  _lib.ofptr(fixed), _lib.fptr(mean0), C.byref(o), C.byref(res))
        hl = int(res.history_len)
        per_latent, off = [], 0
        for prov in provs:
            per_latent.append([float(v) for v in out_params[off:off + prov.nparams]])
            prov.params = out_params[off:off + prov.nparams].copy()
            prov.noise = 0.0
            off += prov.nparams
        mode = int(infos[0].get("materialization_mode", 0))
        return {
            "status": "trained", "model_type": "lmc", "num_latents": R, "num_tasks": T, "n": n,
            "final_nll": float(res.final_nll), "iterations": int(res.iterations),
            "converged": bool(res.converged), "max_tridiag_iter": o.max_tridiag_iter,
            "precond_rebuild_threshold": o.precond_rebuild_threshold,
            "precond_rebuild_count": int(res.precond_rebuild_count),
            "precond_rank": o.precond_rank, "precond_method": o.precond_method,
            "uses_fixed_observation_noise": fixed is not None,
            "training_route": "materialized" if mode == 1 else "matrix_free",
            "materialization_mode": mode,
            "params_per_latent": per_latent,
            "noise_per_task": [float(v) for v in noise],
            "mean_per_task": [float(v) for v in mean],
            "A_matrices": A, "L_factors": L, "var_diag": vd, "alpha": alpha,
            "nll_history": [float(v) for v in hist[:hl]],
            "iter_times_ms": [float(v) for v in times[:hl]],
        }

    def train_lmc_mixed(self, *args) -> dict[str, Any]:
        """train_lmc_mixed(provider_infos, init_params_per_latent, Y [n, T], num_tasks,
        latent_C_trains, latent_cat_specs, cat_init_params_per_latent, max_iters, lr,
        verbose, num_probes, max_cg_iter, cg_tol, precond_rank, precond_method,
        precond_rebuild_threshold, max_tridiag_iter, init_noise [T], fixed_noise [n, T],
        has_fixed_noise, init_mean [T], method_int [, progress_callback,
        progress_interval]) (train_lmc_mixed_python, jit_engine_lmc_bindings.mojo:54-360).

        latent_cat_specs[s]: one {"levels", "kernel_type"} dict per categorical
        leaf of latent s in tree order; latent_C_trains[s]: their integer
        level columns [n, len(specs)] (the tree provider reads the levels from
        its input columns, so these must match them); cat_init: their raw
        parameters.  Returns the reference's dict (``cat_params_per_latent``
        constrained) plus ``cat_raw_per_latent``."""
        if len(args) < 22 or len(args) > 24:
            raise ValueError("train_lmc_mixed() expects 22 to 24 positional arguments")
        infos = list(args[0])
        provs = [_provider(i) for i in infos]
        R = len(provs)
        Y = _lib.f32(args[2])
        T = int(args[3])
        if Y.ndim != 2 or Y.shape[1] != T:
            raise ValueError("Y must have shape (n, num_tasks)")
        n = Y.shape[0]
        if int(args[21]) == 2:
            raise ValueError("method int 2 is not a public MojoGP training route")
        Cs, specs, cat0 = list(args[4]), list(args[5]), list(args[6])
        if not (len(args[1]) == len(Cs) == len(specs) == len(cat0) == R):
            raise ValueError("train_lmc_mixed() needs one entry per latent in every "
                             "per-latent list")
        init_params, counts, kinds, raws = [], [], [], []
        for s, prov in enumerate(provs):
            p = _lib.f32(args[1][s]).ravel()
            if p.shape[0] != prov.nparams:
                raise ValueError("train_lmc_mixed() initial params length does not match "
                                 "provider gradient params")
            init_params.append(p)
            Cm = np.asarray(Cs[s])
            if Cm.ndim != 2 or Cm.shape != (n, len(specs[s])):
                raise ValueError(f"latent {s}: C_train must have shape (n, number of "
                                 "categorical leaves)")
            counts.append(len(specs[s]))
            kinds.extend(self._CAT_KIND[str(sp["kernel_type"]).lower()] for sp in specs[s])
            raws.append(_lib.f32(cat0[s]).ravel())
        o = _lib.LMCTrainOpts()
        o.max_iterations = int(args[7])
        o.learning_rate = float(args[8])
        o.num_probes = int(args[10])
        o.max_cg_iter = int(args[11])
        o.cg_tol = float(args[12])
        o.precond_rank = int(args[13])
        o.precond_method = int(args[14])
        o.precond_rebuild_threshold = float(args[15])
        o.max_tridiag_iter = int(args[16])
        o.early_stop_tol = 1e-4
        o.early_stop_patience = 15
        if o.max_iterations <= 0:
            raise ValueError("max_iterations must be > 0")
        noise0 = _lib.f32(args[17]).ravel()
        fixed = None
        if bool(args[19]):
            fn = _lib.f32(args[18])
            if fn.shape != (n, T):
                raise ValueError("train_lmc_mixed() fixed observation noise must have shape [n, T]")
            fixed = np.ascontiguousarray(fn.T)
        mean0 = _lib.f32(args[20]).ravel()
        y_blocked = np.ascontiguousarray(Y.T)
        flat_p = np.concatenate(init_params).astype(np.float32)
        flat_raw = (np.concatenate(raws) if raws else np.zeros(0)).astype(np.float32)
        cnt = np.asarray(counts, np.int32)
        knd = np.asarray(kinds if kinds else [0], np.int32)
        it_max = o.max_iterations
        out_params = np.zeros_like(flat_p)
        A = np.zeros((R, T, T), np.float32)
        L = np.zeros((R, T, T), np.float32)
        vd = np.zeros((R, T), np.float32)
        noise = np.zeros(T, np.float32)
        mean = np.zeros(T, np.float32)
        alpha = np.zeros(n * T, np.float32)
        hist = np.zeros(it_max, np.float32)
        times = np.zeros(it_max, np.float64)
        raw_out = np.zeros(max(flat_raw.size, 1), np.float32)
        con_out = np.zeros(max(flat_raw.size, 1), np.float32)
        res = _lib.LMCTrainResult()
        res.params, res.A, res.L = _lib.fptr(out_params), _lib.fptr(A), _lib.fptr(L)
        res.var_diag, res.noise, res.mean = _lib.fptr(vd), _lib.fptr(noise), _lib.fptr(mean)
        res.alpha, res.nll_history = _lib.fptr(alpha), _lib.fptr(hist)
        res.iter_times_ms = _lib.dptr(times)
        _lib.call("mgp_lmc_train_mixed", _lib.handles(provs), R, T, _lib.fptr(y_blocked),
                  _lib.fptr(flat_p), _lib.fptr(noise0), _lib.ofptr(fixed), _lib.fptr(mean0),
                  cnt.ctypes.data_as(_lib.c_int_p), knd.ctypes.data_as(_lib.c_int_p),
                  _lib.fptr(flat_raw if flat_raw.size else raw_out), int(flat_raw.size),
                  C.byref(o), C.byref(res), _lib.fptr(raw_out), _lib.fptr(con_out))
        hl = int(res.history_len)
        per_latent, cat_con, cat_raw = [], [], []
        off = roff = koff = 0
        for s, prov in enumerate(provs):
            per_latent.append([float(v) for v in out_params[off:off + prov.nparams]])
            prov.params = out_params[off:off + prov.nparams].copy()
            prov.noise = 0.0
            off += prov.nparams
            k = raws[s].size
            cat_con.append([float(v) for v in con_out[roff:roff + k]])
            cat_raw.append(raw_out[roff:roff + k].copy())
            if counts[s]:
                prov.cat_kinds = knd[koff:koff + counts[s]].copy()
                prov.cat_raw = cat_raw[-1]
            roff += k
            koff += counts[s]
        mode = int(args[21])
        return {
            "status": "trained", "model_type": "lmc_mixed", "num_latents": R, "num_tasks": T,
            "n": n, "final_nll": float(res.final_nll), "iterations": int(res.iterations),
            "converged": bool(res.converged), "max_tridiag_iter": o.max_tridiag_iter,
            "precond_rebuild_threshold": o.precond_rebuild_threshold,
            "precond_rebuild_count": int(res.precond_rebuild_count),
            "precond_rank": o.precond_rank, "precond_method": o.precond_method,
            "uses_fixed_observation_noise": fixed is not None,
            "training_route": "materialized" if mode == 1 else "matrix_free",
            "materialization_mode": mode,
            "params_per_latent": per_latent, "cat_params_per_latent": cat_con,
            "cat_raw_per_latent": cat_raw,
            "noise_per_task": [float(v) for v in noise],
            "mean_per_task": [float(v) for v in mean],
            "A_matrices": A, "L_factors": L, "var_diag": vd, "alpha": alpha,
            "nll_history": [float(v) for v in hist[:hl]],
            "iter_times_ms": [float(v) for v in times[:hl]],
        }

    def predict_lmc(self, *args) -> dict[str, Any]:
        """predict_lmc(provider_infos, alpha [n*T], A [R, T, T], X_test [m, d],
        params_per_latent, mean_per_task [T], n_train, num_tasks
        [, noise_per_task [T], variance_method, max_cg_iter, cg_tol, precond_rank,
        lanczos_rank]) (predict_lmc_python, jit_engine_lmc_bindings.mojo:1102-1394)."""
        if len(args) < 8:
            raise ValueError("predict_lmc() expects at least 8 positional arguments")
        infos = list(args[0])
        provs = [_provider(i) for i in infos]
        R = len(provs)
        T = int(args[7])
        alpha = _lib.f32(args[1]).ravel()
        A = _lib.f32(args[2]).reshape(R, T, T)
        Xs = _lib.f32(args[3])
        for s, prov in enumerate(provs):
            prov.update_params(_lib.f32(args[4][s]).ravel())
        mean = _lib.f32(args[5]).ravel()
        if alpha.shape[0] != int(args[6]) * T:
            raise ValueError("alpha must have n_train * num_tasks entries")
        noise = _lib.f32(args[8]).ravel() if len(args) > 8 else None
        vm = int(args[9]) if len(args) > 9 else 0
        max_cg = int(args[10]) if len(args) > 10 else 100
        tol = float(args[11]) if len(args) > 11 else 1e-2
        prank = int(args[12]) if len(args) > 12 else 10
        lrank = int(args[13]) if len(args) > 13 else 0
        if lrank <= 0:
            lrank = _DEFAULT_PREDICT_LANCZOS_RANK
            if any(i.get("is_ard") for i in infos):
                lrank = max(lrank, _DEFAULT_ARD_PREDICT_LANCZOS_RANK)
        if noise is None:
            vm = 0
        m = Xs.shape[0]
        mean_out = np.zeros((m, T), np.float32)
        var = np.zeros((m, T), np.float32) if vm else None
        lat = np.zeros((R, m), np.float32) if vm else None
        _lib.call("mgp_lmc_predict", _lib.handles(provs), R, T, _lib.fptr(A), _lib.fptr(alpha),
                  _lib.fptr(mean), _lib.ofptr(noise), _lib.fptr(Xs), m, vm, max_cg, tol, prank,
                  lrank, _lib.fptr(mean_out), _lib.ofptr(var), _lib.ofptr(lat))
        out = {"mean": mean_out, "lanczos_rank_used": lrank}
        if vm:
            out["variance"] = var
            out["std"] = np.sqrt(var)
            out["latent_variances"] = lat
        return out

    def sample_lmc_pathwise(self, *args) -> dict[str, Any]:
        """sample_lmc_pathwise(provider_infos, residual [n, T] (or [S, n, T]), A, X_test,
        params_per_latent, noise_per_task [, max_cg_iter, cg_tol, fixed_noise [n, T]])
        (sample_lmc_pathwise_python, jit_engine_lmc_bindings.mojo:599-797).  A 3-D
        residual stack is corrected in one batched solve; 'correction' then has
        shape [S, m, T]."""
        if len(args) < 6 or len(args) > 9:
            raise ValueError("sample_lmc_pathwise() expects 6-9 positional arguments")
        infos = list(args[0])
        provs = [_provider(i) for i in infos]
        R = len(provs)
        resid = _lib.f32(args[1])
        single = resid.ndim == 2
        if single:
            resid = resid[None]
        S, n, T = resid.shape
        A = _lib.f32(args[2]).reshape(R, T, T)
        Xs = _lib.f32(args[3])
        for s, prov in enumerate(provs):
            prov.update_params(_lib.f32(args[4][s]).ravel())
            prov.update_noise(0.0)
        noise = _lib.f32(args[5]).ravel()
        max_cg = int(args[6]) if len(args) > 6 else 100
        tol = float(args[7]) if len(args) > 7 else 1e-2
        fixed = None
        if len(args) > 8:
            fn = _lib.f32(args[8])
            if fn.size == n * T:
                fixed = np.ascontiguousarray(fn.reshape(n, T).T)
        blocked = np.ascontiguousarray(resid.transpose(0, 2, 1))
        m = Xs.shape[0]
        corr = np.zeros((S, m, T), np.float32)
        its = C.c_int(0)
        _lib.call("mgp_lmc_pathwise_correction", _lib.handles(provs), R, T, _lib.fptr(A),
                  _lib.fptr(noise), _lib.ofptr(fixed), _lib.fptr(blocked), S, _lib.fptr(Xs), m,
                  max_cg, tol, _lib.fptr(corr), C.byref(its))
        return {"correction": corr[0] if single else corr, "cg_iterations": int(its.value)}


    # ------------------------------------------------------------ ICM
    def train_multi_output(self, *args) -> dict[str, Any]:
        """train_multi_output(provider_info, Y [n, T], initial_params, trainable_mask,
        initial_noise_per_task [T], initial_outputscale, initial_mean_per_task [T],
        num_tasks, max_iterations, learning_rate, task_rank, verbose, num_probes,
        max_cg_iter, cg_tol, precond_rank, precond_method, precond_rebuild_threshold,
        max_tridiag_iter, early_stop_patience, early_stop_tol [, use_cosine_lr,
        fixed_observation_noise [n, T], progress_callback, progress_interval])
        (train_multi_output_python, jit_engine_multi_output_bindings.mojo:57-326)."""
        if len(args) < 21 or len(args) > 25:
            raise ValueError("train_multi_output() expects 21 to 25 positional arguments")
        info = args[0]
        prov = _provider(info)
        T = int(args[7])
        Y = _lib.f32(args[1])
        if Y.ndim != 2 or Y.shape[1] != T:
            raise ValueError("Y must have shape (n, num_tasks)")
        n = Y.shape[0]
        params = _lib.f32(args[2]).ravel()
        mask = np.ascontiguousarray(args[3], dtype=bool).ravel()
        if mask.shape[0] != prov.nparams:
            raise ValueError("train_multi_output() trainable mask length does not match "
                             "provider gradient params")
        if params.shape[0] != prov.nparams:
            raise ValueError("train_multi_output() initial params length does not match "
                             "provider gradient params")
        noise0 = (np.full(T, 0.1, np.float32) if args[4] is None
                  else _lib.f32(args[4]).ravel())
        os0 = float(args[5])
        mean0 = _lib.f32(args[6]).ravel()
        o = _lib.ICMTrainOpts()
        o.max_iterations = int(args[8])
        o.learning_rate = float(args[9])
        o.task_rank = int(args[10])
        o.num_probes = int(args[12])
        o.max_cg_iter = int(args[13])
        o.cg_tol = float(args[14])
        o.precond_rank = int(args[15])
        o.precond_method = int(args[16])
        o.precond_rebuild_threshold = float(args[17])
        o.max_tridiag_iter = int(args[18])
        o.early_stop_patience = int(args[19])
        o.early_stop_tol = float(args[20])
        o.use_cosine_lr = int(bool(args[21])) if len(args) > 21 else 0
        fixed = None
        if len(args) > 22 and args[22] is not None:
            fn = _lib.f32(args[22])
            if fn.shape != (n, T):
                raise ValueError("train_multi_output() fixed observation noise must have "
                                 "shape [n, T]")
            fixed = np.ascontiguousarray(fn.T)
        callback = args[23] if len(args) > 23 else None
        o.progress_interval = int(args[24]) if len(args) > 24 else 1
        if o.max_iterations <= 0:
            raise ValueError("max_iterations must be > 0")
        it_max = o.max_iterations
        out_params = np.zeros(prov.nparams, np.float32)
        noise = np.zeros(T, np.float32)
        mean = np.zeros(T, np.float32)
        B = np.zeros(T * T, np.float32)
        alpha = np.zeros(n * T, np.float32)
        hist = np.zeros(it_max, np.float32)
        cg_hist = np.zeros(it_max, np.int32)
        times = np.zeros(it_max, np.float64)
        res = _lib.ICMTrainResult()
        res.params, res.noise, res.mean = _lib.fptr(out_params), _lib.fptr(noise), _lib.fptr(mean)
        res.B, res.alpha, res.nll_history = _lib.fptr(B), _lib.fptr(alpha), _lib.fptr(hist)
        res.cg_iterations_history = cg_hist.ctypes.data_as(_lib.c_int_p)
        res.iter_times_ms = _lib.dptr(times)
        cfun, keep = _progress_bridge(callback, model="multi_output_icm")
        mask_i = mask.astype(np.int32)
        y_blocked = np.ascontiguousarray(Y.T)
        _lib.call("mgp_icm_train", prov.handle, T, _lib.fptr(y_blocked), _lib.fptr(params),
                  mask_i.ctypes.data_as(_lib.c_int_p), _lib.fptr(noise0), os0, _lib.fptr(mean0),
                  _lib.ofptr(fixed), C.byref(o), cfun, None, C.byref(res))
        del keep
        hl = int(res.history_len)
        prov.params = out_params.copy()
        prov.noise = 0.0
        mode = int(info.get("materialization_mode", 0))
        return {
            "final_nll": float(res.final_nll), "outputscale": float(res.outputscale),
            "iterations": int(res.iterations), "converged": bool(res.converged),
            "num_tasks": T, "task_rank": int(res.task_rank),
            "max_tridiag_iter": o.max_tridiag_iter,
            "precond_rebuild_threshold": float(o.precond_rebuild_threshold),
            "precond_rebuild_count": int(res.precond_rebuild_count),
            "precond_rank": o.precond_rank, "precond_method": o.precond_method,
            "early_stop_patience": o.early_stop_patience,
            "early_stop_tol": float(o.early_stop_tol),
            "use_cosine_lr": bool(o.use_cosine_lr),
            "training_route": "materialized" if mode == 1 else "matrix_free",
            "materialization_mode": mode,
            "noise_mode": "fixed_per_sample_task" if fixed is not None else "per_task",
            "has_observation_noise_vector": fixed is not None,
            "cg_iterations_history": [int(v) for v in cg_hist[:hl]],
            "iter_times_ms": [float(v) for v in times[:hl]],
            "nll_history": [float(v) for v in hist[:hl]],
            "params": [float(v) for v in out_params],
            "noise_per_task": [float(v) for v in noise],
            "mean_per_task": [float(v) for v in mean],
            "B_flat": [float(v) for v in B],
            "alpha": alpha,
        }

    def train_multi_output_mixed(self, *args) -> dict[str, Any]:
        """train_multi_output_mixed(provider_info, Y [n, T], params, noise_per_task [T],
        initial_outputscale, mean_per_task [T], num_tasks, cat_data [n, ncat],
        cat_specs, cat_params (raw), max_iterations, learning_rate, task_rank,
        verbose, num_probes, max_cg_iter, cg_tol, precond_rank, precond_method,
        precond_rebuild_threshold, method_int, max_tridiag_iter,
        early_stop_patience, early_stop_tol [, use_cosine_lr, progress_callback,
        progress_interval]) (train_multi_output_mixed_python,
        jit_engine_multi_output_bindings.mojo:953-1200).  The tree provider
        reads each leaf's levels from its input column (cat_data must match
        it); ``cat_params`` of the result are the best raw values."""
        if len(args) < 24 or len(args) > 27:
            raise ValueError("train_multi_output_mixed() expects 24 to 27 positional arguments")
        info = args[0]
        prov = _provider(info)
        T = int(args[6])
        Y = _lib.f32(args[1])
        if Y.ndim != 2 or Y.shape[1] != T:
            raise ValueError("Y must have shape (n, num_tasks)")
        n = Y.shape[0]
        params = _lib.f32(args[2]).ravel()
        if params.shape[0] != prov.nparams:
            raise ValueError("train_multi_output_mixed() initial params length does not match "
                             "provider gradient params")
        noise0 = _lib.f32(args[3]).ravel()
        os0 = float(args[4])
        mean0 = _lib.f32(args[5]).ravel()
        Cmat = np.asarray(args[7])
        specs = list(args[8])
        if Cmat.ndim != 2 or Cmat.shape != (n, len(specs)):
            raise ValueError("cat_data must have shape (n, number of categorical leaves)")
        kinds = np.array([self._CAT_KIND[str(sp["kernel_type"]).lower()] for sp in specs],
                         np.int32)
        cat0 = _lib.f32(args[9]).ravel()
        o = _lib.ICMTrainOpts()
        o.max_iterations = int(args[10])
        o.learning_rate = float(args[11])
        o.task_rank = int(args[12])
        o.num_probes = int(args[14])
        o.max_cg_iter = int(args[15])
        o.cg_tol = float(args[16])
        o.precond_rank = int(args[17])
        o.precond_method = int(args[18])
        o.precond_rebuild_threshold = float(args[19])
        mode = int(args[20])
        o.max_tridiag_iter = int(args[21])
        o.early_stop_patience = int(args[22])
        o.early_stop_tol = float(args[23])
        o.use_cosine_lr = int(bool(args[24])) if len(args) > 24 else 0
        callback = args[25] if len(args) > 25 else None
        o.progress_interval = int(args[26]) if len(args) > 26 else 1
        if o.max_iterations <= 0:
            raise ValueError("max_iterations must be > 0")
        it_max = o.max_iterations
        out_params = np.zeros(prov.nparams, np.float32)
        noise = np.zeros(T, np.float32)
        mean = np.zeros(T, np.float32)
        B = np.zeros(T * T, np.float32)
        alpha = np.zeros(n * T, np.float32)
        hist = np.zeros(it_max, np.float32)
        cg_hist = np.zeros(it_max, np.int32)
        times = np.zeros(it_max, np.float64)
        cat_out = np.zeros(max(cat0.size, 1), np.float32)
        res = _lib.ICMTrainResult()
        res.params, res.noise, res.mean = _lib.fptr(out_params), _lib.fptr(noise), _lib.fptr(mean)
        res.B, res.alpha, res.nll_history = _lib.fptr(B), _lib.fptr(alpha), _lib.fptr(hist)
        res.cg_iterations_history = cg_hist.ctypes.data_as(_lib.c_int_p)
        res.iter_times_ms = _lib.dptr(times)
        cfun, keep = _progress_bridge(callback, model="multi_output_icm")
        y_blocked = np.ascontiguousarray(Y.T)
        _lib.call("mgp_icm_train_mixed", prov.handle, T, _lib.fptr(y_blocked),
                  _lib.fptr(params), _lib.fptr(noise0), os0, _lib.fptr(mean0),
                  kinds.ctypes.data_as(_lib.c_int_p), int(kinds.size),
                  _lib.fptr(cat0 if cat0.size else cat_out), int(cat0.size), C.byref(o), cfun,
                  None, C.byref(res), _lib.fptr(cat_out))
        del keep
        hl = int(res.history_len)
        prov.params = out_params.copy()
        prov.noise = 0.0
        prov.cat_kinds, prov.cat_raw = kinds, cat_out[:cat0.size].copy()
        return {
            "final_nll": float(res.final_nll), "outputscale": float(res.outputscale),
            "iterations": int(res.iterations), "converged": bool(res.converged),
            "num_tasks": T, "task_rank": int(res.task_rank),
            "max_tridiag_iter": o.max_tridiag_iter,
            "precond_rebuild_threshold": float(o.precond_rebuild_threshold),
            "precond_rebuild_count": int(res.precond_rebuild_count),
            "precond_rank": o.precond_rank, "precond_method": o.precond_method,
            "early_stop_patience": o.early_stop_patience,
            "early_stop_tol": float(o.early_stop_tol),
            "use_cosine_lr": bool(o.use_cosine_lr),
            "training_route": "materialized" if mode == 1 else "matrix_free",
            "materialization_mode": mode,
            "cg_iterations_history": [int(v) for v in cg_hist[:hl]],
            "iter_times_ms": [float(v) for v in times[:hl]],
            "nll_history": [float(v) for v in hist[:hl]],
            "params": [float(v) for v in out_params],
            "cat_params": cat_out[:cat0.size].copy(),
            "noise_per_task": [float(v) for v in noise],
            "mean_per_task": [float(v) for v in mean],
            "B_flat": [float(v) for v in B],
            "alpha": alpha,
        }

    def predict_multi_output(self, *args) -> dict[str, Any]:
        """predict_multi_output(provider_info, alpha_rotated [n, T], Q [T, T],
        effective_scales [T], X_test [m, d], params, noise, variance_method
        [, max_cg_iter, cg_tol, precond_rank, lanczos_rank])
        (predict_multi_output_python, jit_engine_multi_output_bindings.mojo:329-549)."""
        if len(args) < 8 or len(args) > 12:
            raise ValueError("predict_multi_output() expects 8-12 positional arguments")
        info = args[0]
        prov = _provider(info)
        alpha_rot = _lib.f32(args[1])
        if alpha_rot.ndim != 2:
            raise ValueError("alpha_rotated must have shape [n, T]")
        n, T = alpha_rot.shape
        Q = _lib.f32(args[2]).reshape(T, T)
        scales = _lib.f32(args[3]).ravel()
        Xs = _lib.f32(args[4])
        prov.update_params(_lib.f32(args[5]).ravel())
        noise = float(args[6])
        prov.update_noise(noise)
        vm = int(args[7])
        max_cg = int(args[8]) if len(args) > 8 else 100
        tol = float(args[9]) if len(args) > 9 else 1e-2
        prank = int(args[10]) if len(args) > 10 else 10
        lrank = _resolve_lanczos_rank(info, int(args[11]) if len(args) > 11 else 0)
        m = Xs.shape[0]
        mean = np.zeros((m, T), np.float32)
        var = np.zeros((m, T), np.float32) if vm else None
        _lib.call("mgp_icm_predict", prov.handle, T, _lib.fptr(np.ascontiguousarray(alpha_rot.T)),
                  _lib.fptr(Q), _lib.fptr(scales), _lib.fptr(Xs), m, noise, vm, max_cg, tol,
                  prank, lrank, _lib.fptr(mean), _lib.ofptr(var))
        out = {"mean": mean, "lanczos_rank_used": lrank}
        if vm:
            out["variance"] = var
            out["std"] = np.sqrt(var)
        return out

    def sample_multi_output_pathwise(self, *args) -> dict[str, Any]:
        """sample_multi_output_pathwise(provider_info, residual [n, T] (or [S, n, T]),
        B [T, T] (outputscale included), X_test [m, d], params, noise_per_task [T]
        [, max_cg_iter, cg_tol]) (sample_multi_output_pathwise_python,
        jit_engine_multi_output_bindings.mojo:552-712): beta = (B (x) K + D)^-1 r by
        unpreconditioned CG per column, correction = B (x) K(X*, X) beta.  A 3-D
        residual stack is corrected in one batched solve."""
        if len(args) < 6 or len(args) > 8:
            raise ValueError("sample_multi_output_pathwise() expects 6-8 positional arguments")
        info = args[0]
        prov = _provider(info)
        resid = _lib.f32(args[1])
        single = resid.ndim == 2
        if single:
            resid = resid[None]
        S, n, T = resid.shape
        B = _lib.f32(args[2]).reshape(1, T, T)
        Xs = _lib.f32(args[3])
        prov.update_params(_lib.f32(args[4]).ravel())
        prov.update_noise(0.0)
        noise = _lib.f32(args[5]).ravel()
        max_cg = int(args[6]) if len(args) > 6 else 100
        tol = float(args[7]) if len(args) > 7 else 1e-2
        blocked = np.ascontiguousarray(resid.transpose(0, 2, 1))
        m = Xs.shape[0]
        corr = np.zeros((S, m, T), np.float32)
        its = C.c_int(0)
        _lib.call("mgp_lmc_pathwise_correction", _lib.handles([prov]), 1, T, _lib.fptr(B),
                  _lib.fptr(noise), None, _lib.fptr(blocked), S, _lib.fptr(Xs), m, max_cg, tol,
                  _lib.fptr(corr), C.byref(its))
        return {"correction": corr[0] if single else corr, "cg_iterations": int(its.value)}


_ENGINE = Engine()


def load_engine() -> Engine:
    """Counterpart of mojogp.loader.load_engine (loader.py:239-328)."""
    _lib.load()
    return _ENGINE


def load_kernel_module(kind, ard: bool, dim: int, default_dims=None) -> KernelModule:
    """Counterpart of mojogp.loader.load_kernel_module_engine (loader.py:331-429).

    ``kind``: a kind code / name, or a (resolved) KernelNode; nodes other than a
    single RBF / Matern leaf on all inputs get the kernel-tree products."""
    _lib.load()
    from .kernel import KernelNode
    if isinstance(kind, KernelNode):
        if kind.is_native_leaf():
            return KernelModule(kind.native_kind(), kind.ard_dim is not None, dim)
        return KernelModule(None, False, dim, tree_spec=kind.to_tree_spec(dim, default_dims))
    return KernelModule(kind, ard, dim)
