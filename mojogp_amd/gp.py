"""SingleOutputGP — the reference's exact-GP surface over the gfx950 engine.

Follows mojogp/gp.py (fit 860-1552, _fit_continuous 1554-1606, _fit_engine
1608-1883, _predict_engine 1885-2047, predict 2446-2674,
_predict_continuous 2811-2960): the same argument names and defaults, CG
presets, route and preconditioner heuristics, initial-lengthscale caps,
prediction solver budgets and cached-alpha rules.  The hot path runs in
libmojogp_amd.so through ``mojogp_amd._engine``.

Scope: continuous inputs, RBF / Matern-5/2 kernels (isotropic or ARD), scalar
learned noise.  Heteroskedastic noise models, categorical/mixed kernels and
composite kernel trees raise ``NotImplementedError``.
"""

from __future__ import annotations

import json
import warnings
from dataclasses import dataclass
from pathlib import Path
from typing import Any, Optional, Tuple, Union

import numpy as np

from . import _engine
from .kernel import KernelNode, KernelType, cat_default_raw_param, make_ard_kernel

_MODEL_SCHEMA_VERSION = 1
_DEFAULT_PREDICT_LANCZOS_RANK = 100
_DEFAULT_ARD_PREDICT_LANCZOS_RANK = 200
_DEFAULT_EXACT_PREDICT_MAX_CG_ITER = 300
_DEFAULT_EXACT_PREDICT_CG_TOL = 1e-3
_DEFAULT_PREDICT_MAX_CG_ITER = _DEFAULT_EXACT_PREDICT_MAX_CG_ITER
_DEFAULT_PREDICT_CG_TOL = _DEFAULT_EXACT_PREDICT_CG_TOL

_FIT_METHOD_ALIASES = {"mat": "materialized", "mf": "matrix_free"}


def _evaluate_noise_fn(fn, X, expected_n: int, name: str, floor: float) -> np.ndarray:
    """observation_noise_fn(X) -> [n] variances, validated (gp.py:2705-2730)."""
    if not callable(fn):
        raise ValueError(f"{name} must be callable")
    try:
        noise = fn(np.ascontiguousarray(X, dtype=np.float32))
    except Exception as exc:
        raise ValueError(f"{name} failed while evaluating observation noise") from exc
    obs = np.ascontiguousarray(noise, dtype=np.float32)
    if obs.shape != (expected_n,):
        raise ValueError(f"{name} must return shape ({expected_n},), got {obs.shape}")
    if np.any(~np.isfinite(obs)):
        raise ValueError(f"{name} returned NaN or Inf values")
    if np.any(obs < floor):
        raise ValueError(f"{name} values must be >= noise_floor")
    return obs


def normalize_fit_method(method: str, *, allow_auto: bool = False) -> str:
    """Canonical training route name (mojogp/_routes.py:12-28)."""
    if not isinstance(method, str):
        raise ValueError("method must be a string")
    if method in _FIT_METHOD_ALIASES:
        return _FIT_METHOD_ALIASES[method]
    valid = ["materialized", "matrix_free"] + (["auto"] if allow_auto else [])
    if method in valid:
        return method
    aliases = ", ".join(f"'{a}'" for a in sorted(_FIT_METHOD_ALIASES))
    raise ValueError(f"method must be one of {', '.join(repr(v) for v in valid)}; "
                     f"accepted aliases: {aliases}")


def _prediction_lanczos_rank(rank_hint, training_method, is_ard: bool) -> int:
    """gp.py:100-125 (single-output, non-mixed)."""
    rank = int(rank_hint) if rank_hint is not None else 0
    min_rank = _DEFAULT_PREDICT_LANCZOS_RANK
    if is_ard:
        min_rank = max(min_rank, _DEFAULT_ARD_PREDICT_LANCZOS_RANK)
    return max(rank, min_rank)


def _prediction_solver_config(train_info, rank_hint, training_method, *, is_ard,
                              max_cg_iterations=None, cg_tolerance=None, precond_rank=None,
                              max_root_decomposition_size=None) -> dict:
    """gp.py:141-198."""
    train_info = train_info or {}
    resolved_precond_rank = int(precond_rank if precond_rank is not None
                                else train_info.get("precond_rank", 10))
    predict_rank = _prediction_lanczos_rank(rank_hint, training_method, is_ard)
    if max_root_decomposition_size is not None:
        predict_rank = int(max_root_decomposition_size)
    tmax = int(train_info.get("max_cg_iterations",
                              train_info.get("max_cg_iter", _DEFAULT_PREDICT_MAX_CG_ITER)))
    ttol = float(train_info.get("cg_tolerance", train_info.get("cg_tol", _DEFAULT_PREDICT_CG_TOL)))
    return {
        "max_cg_iterations": int(max_cg_iterations if max_cg_iterations is not None
                                 else max(tmax, _DEFAULT_EXACT_PREDICT_MAX_CG_ITER)),
        "cg_tolerance": float(cg_tolerance if cg_tolerance is not None
                              else min(ttol, _DEFAULT_EXACT_PREDICT_CG_TOL)),
        "precond_rank": resolved_precond_rank,
        "max_root_decomposition_size": predict_rank,
    }


@dataclass
class TrainingResult:
    params: np.ndarray
    noise: float
    mean: float
    nll: float
    iterations: int
    converged: bool
    lanczos_root: Optional[np.ndarray]
    lanczos_rank: int
    nll_history: Optional[np.ndarray] = None
    cg_iterations_history: Optional[np.ndarray] = None
    iter_times_ms: Optional[np.ndarray] = None


@dataclass
class MixedTrainingResult(TrainingResult):
    """TrainingResult of a mixed continuous x categorical model: ``params``
    in the public layout (categorical slots at their defaults), ``cat_params``
    the trained raw categorical parameters (gp.py:2405-2418)."""
    cat_params: Optional[np.ndarray] = None


@dataclass
class PredictionResult:
    mean: np.ndarray
    variance: np.ndarray
    std: np.ndarray



# Provider noise modes of the learned per-sample models (fn_ptr_module.py:297-327).
_LEARNED_NOISE_MODES = {"learned_vector": 2, "learned_grouped": 3, "learned_input_dependent": 4}


def _cat_kernel_summary(specs, cat_dims):
    """The reference's cat_kernel config value: one name when every
    categorical leaf uses the same family, else a column -> name map."""
    if not specs:
        return "ehh"
    names = [sp["kernel_type"] for sp in specs]
    if len(set(names)) == 1:
        return names[0]
    return {str(col): nm for col, nm in zip(cat_dims, names)}

def _check_served(kernel: KernelNode, dim: int, default_dims=None) -> None:
    """Raise NotImplementedError for kernels the gfx950 engine does not serve
    (single RBF / Matern leaves run on the tile path, other stationary trees
    and mixed categorical trees on the kernel-tree products)."""
    if kernel.is_native_leaf():
        kernel.native_kind()
    else:
        kernel.to_tree_spec(dim, default_dims)

class SingleOutputGP:
    """Exact Gaussian process regression on one MI355X.

        >>> gp = SingleOutputGP(RBF())
        >>> gp.fit(X, y, max_iterations=50, method="matrix_free")
        >>> mean, std = gp.predict(X_test, return_std=True, variance_method="love")
    """

    _PRECOND_METHOD_MAP = {"greedy": 0, "rpcholesky": 1, "nystrom": 2, "auto": 2}
    _PRESETS = {
        "fast": {"max_cg_iter": 50, "cg_tol": 5e-2, "num_probes": 5, "max_tridiag_iter": 15,
                 "precond_rank": 50, "precond_rebuild_threshold": 0.75, "precond": "greedy"},
        "balanced": {"max_cg_iter": 100, "cg_tol": 1e-2, "num_probes": 10, "max_tridiag_iter": 30,
                     "precond_rank": 100, "precond_rebuild_threshold": 0.5, "precond": "greedy"},
        "accurate": {"max_cg_iter": 200, "cg_tol": 1e-3, "num_probes": 20, "max_tridiag_iter": 60,
                     "precond_rank": 200, "precond_rebuild_threshold": 0.25, "precond": "greedy"},
    }

    def __init__(self, kernel: KernelNode, *, init_mean: Optional[float] = None,
                 verbose: bool = False):
        if not isinstance(kernel, KernelNode):
            raise TypeError("kernel must be a KernelNode instance (e.g. RBF(), Matern52()), "
                            f"got {type(kernel).__name__}")
        self._original_kernel = kernel
        self._kernel_pre_ard = kernel
        self.ard = kernel.has_ard()
        self.kernel = kernel
        self.verbose = verbose
        self._init_mean = init_mean
        self._X_train: Optional[np.ndarray] = None
        self._y_train: Optional[np.ndarray] = None
        self.dim: Optional[int] = None
        self._is_trained = False
        self._training_result: Optional[TrainingResult] = None
        self._training_method: Optional[str] = None
        self._kernel_module: Optional[_engine.KernelModule] = None
        self._engine: Optional[_engine.Engine] = None
        self._module_signature: Optional[tuple] = None
        self._provider_info: Optional[dict] = None
        self._provider_state_current = False
        self._cached_alpha: Optional[np.ndarray] = None
        self._cached_alpha_info: Optional[dict] = None
        self._cached_love_method: Optional[str] = None
        self._engine_predict_mean: Optional[float] = None
        self._fitted_mean: Optional[float] = None
        self._backend_train_info: Optional[dict] = None
        self._backend_predict_info: Optional[dict] = None
        self._backend_sample_info: Optional[dict] = None
        self._prediction_cache_handle: Optional[int] = None
        self._prediction_cache_signature: Optional[tuple] = None
        self._prediction_cache_info: Optional[dict] = None
        self._noise_floor = 1e-6
        self._noise_regularization = 0.0
        self._noise_mode = "scalar"
        self._observation_noise_train: Optional[np.ndarray] = None
        self._noise_group_train: Optional[np.ndarray] = None
        self._noise_group_values: Optional[np.ndarray] = None
        self._observation_noise_fn = None
        self._noise_function_params: Optional[np.ndarray] = None
        # mixed continuous x categorical models
        self.cat_dims: dict = {}
        self._cat_specs: list = []
        self._cont_cols: Optional[list] = None
        self._cat_params_raw: Optional[np.ndarray] = None

    # ------------------------------------------------------------ properties
    @property
    def num_params(self) -> int:
        return self.kernel.num_params()

    @property
    def param_names(self) -> list:
        return self.kernel.get_param_names()

    @property
    def is_trained(self) -> bool:
        return self._is_trained

    @property
    def training_result(self) -> Optional[TrainingResult]:
        return self._training_result

    @property
    def backend_train_info(self) -> Optional[dict]:
        return self._backend_train_info

    @property
    def backend_predict_info(self) -> Optional[dict]:
        return self._backend_predict_info

    @property
    def nll_history(self) -> Optional[np.ndarray]:
        """NLL per training iteration (gp.py:759-764)."""
        if self._training_result is None:
            return None
        return self._training_result.nll_history

    @property
    def backend_sample_info(self) -> Optional[dict]:
        """Sampling-route metadata of the most recent sample_posterior call
        (gp.py:776-779)."""
        return self._backend_sample_info

    def _is_single_kernel_type(self, kt: KernelType) -> bool:
        return self.kernel.operator is None and self.kernel.kernel_type == kt

    def _has_periodic_kernel(self) -> bool:
        """Any periodic leaf in the tree (gp.py:702-716)."""
        def walk(node) -> bool:
            if node is None or not isinstance(node, KernelNode):
                return False
            if node.kernel_type == KernelType.PERIODIC:
                return True
            return walk(node.left) or walk(node.right)
        return walk(self.kernel)

    # ------------------------------------------------------------ lifecycle
    def _current_module_signature(self) -> tuple:
        cont = self._cont_cols if self.kernel.has_categorical() else None
        return (repr(self.kernel.to_dict()), self.dim, None if cont is None else tuple(cont))

    def _ensure_compiled(self) -> None:
        if self._kernel_module is None or self._engine is None:
            cont = self._cont_cols if self.kernel.has_categorical() else None
            self._kernel_module = _engine.load_kernel_module(self.kernel, False, self.dim,
                                                             default_dims=cont)
            self._engine = _engine.load_engine()
            self._module_signature = self._current_module_signature()

    def _resolve_mixed(self, X) -> None:
        """Categorical columns, levels and continuous columns of a mixed kernel
        (analyze_kernel_tree, kernel.py:1118-1166, gp.py:1176-1206); levels
        must be integer codes in [0, L)."""
        leaves = self._kernel_pre_ard.categorical_leaves()
        self.cat_dims, self._cat_specs = {}, []
        for lf in leaves:
            col = int(lf.active_dims[0])
            if col in self.cat_dims:
                raise ValueError(f"input column {col} has more than one categorical kernel")
            self.cat_dims[col] = int(lf.levels)
            self._cat_specs.append({"levels": int(lf.levels),
                                    "kernel_type": lf.kernel_type.name.lower()})
        for col, L in self.cat_dims.items():
            if col >= X.shape[1]:
                raise ValueError(f"categorical column {col} out of range")
            v = X[:, col]
            if np.any(v != np.round(v)) or np.any(v < 0) or np.any(v >= L):
                raise ValueError(f"column {col} must hold integer levels in [0, {L})")
        self._cont_cols = [c for c in range(X.shape[1]) if c not in self.cat_dims]
        if not self._cont_cols:
            raise ValueError("Pure categorical kernels (all dimensions categorical, no "
                             "continuous) are not supported")

    def _set_categorical_tables(self, info) -> None:
        raw = getattr(self, "_cat_params_raw", None)
        if raw is None or not self.kernel.has_categorical():
            return
        kinds = [_engine.Engine._CAT_KIND[s["kernel_type"]] for s in self._cat_specs]
        _engine._provider(info).set_categorical_params(kinds, raw)

    def _destroy_prediction_cache(self) -> None:
        if self._prediction_cache_handle and self._engine is not None:
            try:
                self._engine.destroy_prediction_cache(self._prediction_cache_handle)
            except Exception:
                pass
        self._prediction_cache_handle = None
        self._prediction_cache_signature = None
        self._prediction_cache_info = None

    def _destroy_provider_info(self) -> None:
        self._destroy_prediction_cache()
        destroy = getattr(self._kernel_module, "destroy_provider", None)
        if self._provider_info is not None and destroy is not None:
            destroy(self._provider_info)
        self._provider_info = None
        self._provider_state_current = False

    def __del__(self):  # pragma: no cover - best effort
        try:
            self._destroy_provider_info()
        except Exception:
            pass

    def _build_provider_info(self, X, engine_params, noise, method=None,
                             training: bool = False) -> dict:
        """Provider for training or prediction.  A learned noise mode trains
        with its provider mode (2-4); afterwards, and for prediction, the
        learned training variances are a fixed vector (mode 1)."""
        self._ensure_compiled()
        obs = getattr(self, "_observation_noise_train", None)
        mode = None if obs is None else 1
        groups = ngroups = None
        if training and self._noise_mode in _LEARNED_NOISE_MODES:
            mode = _LEARNED_NOISE_MODES[self._noise_mode]
            if mode == 3:
                groups = self._noise_group_train
                ngroups = int(self._noise_group_values.size)
        # Positional, optional tail only when present (gp.py:470-482).
        provider_args = [np.ascontiguousarray(X, dtype=np.float32),
                         np.ascontiguousarray(engine_params, np.float32), float(noise)]
        if obs is not None:
            provider_args.append(obs)
            if mode is not None:
                provider_args.append(int(mode))
                if groups is not None:
                    provider_args.extend([groups, int(ngroups or 0)])
        info = self._kernel_module.init_provider(*provider_args)
        if not training:
            self._set_categorical_tables(info)
        if (method or self._training_method) == "materialized":
            self._kernel_module.materialize(info)
        return info

    # ------------------------------------------------------------ CG params
    @staticmethod
    def _resolve_cg_params(preset=None, max_cg_iter=None, cg_tol=None, num_probes=None,
                           max_tridiag_iter=None, precond_rank=None,
                           precond_rebuild_threshold=None, precond=None) -> dict:
        """gp.py:821-858."""
        base = dict(SingleOutputGP._PRESETS[preset or "balanced"])
        for key, val in (("max_cg_iter", max_cg_iter), ("cg_tol", cg_tol),
                         ("num_probes", num_probes), ("max_tridiag_iter", max_tridiag_iter),
                         ("precond_rank", precond_rank),
                         ("precond_rebuild_threshold", precond_rebuild_threshold),
                         ("precond", precond)):
            if val is not None:
                base[key] = val
        base.setdefault("precond", "auto")
        base["precond_method"] = SingleOutputGP._PRECOND_METHOD_MAP.get(base["precond"], 2)
        return base

    # ------------------------------------------------------------ fit
    def fit(self, X, y, max_iterations: int = 100, learning_rate: float = 0.01,
            initial_noise: float = 0.1, initial_params=None, method: str = "auto",
            enable_early_stopping: bool = False, early_stop_patience: int = 10,
            early_stop_tol: float = 1e-4, verbose: Optional[bool] = None,
            preset: Optional[str] = None, max_cg_iterations: Optional[int] = None,
            cg_tolerance: Optional[float] = None, num_probes: Optional[int] = None,
            max_tridiag_iterations: Optional[int] = None,
            preconditioner_rank: Optional[int] = None,
            precond_rebuild_threshold: Optional[float] = None,
            use_fused_kernels: bool = True, preconditioner: Optional[str] = None,
            use_preconditioner: Optional[bool] = None, lr_schedule: str = "constant",
            prepare_prediction_cache: bool = False,
            prediction_cache_rank: Optional[int] = None, observation_noise=None,
            observation_noise_fn=None, noise_function=None, learn_noise: bool = True,
            noise_floor: float = 1e-6, noise_regularization: float = 0.01,
            noise_model: str = "scalar", noise_group_train=None, group_noise=None,
            progress: Any = None, progress_stats: Any = None,
            progress_interval: int = 1) -> TrainingResult:
        X = np.ascontiguousarray(X, dtype=np.float32)
        y = np.ascontiguousarray(y, dtype=np.float32)
        if X.ndim != 2:
            raise ValueError(f"X must be 2D, got shape {X.shape}")
        if y.ndim != 1:
            raise ValueError(f"y must be 1D, got shape {y.shape}")
        if X.shape[0] != y.shape[0]:
            raise ValueError(f"X has {X.shape[0]} samples, y has {y.shape[0]}")
        if np.any(~np.isfinite(X)):
            raise ValueError("X contains NaN or Inf values")
        if np.any(~np.isfinite(y)):
            raise ValueError("y contains NaN or Inf values")
        if noise_floor <= 0 or not np.isfinite(noise_floor):
            raise ValueError("noise_floor must be finite and > 0")
        if noise_regularization < 0 or not np.isfinite(noise_regularization):
            raise ValueError("noise_regularization must be finite and >= 0")
        obs_train, noise_mode, groups_arr, gnoise_arr = self._resolve_noise_model(
            X, noise_model, observation_noise, observation_noise_fn, noise_function,
            learn_noise, noise_floor, initial_noise, noise_group_train, group_noise)
        if preset is not None and preset not in self._PRESETS:
            raise ValueError(f"Unknown preset '{preset}'. Must be one of: {list(self._PRESETS)}")
        if max_iterations <= 0:
            raise ValueError(f"max_iterations must be > 0, got {max_iterations}")
        if int(progress_interval) <= 0:
            raise ValueError("progress_interval must be a positive integer")
        if learning_rate <= 0:
            raise ValueError(f"learning_rate must be > 0, got {learning_rate}")
        if initial_noise <= 0:
            raise ValueError(f"initial_noise must be > 0, got {initial_noise}")
        if early_stop_patience < 0:
            raise ValueError(f"early_stop_patience must be >= 0, got {early_stop_patience}")
        if early_stop_tol < 0:
            raise ValueError(f"early_stop_tol must be >= 0, got {early_stop_tol}")
        if prediction_cache_rank is not None and prediction_cache_rank <= 0:
            raise ValueError("prediction_cache_rank must be positive or None")
        if not enable_early_stopping and (early_stop_patience != 10 or early_stop_tol != 1e-4):
            warnings.warn("early_stop_patience and early_stop_tol are set but "
                          "enable_early_stopping=False, so training will run to "
                          "max_iterations.", UserWarning, stacklevel=2)
        if not use_fused_kernels:
            warnings.warn("use_fused_kernels=False has no effect: the JIT engine always uses "
                          "fused GPU kernels.", UserWarning, stacklevel=2)
        if lr_schedule not in ("cosine", "constant"):
            raise ValueError(f"lr_schedule must be 'cosine' or 'constant', got '{lr_schedule}'")
        if preconditioner is not None and preconditioner not in self._PRECOND_METHOD_MAP:
            raise ValueError(f"Unknown preconditioner '{preconditioner}'. Must be one of: "
                             f"{list(self._PRECOND_METHOD_MAP)}")
        use_cosine_lr = lr_schedule == "cosine"

        self._destroy_provider_info()
        self._X_train, self._y_train = X, y
        self._observation_noise_train = obs_train
        self._noise_mode = noise_mode
        self._noise_group_train = groups_arr
        self._noise_group_values = gnoise_arr
        self._observation_noise_fn = observation_noise_fn
        self._noise_function_params = None
        self.dim = X.shape[1]
        self._noise_floor = float(noise_floor)
        self._noise_regularization = float(noise_regularization)
        mixed = self._kernel_pre_ard.has_categorical()
        self._cat_params_raw = None
        if mixed:
            self._resolve_mixed(X)
            if noise_mode != "scalar":
                raise NotImplementedError("mixed categorical models train with scalar noise")
        cont_dim = len(self._cont_cols) if mixed else self.dim
        self.kernel = (make_ard_kernel(self._kernel_pre_ard, cont_dim) if self.ard
                       else self._kernel_pre_ard)
        _check_served(self.kernel, self.dim, self._cont_cols if mixed else None)
        if (self._module_signature is not None
                and self._module_signature != self._current_module_signature()):
            # Another kernel layout or input dimension: reload the modules
            # (modules set by a caller before the first fit are kept, as the
            # reference's engine-plumbing tests inject them).
            self._kernel_module = None
            self._engine = None

        default_initial_params = initial_params is None
        if default_initial_params:
            initial_params = self.kernel.get_initial_params()
        else:
            initial_params = np.asarray(initial_params, dtype=np.float32)
            if initial_params.shape[0] != self.num_params:
                raise ValueError(f"initial_params has {initial_params.shape[0]} values, "
                                 f"expected {self.num_params}")
        # Noise floor for periodic kernels (gp.py:1331-1333).
        if self._has_periodic_kernel() and initial_noise < 0.05:
            initial_noise = max(initial_noise, 0.05)
        _verbose = verbose if verbose is not None else self.verbose

        method = normalize_fit_method(method, allow_auto=True)
        resolved = method
        if method == "auto" and X.shape[0] <= 2000:
            resolved = "materialized"
        elif method == "auto":
            resolved = "matrix_free"
        self._training_method = resolved
        self._ensure_compiled()

        # Initial-lengthscale caps (gp.py:1370-1408).
        if (default_initial_params and resolved == "materialized" and learning_rate <= 0.05
                and self._is_single_kernel_type(KernelType.RBF) and self.dim == 1
                and initial_params.shape[0] >= 1):
            initial_params = initial_params.copy()
            initial_params[0] = min(float(initial_params[0]), 0.5)
        if (default_initial_params and resolved == "matrix_free" and learning_rate <= 0.05
                and self._is_single_kernel_type(KernelType.RBF) and not self.ard
                and 1 < self.dim <= 8 and X.shape[0] >= 10000 and initial_params.shape[0] >= 1):
            initial_params = initial_params.copy()
            initial_params[0] = min(float(initial_params[0]), 0.6)

        # Preconditioner defaults (gp.py:1410-1467).
        resolved_precond = preconditioner
        resolved_precond_rank = preconditioner_rank
        explicit = (preconditioner is not None or preconditioner_rank is not None
                    or use_preconditioner is not None)
        if (resolved_precond is None and resolved == "materialized" and learning_rate <= 0.05
                and self._is_single_kernel_type(KernelType.MATERN32)):
            resolved_precond = "greedy"
        if not explicit and resolved == "materialized" and self._is_single_kernel_type(KernelType.LINEAR):
            resolved_precond_rank = 0
        if not explicit and resolved == "matrix_free":
            if (self._is_single_kernel_type(KernelType.RBF) and not self.ard
                    and 1 < self.dim <= 8 and X.shape[0] >= 5000):
                resolved_precond = "greedy"
                resolved_precond_rank = 256
            else:
                resolved_precond_rank = 0
        resolved_threshold = precond_rebuild_threshold
        if resolved_threshold is None and resolved == "materialized" and self.ard:
            resolved_threshold = 0.1
        cg = self._resolve_cg_params(preset=preset, max_cg_iter=max_cg_iterations,
                                     cg_tol=cg_tolerance, num_probes=num_probes,
                                     max_tridiag_iter=max_tridiag_iterations,
                                     precond_rank=resolved_precond_rank,
                                     precond_rebuild_threshold=resolved_threshold,
                                     precond=resolved_precond)
        init_mean = self._init_mean if self._init_mean is not None else float(np.mean(y))
        if mixed:
            return self._fit_mixed(X, y, initial_params, initial_noise, max_iterations,
                                   learning_rate, resolved, enable_early_stopping,
                                   early_stop_patience, early_stop_tol, _verbose, cg, progress,
                                   progress_interval)
        result = self._fit_engine(X, y, initial_params, initial_noise, max_iterations,
                                  learning_rate, resolved, enable_early_stopping, _verbose, cg,
                                  use_cosine_lr, init_mean, use_preconditioner,
                                  early_stop_patience, early_stop_tol, learn_noise,
                                  progress, progress_interval)
        if prepare_prediction_cache:
            self.prepare_prediction_cache(variance_method="love",
                                          max_root_decomposition_size=prediction_cache_rank)
        return result

    def _fit_mixed(self, X, y, initial_params, initial_noise, max_iterations, learning_rate,
                   route, enable_early_stopping, early_stop_patience, early_stop_tol, verbose,
                   cg, progress, progress_interval) -> MixedTrainingResult:
        """gp.py:2281-2440: continuous kernel on the tree provider, categorical
        tables from default raw parameters, split-Adam training."""
        engine_params = self.kernel.to_engine_params(np.asarray(initial_params, np.float32))
        self._destroy_provider_info()
        self._provider_info = self._build_provider_info(X, engine_params, initial_noise, route,
                                                        training=True)
        self._provider_state_current = True
        leaves = self.kernel.categorical_leaves()
        cat_init = np.concatenate([
            [cat_default_raw_param(lf.kernel_type, i, lf.levels) for i in range(lf.num_params())]
            for lf in leaves]).astype(np.float32)
        Cm = np.stack([X[:, int(lf.active_dims[0])] for lf in leaves], 1).astype(np.int32)
        args = [self._provider_info, y.astype(np.float32), engine_params, float(initial_noise),
                Cm, self._cat_specs, cat_init, max_iterations, float(learning_rate),
                int(cg["num_probes"]), int(cg["max_cg_iter"]), float(cg["cg_tol"]),
                int(cg["precond_rank"]), bool(verbose), 1 if route == "materialized" else 0,
                int(cg["precond_method"]), bool(enable_early_stopping), int(early_stop_patience),
                float(early_stop_tol)]
        if callable(progress):
            args.extend([progress, int(progress_interval)])
        result = self._engine.train_mixed(*args)
        self._is_trained = True
        self._provider_state_current = False
        self._invalidate_prediction_caches()
        self._cat_params_raw = np.asarray(result["cat_params"], np.float32)
        self._fitted_mean = self._engine_predict_mean = float(result["mean"])
        nll_h = np.array(result["nll_history"], np.float32)
        times = np.array(result["iter_times_ms"], np.float64)
        cg_h = np.array(result["cg_iterations_history"], np.int32)
        self._training_result = MixedTrainingResult(
            params=self.kernel.from_engine_params(np.array(result["params"], np.float32)),
            noise=float(result["noise"]), mean=float(result["mean"]), nll=float(result["nll"]),
            iterations=int(result["iterations"]), converged=bool(result["converged"]),
            lanczos_root=None, lanczos_rank=int(cg["max_tridiag_iter"]), nll_history=nll_h,
            cg_iterations_history=cg_h, iter_times_ms=times, cat_params=self._cat_params_raw)
        self._backend_train_info = {
            "training_route": result["training_route"], "is_mixed": True,
            "materialization_mode": int(result["materialization_mode"]),
            "precond_method": int(result["precond_method"]),
            "precond_rank": int(result["precond_rank"]), "noise_mode": "scalar",
            "num_cat_vars": int(result["num_cat_vars"]),
            "total_cat_params": int(result["total_cat_params"]),
            "cat_dims": dict(self.cat_dims),
            "cg_iterations_history": cg_h.tolist(), "iter_times_ms": times.tolist(),
        }
        return self._training_result

    def _resolve_noise_model(self, X, noise_model, observation_noise, observation_noise_fn,
                             noise_function, learn_noise, noise_floor, initial_noise,
                             noise_group_train, group_noise):
        """Noise-model resolution of gp.py:1010-1161.  Returns (initial
        per-point vector or None, resolved mode name, group ids, group values).

        Fixed modes (observation_noise, observation_noise_fn, fixed grouped
        variances) train K + diag(noise_i) with the noise frozen; learned
        modes ('learned_vector', grouped with learn_noise=True,
        'learned_input_dependent' with noise_function='linear') learn the
        per-point variances during fit."""
        if noise_model not in ("scalar", "fixed_vector", "input_dependent", "grouped",
                               "learned_vector", "learned_input_dependent"):
            raise ValueError("noise_model must be one of 'scalar', 'fixed_vector', "
                             "'input_dependent', 'grouped', 'learned_vector', or "
                             "'learned_input_dependent'")
        if noise_function is not None and noise_model != "learned_input_dependent":
            raise ValueError("noise_function is only supported with "
                             "noise_model='learned_input_dependent'")
        if observation_noise_fn is not None and not callable(observation_noise_fn):
            raise ValueError("observation_noise_fn must be callable")
        if observation_noise_fn is not None and observation_noise is not None:
            raise ValueError("Pass either observation_noise or observation_noise_fn, not both")
        if observation_noise_fn is not None and noise_model == "grouped":
            raise ValueError("noise_model='grouped' expands group_noise to observation_noise; "
                             "do not also pass observation_noise_fn")
        if noise_model == "input_dependent" and observation_noise_fn is None:
            raise ValueError("noise_model='input_dependent' requires observation_noise_fn")
        if noise_model == "learned_input_dependent":
            if noise_function != "linear":
                raise ValueError("noise_model='learned_input_dependent' requires "
                                 "noise_function='linear'")
            if observation_noise is not None:
                raise ValueError("noise_model='learned_input_dependent' learns training noise; "
                                 "do not also pass observation_noise")
            if observation_noise_fn is not None:
                raise ValueError("noise_model='learned_input_dependent' learns its own noise "
                                 "function; do not also pass observation_noise_fn")
            if noise_group_train is not None or group_noise is not None:
                raise ValueError("noise_model='learned_input_dependent' does not use grouped "
                                 "noise inputs")
            if not learn_noise:
                raise ValueError("learn_noise must be True for "
                                 "noise_model='learned_input_dependent'")
            if initial_noise <= noise_floor:
                raise ValueError("initial_noise must be greater than noise_floor for learned "
                                 "input-dependent noise")
        if observation_noise is not None and noise_model == "grouped":
            raise ValueError("noise_model='grouped' expands group_noise to observation_noise; "
                             "do not also pass observation_noise")
        if observation_noise_fn is not None:
            if learn_noise:
                raise ValueError("learn_noise must be False when observation_noise_fn is "
                                 "supplied")
            observation_noise = _evaluate_noise_fn(observation_noise_fn, X, X.shape[0],
                                                   "observation_noise_fn", noise_floor)
            noise_model = "fixed_input_dependent"
        if observation_noise is not None and noise_model == "scalar":
            noise_model = "fixed_vector"
        groups_arr = gnoise_arr = None
        if noise_model == "grouped":
            if noise_group_train is None:
                raise ValueError("noise_model='grouped' requires noise_group_train")
            groups_arr = np.ascontiguousarray(noise_group_train, dtype=np.int32)
            if groups_arr.shape != (X.shape[0],):
                raise ValueError(f"noise_group_train must have shape ({X.shape[0]},), got "
                                 f"{groups_arr.shape}")
            if np.any(groups_arr < 0):
                raise ValueError("noise_group_train must contain non-negative group ids")
            max_group = int(groups_arr.max(initial=-1))
            if learn_noise:
                if initial_noise <= noise_floor:
                    raise ValueError("initial_noise must be greater than noise_floor for "
                                     "learned grouped noise")
                gnoise_arr = (np.full(max_group + 1, float(initial_noise), np.float32)
                              if group_noise is None
                              else np.ascontiguousarray(group_noise, dtype=np.float32))
                noise_model = "learned_grouped"
            else:
                if group_noise is None:
                    raise ValueError("noise_model='grouped' requires group_noise when "
                                     "learn_noise=False")
                gnoise_arr = np.ascontiguousarray(group_noise, dtype=np.float32)
                noise_model = "fixed_grouped"
            if gnoise_arr.ndim != 1:
                raise ValueError("group_noise must be a 1D array")
            if gnoise_arr.size == 0:
                raise ValueError("group_noise must contain at least one group variance")
            if np.any(~np.isfinite(gnoise_arr)):
                raise ValueError("group_noise contains NaN or Inf values")
            if np.any(gnoise_arr < noise_floor):
                raise ValueError("group_noise values must be >= noise_floor")
            if max_group >= gnoise_arr.shape[0]:
                raise ValueError("noise_group_train references a group id outside group_noise")
            observation_noise = gnoise_arr[groups_arr]
        elif noise_group_train is not None or group_noise is not None:
            raise ValueError("noise_group_train and group_noise require noise_model='grouped'")
        obs = None
        if noise_model == "learned_vector":
            if observation_noise is not None:
                raise ValueError("noise_model='learned_vector' learns training noise; do not "
                                 "also pass observation_noise")
            if not learn_noise:
                raise ValueError("learn_noise must be True for noise_model='learned_vector'")
            if initial_noise <= noise_floor:
                raise ValueError("initial_noise must be greater than noise_floor for "
                                 "learned_vector noise")
            obs = np.full(X.shape[0], float(initial_noise), np.float32)
        if noise_model == "learned_grouped":
            obs = np.ascontiguousarray(observation_noise, dtype=np.float32)
        if noise_model == "learned_input_dependent":
            obs = np.full(X.shape[0], float(initial_noise), np.float32)
        if observation_noise is None and noise_model == "fixed_vector":
            raise ValueError("noise_model='fixed_vector' requires observation_noise")
        if observation_noise is None and not learn_noise:
            raise NotImplementedError(
                "Fixed scalar noise is not implemented in the JIT training API yet; use "
                "learn_noise=True or provide observation_noise")
        if observation_noise is not None and noise_model != "learned_grouped":
            if learn_noise:
                raise ValueError("learn_noise must be False when observation_noise is supplied")
            obs = np.ascontiguousarray(observation_noise, dtype=np.float32)
            if obs.shape != (X.shape[0],):
                raise ValueError(f"observation_noise must have shape ({X.shape[0]},), got "
                                 f"{obs.shape}")
            if np.any(~np.isfinite(obs)):
                raise ValueError("observation_noise contains NaN or Inf values")
            if np.any(obs < noise_floor):
                raise ValueError("observation_noise values must be >= noise_floor")
        return obs, noise_model, groups_arr, gnoise_arr

    def _evaluate_learned_noise_function(self, X) -> np.ndarray:
        """softplus(w0 + X w) + noise_floor of a learned linear noise function
        (gp.py:2732-2757)."""
        if self._noise_mode != "learned_input_dependent":
            raise ValueError("learned noise function is only available for "
                             "learned_input_dependent models")
        w = self._noise_function_params
        if w is None:
            raise ValueError("learned input-dependent noise parameters are unavailable")
        X = np.ascontiguousarray(X, dtype=np.float32)
        w = np.asarray(w, dtype=np.float32)
        if w.shape != (X.shape[1] + 1,):
            raise ValueError("learned input-dependent noise parameters do not match the model "
                             "input dimension")
        raw = w[0] + X @ w[1:]
        return (np.logaddexp(0.0, raw.astype(np.float64)) + self._noise_floor).astype(np.float32)

    def _observed_noise(self, X, observation_noise, observation_noise_fn, noise_group_test):
        """Test-point noise for target='observed' (gp.py:2611-2650): explicit
        values, a callable, test group ids, or the stored training callable."""
        m = X.shape[0]
        if observation_noise_fn is not None:
            if observation_noise is not None or noise_group_test is not None:
                raise ValueError("Pass only one of observation_noise, observation_noise_fn, "
                                 "or noise_group_test")
            return _evaluate_noise_fn(observation_noise_fn, X, m, "observation_noise_fn",
                                      self._noise_floor)
        if noise_group_test is not None:
            if observation_noise is not None:
                raise ValueError("Pass either observation_noise or noise_group_test, not both")
            if self._noise_group_values is None:
                raise ValueError("noise_group_test requires a model fitted with grouped noise")
            groups = np.ascontiguousarray(noise_group_test, dtype=np.int32)
            if groups.shape != (m,):
                raise ValueError(f"noise_group_test must have shape ({m},), got {groups.shape}")
            if np.any(groups < 0) or int(groups.max(initial=-1)) >= self._noise_group_values.size:
                raise ValueError("noise_group_test references a group id outside group_noise")
            return self._noise_group_values[groups].astype(np.float32)
        if observation_noise is None and self._observation_noise_fn is not None:
            return _evaluate_noise_fn(self._observation_noise_fn, X, m,
                                      "stored observation_noise_fn", self._noise_floor)
        if observation_noise is None and self._noise_mode == "learned_input_dependent":
            return self._evaluate_learned_noise_function(X)
        if observation_noise is None:
            raise ValueError("predict_observed()/predict(target='observed') requires "
                             "observation_noise for test points")
        obs = np.ascontiguousarray(observation_noise, dtype=np.float32)
        if obs.shape != (m,):
            raise ValueError(f"observation_noise must have shape ({m},), got {obs.shape}")
        return obs

    def _fit_engine(self, X, y, initial_params, initial_noise, max_iterations, learning_rate,
                    route, enable_early_stopping, verbose, cg, use_cosine_lr, init_mean,
                    use_preconditioner, early_stop_patience, early_stop_tol, learn_noise,
                    progress, progress_interval) -> TrainingResult:
        """gp.py:1608-1883."""
        engine_params = self.kernel.to_engine_params(np.asarray(initial_params, np.float32))
        self._destroy_provider_info()
        self._provider_info = self._build_provider_info(X, engine_params, initial_noise, route,
                                                        training=True)
        self._provider_state_current = True
        resolved_use_pc = (bool(use_preconditioner) if use_preconditioner is not None
                           else int(cg["precond_rank"]) > 0)
        eff_rank = int(cg["precond_rank"]) if resolved_use_pc else 0
        args = [self._provider_info, y.astype(np.float32), engine_params, float(initial_noise),
                max_iterations, float(learning_rate), cg["num_probes"], cg["max_cg_iter"],
                float(cg["cg_tol"]), eff_rank, verbose, use_cosine_lr, resolved_use_pc,
                cg["max_tridiag_iter"], float(cg["precond_rebuild_threshold"]),
                cg["precond_method"], float(init_mean), bool(enable_early_stopping),
                int(early_stop_patience), float(early_stop_tol), bool(learn_noise),
                float(self._noise_floor), float(self._noise_regularization)]
        callback = progress if callable(progress) else None
        if callback is not None:
            args.extend([callback, int(progress_interval)])
        result = self._engine.train(*args)
        self._is_trained = True
        self._provider_state_current = False
        self._invalidate_prediction_caches()
        learned_mean = float(result.get("mean", init_mean))
        self._engine_predict_mean = learned_mean
        self._fitted_mean = learned_mean
        info = {
            "training_route": route,
            "materialization_mode": int(self._provider_info.get("materialization_mode", 0)),
            "is_ard": bool(self._provider_info.get("is_ard", False)),
            "precond_method": int(result.get("precond_method", cg["precond_method"])),
            "precond_rank": int(result.get("precond_rank", cg["precond_rank"])),
            "max_cg_iter": int(cg["max_cg_iter"]),
            "max_cg_iterations": int(cg["max_cg_iter"]),
            "cg_tol": float(cg["cg_tol"]),
            "cg_tolerance": float(cg["cg_tol"]),
            "max_tridiag_iter": int(cg["max_tridiag_iter"]),
            "precond_rebuild_threshold": float(cg["precond_rebuild_threshold"]),
            "enable_early_stopping": bool(enable_early_stopping),
            "early_stop_patience": int(early_stop_patience),
            "early_stop_tol": float(early_stop_tol),
            "use_preconditioner": bool(resolved_use_pc),
            "noise_mode": self._noise_mode,
            "learn_noise": bool(learn_noise),
            "has_observation_noise_vector": self._observation_noise_train is not None,
            "noise_regularization": float(self._noise_regularization),
        }
        for key in ("actual_precond_rank", "precond_build_count", "precond_rebuild_count",
                    "precond_build_total_ms", "precond_rank_history", "precond_rebuild_steps"):
            if key in result:
                info[key] = result[key]
        params = self.kernel.from_engine_params(np.array(result["params"], dtype=np.float32))
        nll_h = np.array(result.get("nll_history", []), dtype=np.float32)
        times = np.array(result.get("iter_times_ms", []), dtype=np.float32)
        cg_h = np.array(result.get("cg_iterations_history", []), dtype=np.int32)
        self._training_result = TrainingResult(
            params=params, noise=float(result["noise"]), mean=learned_mean,
            nll=float(result["final_nll"]), iterations=int(result["iterations"]),
            converged=bool(result["converged"]), lanczos_root=None,
            lanczos_rank=int(cg["max_tridiag_iter"]), nll_history=nll_h,
            cg_iterations_history=cg_h, iter_times_ms=times)
        learned = result.get("learned_observation_noise")
        if learned is not None:
            # gp.py:1809-1838: the learned variances become the training noise
            # vector; grouped models keep per-group means, linear ones the
            # function weights.
            self._observation_noise_train = np.ascontiguousarray(learned, dtype=np.float32)
            info["has_observation_noise_vector"] = True
            info["learned_observation_noise_min"] = float(np.min(learned))
            info["learned_observation_noise_max"] = float(np.max(learned))
            info["learned_observation_noise_mean"] = float(np.mean(learned))
            if self._noise_mode == "learned_grouped" and self._noise_group_train is not None:
                gv = np.zeros(int(np.max(self._noise_group_train)) + 1, dtype=np.float32)
                for gid in range(gv.size):
                    mask = self._noise_group_train == gid
                    if np.any(mask):
                        gv[gid] = float(np.mean(self._observation_noise_train[mask]))
                self._noise_group_values = gv
                info["learned_group_noise"] = gv.tolist()
        fnp = result.get("learned_noise_function_params")
        if fnp is not None:
            self._noise_function_params = np.ascontiguousarray(fnp, dtype=np.float32)
            info["learned_noise_function"] = "linear"
            info["learned_noise_function_params"] = self._noise_function_params.tolist()
        if (result.get("cached_alpha") is not None
                and self._noise_mode not in _LEARNED_NOISE_MODES):
            self._store_cached_alpha(result["cached_alpha"],
                                     {"max_cg_iterations": int(cg["max_cg_iter"]),
                                      "cg_tolerance": float(cg["cg_tol"]),
                                      "precond_rank": int(cg["precond_rank"])}, "training")
        if len(times):
            info["iter_times_ms"] = times.tolist()
            info["iter_time_median_ms"] = float(np.median(times))
            info["iter_time_p5_ms"] = float(np.percentile(times, 5))
            info["iter_time_p95_ms"] = float(np.percentile(times, 95))
        if len(cg_h):
            info["cg_iterations_history"] = cg_h.tolist()
            info["cg_iterations_total"] = int(cg_h.sum())
            info["cg_iterations_mean"] = float(cg_h.mean())
            info["cg_iterations_max"] = int(cg_h.max())
            info["cg_iterations_final_step"] = int(cg_h[-1])
            info["cg_iterations_measured"] = True
        self._backend_train_info = info
        return self._training_result

    # ------------------------------------------------------------ alpha cache
    def _invalidate_prediction_caches(self) -> None:
        self._cached_alpha = None
        self._cached_alpha_info = None
        self._cached_love_method = None
        self._destroy_prediction_cache()

    def _store_cached_alpha(self, alpha, solver_config, source) -> None:
        self._cached_alpha = np.asarray(alpha, dtype=np.float32)
        self._cached_alpha_info = {"source": source,
                                   "max_cg_iterations": int(solver_config["max_cg_iterations"]),
                                   "cg_tolerance": float(solver_config["cg_tolerance"]),
                                   "precond_rank": int(solver_config["precond_rank"])}

    def _cached_alpha_for_solver(self, solver_config) -> Optional[np.ndarray]:
        """gp.py:2103-2122: reuse only an alpha solved at least as tightly."""
        a = self._cached_alpha
        if a is None or self._y_train is None or len(a) != len(self._y_train):
            return None
        info = self._cached_alpha_info or {}
        if (int(info.get("max_cg_iterations", 0) or 0) < int(solver_config["max_cg_iterations"])
                or float(info.get("cg_tolerance", float("inf"))) > float(solver_config["cg_tolerance"])):
            return None
        return a

    # ------------------------------------------------------------ predict
    def _solver_config(self, max_cg_iterations=None, cg_tolerance=None, preconditioner_rank=None,
                       max_root_decomposition_size=None) -> dict:
        tr = self._training_result
        return _prediction_solver_config(
            self._backend_train_info, getattr(tr, "lanczos_rank", 0), self._training_method,
            is_ard=self.ard, max_cg_iterations=max_cg_iterations, cg_tolerance=cg_tolerance,
            precond_rank=preconditioner_rank,
            max_root_decomposition_size=max_root_decomposition_size)

    def _provider_for_prediction(self, params, noise):
        """Reuse the training provider (its state is re-uploaded unless current)."""
        if self._provider_info is None:
            self._provider_info = self._build_provider_info(self._X_train, params, noise)
            self._provider_state_current = True
        return self._provider_info

    def predict(self, X, return_var: bool = False, return_std: bool = False,
                variance_method: str = "love", method: Optional[str] = None,
                target: str = "latent", observation_noise=None, observation_noise_fn=None,
                noise_group_test=None, *, max_cg_iterations: Optional[int] = None,
                cg_tolerance: Optional[float] = None, preconditioner_rank: Optional[int] = None,
                max_root_decomposition_size: Optional[int] = None,
                exact_prediction_block_cols: Optional[int] = None, progress: Any = None,
                progress_stats: Any = None) -> Union[PredictionResult, Tuple[np.ndarray, np.ndarray]]:
        if not self._is_trained:
            raise RuntimeError("GP must be trained before prediction. Call fit() first.")
        if return_var and return_std:
            raise ValueError("Only one of return_var or return_std may be True.")
        if variance_method not in ("love", "exact", "mean_only"):
            raise ValueError("variance_method must be one of ('love', 'exact', 'mean_only'), "
                             f"got '{variance_method}'")
        if method not in (None, "materialized", "matrix_free"):
            raise ValueError("method must be one of None, 'materialized', or 'matrix_free', "
                             f"got '{method}'")
        if target not in ("latent", "observed"):
            raise ValueError("target must be 'latent' or 'observed'")
        if exact_prediction_block_cols is not None and exact_prediction_block_cols <= 0:
            raise ValueError("exact_prediction_block_cols must be positive or None")
        X = np.asarray(X, dtype=np.float32)
        if X.ndim != 2:
            raise ValueError(f"X must be 2D, got shape {X.shape}")
        if X.shape[1] != self.dim:
            raise ValueError(f"X has {X.shape[1]} features, expected {self.dim}")
        if np.any(~np.isfinite(X)):
            raise ValueError("X_test contains NaN or Inf values")
        obs_test = (self._observed_noise(X, observation_noise, observation_noise_fn,
                                         noise_group_test) if target == "observed" else None)

        tr = self._training_result
        params = self.kernel.to_engine_params(np.array(tr.params, dtype=np.float32))
        sc = self._solver_config(max_cg_iterations, cg_tolerance, preconditioner_rank,
                                 max_root_decomposition_size)
        vm = {"exact": 2, "love": 1, "mean_only": 0}[variance_method]
        prediction_method = method or self._training_method or "matrix_free"
        info = self._provider_for_prediction(params, tr.noise)
        mean_value = float(self._engine_predict_mean if self._engine_predict_mean is not None
                           else tr.mean)
        if self._prediction_cache_valid(prediction_method, variance_method, sc, params,
                                        float(tr.noise), mean_value):
            res = self._engine.predict_with_cache(info, int(self._prediction_cache_handle),
                                                  X.astype(np.float32), params, float(tr.noise),
                                                  mean_value, vm)
        else:
            cached_alpha = self._cached_alpha_for_solver(sc)
            root = None
            if variance_method == "love" and tr.lanczos_root is not None \
                    and self._cached_love_method == prediction_method \
                    and len(tr.lanczos_root) == len(self._y_train) * int(sc["max_root_decomposition_size"]):
                root = np.ascontiguousarray(tr.lanczos_root, dtype=np.float32)
            args = [info, self._y_train.astype(np.float32), X.astype(np.float32), params,
                    float(tr.noise), mean_value, vm, int(sc["max_cg_iterations"]),
                    float(sc["cg_tolerance"]), int(sc["precond_rank"]),
                    int(sc["max_root_decomposition_size"]), bool(self._provider_state_current),
                    int(exact_prediction_block_cols or 0)]
            if cached_alpha is not None:
                args.append(np.ascontiguousarray(cached_alpha, dtype=np.float32))
                if root is not None:
                    args.append(root)
            res = self._engine.predict(*args)
            if res.get("cached_alpha") is not None:
                self._store_cached_alpha(res["cached_alpha"], sc, "prediction")
            if res.get("cached_lanczos_root") is not None:
                tr.lanczos_root = np.asarray(res["cached_lanczos_root"], dtype=np.float32)
                self._cached_love_method = prediction_method
        self._provider_state_current = True
        mean = np.asarray(res["mean"], dtype=np.float32)
        variance = np.asarray(res.get("variance", np.zeros(len(X))), dtype=np.float32)
        self._backend_predict_info = {
            "prediction_method": prediction_method,
            "variance_method": variance_method,
            "precond_rank": int(sc["precond_rank"]),
            "max_cg_iterations": int(sc["max_cg_iterations"]),
            "cg_tolerance": float(sc["cg_tolerance"]),
            "max_root_decomposition_size": int(sc["max_root_decomposition_size"]),
            "prediction_total_time_s": float(res.get("total_time_s", 0.0)),
            "prediction_alpha_time_s": float(res.get("alpha_time_s", 0.0)),
            "prediction_mean_time_s": float(res.get("mean_time_s", 0.0)),
            "prediction_variance_time_s": float(res.get("variance_time_s", 0.0)),
            "prediction_love_root_time_s": float(res.get("love_root_time_s", 0.0)),
            "alpha_cache_used": bool(res.get("alpha_cache_used", False)),
            "love_root_cache_used": bool(res.get("love_root_cache_used", False)),
            "alpha_cg_iterations": int(res.get("alpha_cg_iterations", 0)),
        }
        self._backend_predict_info.update(
            {k: v for k, v in res.items() if k.startswith("exact_")})
        if target == "observed":
            variance = variance + obs_test
        std = np.sqrt(np.maximum(variance, 0))
        if return_var:
            return mean, variance
        if return_std:
            return mean, std
        return PredictionResult(mean=mean, variance=variance, std=std)

    def predict_observed(self, X, observation_noise=None, *, observation_noise_fn=None,
                         noise_group_test=None, **kwargs):
        """p(y_test | y_train): test-time noise is explicit (gp.py:2681-2703)."""
        kwargs.pop("target", None)
        return self.predict(X, target="observed", observation_noise=observation_noise,
                            observation_noise_fn=observation_noise_fn,
                            noise_group_test=noise_group_test, **kwargs)

    def predict_latent(self, X, **kwargs):
        """p(f_test | y_train)."""
        kwargs.pop("target", None)
        return self.predict(X, target="latent", **kwargs)

    # ------------------------------------------------------------ scoring
    def score(self, X_test, y_test) -> float:
        """R^2 of the predictive mean on test data (gp.py:3059-3070)."""
        if not self._is_trained:
            raise RuntimeError("Model must be trained before scoring")
        X_test = np.asarray(X_test, dtype=np.float32)
        y_test = np.asarray(y_test, dtype=np.float32)
        mean, _ = self.predict(X_test, return_std=True)
        ss_res = np.sum((y_test - mean) ** 2)
        ss_tot = np.sum((y_test - np.mean(y_test)) ** 2)
        if ss_tot == 0:
            return 0.0
        return float(1.0 - ss_res / ss_tot)

    def get_learned_params(self) -> dict:
        """Learned parameters by name, plus noise (and the learned noise state
        of noise modes 2-4) and mean (gp.py:3072-3099)."""
        if not self._is_trained:
            raise RuntimeError("Model must be trained before getting params")
        tr = self._training_result
        params = {}
        for i, name in enumerate(self.kernel.get_param_names()):
            if i < len(tr.params):
                params[name] = float(tr.params[i])
        params["noise"] = float(tr.noise)
        obs = self._observation_noise_train
        if self._noise_mode == "learned_vector" and obs is not None:
            params["observation_noise_train"] = np.asarray(obs, dtype=np.float32).copy()
        if self._noise_mode == "learned_grouped" and self._noise_group_values is not None:
            params["group_noise"] = np.asarray(self._noise_group_values, dtype=np.float32).copy()
        if self._noise_mode == "learned_input_dependent" and self._noise_function_params is not None:
            params["noise_function"] = "linear"
            params["noise_function_params"] = np.asarray(self._noise_function_params,
                                                         dtype=np.float32).copy()
            if obs is not None:
                params["observation_noise_train"] = np.asarray(obs, dtype=np.float32).copy()
        params["mean"] = float(tr.mean)
        return params

    def log_marginal_likelihood(self) -> float:
        """Log marginal likelihood at the learned hyperparameters: -NLL of the
        training result (gp.py:3642-3646)."""
        if not self._is_trained:
            raise RuntimeError("GP must be trained first.")
        return -float(self._training_result.nll)

    # ------------------------------------------------------------ sampling
    def sample_posterior(self, X_test, n_samples: int = 1, method: str = "diagonal",
                         n_rff_features: int = 1024,
                         rng: Optional[np.random.Generator] = None) -> np.ndarray:
        """Posterior samples [n_samples, m] (gp.py:3101-3196).

        'diagonal': independent draws mean + std z from the predictive std.
        'pathwise': Matheron's rule -- an RFF prior draw (device features,
        pathwise_prior.py) corrected by the engine's solve against the residual
        y - mu - (f_prior(X) + sqrt(noise) eps) (gp.py:3266-3433), for single
        RBF / Matern kernels."""
        if not self._is_trained:
            raise RuntimeError("GP must be trained before sampling.")
        if method not in ("diagonal", "pathwise"):
            raise ValueError(f"method must be 'diagonal' or 'pathwise', got '{method}'")
        if rng is None:
            rng = np.random.default_rng()
        training_route = (self._backend_train_info or {}).get(
            "training_route", self._training_method or "matrix_free")
        if method == "pathwise":
            samples = self._sample_posterior_pathwise(X_test, int(n_samples),
                                                      int(n_rff_features), rng)
            self._backend_sample_info = {
                "requested_method": method,
                "actual_sampling_method": "pathwise",
                "actual_sampling_route": "provider_pathwise",
                "backend_sampling_used": True,
                "backend_correction_used": True,
                "backend_correction_route": "predict",
                "training_route": training_route,
                "prior_sampler_family": "shared_feature_map",
                "n_rff_features": int(n_rff_features),
            }
            return samples
        pred = self.predict(X_test)
        z = rng.standard_normal((int(n_samples), len(pred.mean)))
        samples = pred.mean[np.newaxis, :] + pred.std[np.newaxis, :] * z
        self._backend_sample_info = {
            "requested_method": method,
            "actual_sampling_method": "diagonal",
            "actual_sampling_route": "diagonal_from_predictive_std",
            "backend_sampling_used": True,
            "backend_correction_used": False,
            "training_route": training_route,
        }
        return samples.astype(np.float32)

    _PATHWISE_TEST_CHUNK = 512   # test points per correction call (gp.py:84)

    def _sample_posterior_pathwise(self, X_test, n_samples: int, n_rff_features: int,
                                   rng: np.random.Generator) -> np.ndarray:
        """Per sample: weights w ~ N(0, I_F); prior at the training points plus
        sqrt(noise) eps; residual r = (y - mu) - that; per test chunk the
        engine's mean-only prediction against r (max_cg 100, tol 1e-2,
        rank-10 preconditioner, as the reference passes) gives K* (K + s^2 I)^-1 r,
        and the sample is mu + f_prior(X*) + that correction.  The Generator
        is drawn in the reference's order (features, then per sample weights
        and the noise vector), so a seeded run draws the same prior."""
        from .pathwise_prior import (build_feature_weights, build_pathwise_feature_map,
                                     sample_prior_values)
        kt = self.kernel.kernel_type if self.kernel.operator is None else None
        if kt not in (KernelType.RBF, KernelType.MATERN12, KernelType.MATERN32,
                      KernelType.MATERN52) or self.kernel.active_dims is not None \
                or self._cat_specs:
            raise NotImplementedError(
                "pathwise sampling is served for single RBF / Matern kernels; use "
                "method='diagonal' for kernel trees and mixed kernels")
        X_test = np.ascontiguousarray(X_test, dtype=np.float32)
        if X_test.ndim != 2 or X_test.shape[1] != self.dim:
            raise ValueError(f"X_test must have shape (m, {self.dim})")
        tr = self._training_result
        noise = float(tr.noise)
        mean_val = float(tr.mean)
        y_centered = self._y_train.astype(np.float32) - np.float32(mean_val)
        public = np.ascontiguousarray(tr.params, dtype=np.float32)
        params = self.kernel.to_engine_params(public)
        kind = {KernelType.RBF: 0, KernelType.MATERN52: 1, KernelType.MATERN12: 2,
                KernelType.MATERN32: 3}[kt]
        fmap = build_pathwise_feature_map(kind, public, input_dim=self.dim,
                                          n_features=n_rff_features, rng=rng,
                                          ard=self.kernel.ard_dim is not None)
        n, m = self._X_train.shape[0], X_test.shape[0]
        samples = np.empty((n_samples, m), dtype=np.float32)
        noise_scale = np.float32(np.sqrt(max(noise, 0.0)))
        rank = _prediction_lanczos_rank(getattr(tr, "lanczos_rank", 0), self._training_method,
                                        self.ard)
        info = self._provider_for_prediction(params, noise)
        chunk = min(self._PATHWISE_TEST_CHUNK, max(m, 1))
        for s_i in range(n_samples):
            w = build_feature_weights(fmap, 1, rng)
            prior_train = sample_prior_values(fmap, self._X_train, w)[0]
            obs_prior = prior_train + noise_scale * rng.standard_normal(n).astype(np.float32)
            residual = np.ascontiguousarray(y_centered - obs_prior, dtype=np.float32)
            alpha = None
            for start in range(0, m, chunk):
                Xc = np.ascontiguousarray(X_test[start:start + chunk])
                prior_chunk = sample_prior_values(fmap, Xc, w)[0]
                args = [info, residual, Xc, params, noise, 0.0, 0, 100, 1e-2, 10, rank,
                        bool(self._provider_state_current), 0]
                if alpha is not None:     # one solve per sample, reused by every chunk
                    args.append(alpha)
                res = self._engine.predict(*args)
                self._provider_state_current = True
                if alpha is None and res.get("cached_alpha") is not None:
                    alpha = np.ascontiguousarray(res["cached_alpha"], dtype=np.float32)
                correction = np.asarray(res["mean"], dtype=np.float32)
                samples[s_i, start:start + chunk] = np.float32(mean_val) + prior_chunk + correction
        return samples

    # ------------------------------------------------------------ cache
    def _cache_signature(self, prediction_method, variance_method, sc, params, noise, mean):
        return (prediction_method, variance_method, len(self._y_train), int(self.dim or 0),
                int(sc["max_cg_iterations"]), float(sc["cg_tolerance"]), int(sc["precond_rank"]),
                int(sc["max_root_decomposition_size"]),
                tuple(np.asarray(params, np.float32).ravel().tolist()), float(noise), "scalar",
                None, float(mean))

    def _prediction_cache_valid(self, prediction_method, variance_method, sc, params, noise,
                                mean) -> bool:
        if not self._prediction_cache_handle:
            return False
        want = self._cache_signature(prediction_method, variance_method, sc, params, noise, mean)
        return self._prediction_cache_signature == want

    def prepare_prediction_cache(self, variance_method: str = "love", method: Optional[str] = None,
                                 *, max_cg_iterations: Optional[int] = None,
                                 cg_tolerance: Optional[float] = None,
                                 preconditioner_rank: Optional[int] = None,
                                 max_root_decomposition_size: Optional[int] = None) -> dict:
        """Device-resident alpha (+ LOVE root) for repeated predictions (gp.py:2134-2279)."""
        if not self._is_trained:
            raise RuntimeError("GP must be trained before preparing a prediction cache.")
        if variance_method not in ("love", "mean_only"):
            raise ValueError("prediction cache supports variance_method 'love' or 'mean_only'")
        tr = self._training_result
        params = self.kernel.to_engine_params(np.array(tr.params, dtype=np.float32))
        sc = self._solver_config(max_cg_iterations, cg_tolerance, preconditioner_rank,
                                 max_root_decomposition_size)
        vm = 1 if variance_method == "love" else 0
        prediction_method = method or self._training_method or "matrix_free"
        info = self._provider_for_prediction(params, tr.noise)
        mean_value = float(self._engine_predict_mean if self._engine_predict_mean is not None
                           else tr.mean)
        self._destroy_prediction_cache()
        args = [info, self._y_train.astype(np.float32), params, float(tr.noise), mean_value, vm,
                int(sc["max_cg_iterations"]), float(sc["cg_tolerance"]), int(sc["precond_rank"]),
                int(sc["max_root_decomposition_size"]), bool(self._provider_state_current)]
        cached_alpha = self._cached_alpha_for_solver(sc)
        if cached_alpha is not None:
            args.append(cached_alpha)
        res = self._engine.prepare_prediction_cache(*args)
        self._provider_state_current = True
        self._prediction_cache_handle = int(res["cache_handle"])
        self._prediction_cache_signature = self._cache_signature(
            prediction_method, variance_method, sc, params, float(tr.noise), mean_value)
        self._prediction_cache_info = {"prediction_cache_handle": self._prediction_cache_handle,
                                       "prediction_cache_rank": int(res["lanczos_rank"]) if vm else 0,
                                       "prediction_cache_has_love_root": bool(vm)}
        return dict(self._prediction_cache_info)

    # ------------------------------------------------------------ persistence
    def save(self, path) -> None:
        """``<path>_config.json`` + ``<path>_arrays.npz`` in the reference's
        schema v1 (gp.py:3648-3733): same config keys and array names, so
        models round-trip with files the reference writes and reads."""
        if not self._is_trained:
            raise RuntimeError("GP must be trained before saving.")
        from . import __version__
        path = str(path)
        if path.endswith(".json") or path.endswith(".npz"):
            path = path.rsplit(".", 1)[0]
        tr = self._training_result
        cfg = {
            "schema_version": _MODEL_SCHEMA_VERSION, "mojogp_version": __version__,
            "wrapper": "SingleOutputGP", "dim": int(self.dim), "ard": bool(self.ard),
            "verbose": bool(self.verbose),
            "cat_dims": {str(k): int(v) for k, v in self.cat_dims.items()},
            "cat_kernel": _cat_kernel_summary(self._cat_specs, self.cat_dims),
            "kernel_mojo_type": self.kernel.to_mojo_type(),
            "kernel_tree": self._original_kernel.to_dict(), "is_mixed": bool(self.cat_dims),
            "training_method": self._training_method,
            "engine_mean": self._engine_predict_mean,
            "backend_train_info": self._backend_train_info,
            "cached_love_method": self._cached_love_method, "noise_mode": self._noise_mode,
            "noise_floor": float(self._noise_floor),
            "noise_regularization": float(self._noise_regularization),
            "noise_function": ("linear" if self._noise_mode == "learned_input_dependent"
                               else None),
            "provider_noise_mode_int": (
                _LEARNED_NOISE_MODES.get(self._noise_mode, 1)
                if self._observation_noise_train is not None else None),
            "has_observation_noise_train": self._observation_noise_train is not None,
            "has_observation_noise_fn": self._observation_noise_fn is not None,
            "has_noise_group_train": self._noise_group_train is not None,
            "has_group_noise": self._noise_group_values is not None,
            "result_type": ("MixedTrainingResult" if isinstance(tr, MixedTrainingResult)
                            else "TrainingResult"),
            "noise": float(tr.noise), "mean": float(tr.mean),
            "nll": float(tr.nll), "iterations": int(tr.iterations),
            "converged": bool(tr.converged), "lanczos_rank": int(tr.lanczos_rank),
        }
        Path(path + "_config.json").write_text(json.dumps(cfg, indent=2, default=float))
        arrays = {"X_train": self._X_train, "y_train": self._y_train,
                  "params": np.asarray(tr.params, np.float32)}
        if self._observation_noise_train is not None:
            arrays["observation_noise_train"] = self._observation_noise_train
        if self._noise_group_train is not None:
            arrays["noise_group_train"] = self._noise_group_train
        if self._noise_function_params is not None:
            arrays["noise_function_params"] = self._noise_function_params
        if self._noise_group_values is not None:
            arrays["group_noise"] = self._noise_group_values
        if self._cat_params_raw is not None:
            arrays["cat_params"] = self._cat_params_raw
        np.savez(path + "_arrays.npz", **arrays)

    @classmethod
    def load(cls, path, kernel: Optional[KernelNode] = None) -> "SingleOutputGP":
        """Load a model saved by :meth:`save` or by the reference's
        ``SingleOutputGP.save`` (gp.py:3735-3911) for the continuous, scalar-noise
        models this engine serves."""
        path = str(path)
        if path.endswith(".json") or path.endswith(".npz"):
            path = path.rsplit(".", 1)[0]
        cfg = json.loads(Path(path + "_config.json").read_text())
        if cfg.get("wrapper") != "SingleOutputGP":
            raise ValueError("Saved model is not a SingleOutputGP artifact. Expected "
                             f"wrapper='SingleOutputGP', got {cfg.get('wrapper')!r}.")
        if int(cfg.get("schema_version", 0)) != _MODEL_SCHEMA_VERSION:
            raise ValueError(f"Unsupported SingleOutputGP schema_version="
                             f"{cfg.get('schema_version')}; expected {_MODEL_SCHEMA_VERSION}.")
        if cfg.get("result_type", "TrainingResult") not in ("TrainingResult",
                                                            "MixedTrainingResult"):
            raise ValueError(f"unknown result_type {cfg.get('result_type')!r}")
        mode = cfg.get("noise_mode", "scalar")
        if mode not in ("scalar", "fixed_vector", "fixed_input_dependent", "fixed_grouped",
                        *_LEARNED_NOISE_MODES):
            raise ValueError(f"unknown noise_mode {mode!r} in the artifact")
        arr = np.load(path + "_arrays.npz", allow_pickle=False)
        if mode != "scalar" and "observation_noise_train" not in arr:
            raise ValueError("artifact with fixed per-sample noise lacks observation_noise_train")
        if kernel is None:
            if "kernel_tree" not in cfg:
                raise ValueError("SingleOutputGP artifact is missing required kernel_tree.")
            kernel = KernelNode.from_dict(cfg["kernel_tree"])
        gp = cls(kernel, init_mean=cfg.get("init_mean"), verbose=cfg.get("verbose", False))
        gp._X_train = np.ascontiguousarray(arr["X_train"], np.float32)
        gp._y_train = np.ascontiguousarray(arr["y_train"], np.float32)
        gp.dim = int(gp._X_train.shape[1])
        if gp._kernel_pre_ard.has_categorical():
            gp._resolve_mixed(gp._X_train)
            gp._cat_params_raw = np.ascontiguousarray(arr["cat_params"], np.float32)
        cont_dim = len(gp._cont_cols) if gp.cat_dims else gp.dim
        gp.kernel = (make_ard_kernel(gp._kernel_pre_ard, cont_dim) if gp.ard
                     else gp._kernel_pre_ard)
        gp._training_method = cfg.get("training_method") or "matrix_free"
        gp._backend_train_info = cfg.get("backend_train_info") or {}
        gp._cached_love_method = cfg.get("cached_love_method")
        gp._noise_floor = float(cfg.get("noise_floor", 1e-6))
        gp._noise_regularization = float(cfg.get("noise_regularization", 0.0))
        gp._noise_mode = mode
        if "noise_function_params" in arr:
            gp._noise_function_params = np.ascontiguousarray(arr["noise_function_params"],
                                                             np.float32)
        if "observation_noise_train" in arr:
            gp._observation_noise_train = np.ascontiguousarray(arr["observation_noise_train"],
                                                               np.float32)
        if "noise_group_train" in arr:
            gp._noise_group_train = np.ascontiguousarray(arr["noise_group_train"], np.int32)
        if "group_noise" in arr:
            gp._noise_group_values = np.ascontiguousarray(arr["group_noise"], np.float32)
        gp._training_result = TrainingResult(
            params=np.asarray(arr["params"], np.float32), noise=float(cfg["noise"]),
            mean=float(cfg.get("mean", 0.0)), nll=float(cfg["nll"]),
            iterations=int(cfg["iterations"]), converged=bool(cfg["converged"]),
            lanczos_root=None, lanczos_rank=int(cfg["lanczos_rank"]))
        if gp._cat_params_raw is not None:
            tr0 = gp._training_result
            gp._training_result = MixedTrainingResult(**{**tr0.__dict__,
                                                         "cat_params": gp._cat_params_raw})
        engine_mean = cfg.get("engine_mean")
        gp._engine_predict_mean = float(engine_mean if engine_mean is not None
                                        else gp._training_result.mean)
        gp._fitted_mean = gp._training_result.mean
        gp._is_trained = True
        gp._ensure_compiled()
        return gp
