"""MultiOutputLMCGP — the reference's LMC multi-output surface over the gfx950 engine.

Follows mojogp/multi_output_gp.py: constructor 3534-3660, fit 4561-4820 /
_fit_composite 4821-5143, predict 5406-5557 / _predict_composite 5611-6172,
full exact variance 4360-4515, sample_posterior 6173-6598, score 6600-6636 and
save / load 6638-7013.  Same argument names and defaults; the model is

    K_full = sum_s A_s (x) K_s + diag(noise_t) (+ fixed observation noise),

one latent kernel per s over shared inputs: an RBF / Matern leaf (isotropic or
ARD), a composite kernel tree, or a mixed continuous x categorical tree whose
categorical leaves read integer levels from their input columns
(_fit_mixed_composite, multi_output_gp.py:5144-5405; its categorical
correlation parameters train beside the continuous ones).  Training,
prediction, exact variance and the pathwise correction run in
libmojogp_amd.so; the RFF prior draws use the caller's NumPy Generator exactly
as the reference and are evaluated on the device.

Outside the engine (``NotImplementedError``): isotropic polynomial leaves,
heteroskedastic noise models, fixed observation noise with mixed latents (as
the reference) and pathwise samples of composite latents (no random Fourier
features).
"""

from __future__ import annotations

import json
import warnings
from dataclasses import dataclass, field
from pathlib import Path
from typing import Any, Optional, Union

import numpy as np

from . import _engine
from .gp import normalize_fit_method
from .kernel import (KernelNode, Matern12, Matern32, Matern52, RBF, cat_raw_from_constrained,
                     make_ard_kernel)
from .pathwise_prior import (build_feature_weights, build_pathwise_feature_map,
                             sample_prior_values)

_MODEL_SCHEMA_VERSION = 1
_PRECOND_METHODS = {"greedy": 0, "rpcholesky": 1, "nystrom": 2}
_KERNEL_STRINGS = {"rbf": RBF, "matern12": Matern12, "matern32": Matern32, "matern52": Matern52}
_DEFAULT_PREDICT_LANCZOS_RANK = 100
_DEFAULT_ARD_PREDICT_LANCZOS_RANK = 200


@dataclass
class MultiOutputPredictionResult:
    mean: np.ndarray
    variance: Optional[np.ndarray] = None
    std: Optional[np.ndarray] = None


@dataclass
class LMCTrainingResult:
    final_nll: float
    nll_history: np.ndarray
    iterations: int
    converged: bool
    num_latents: int
    num_tasks: int
    noise_per_task: np.ndarray
    lengthscales: Optional[np.ndarray] = None
    outputscales: Optional[np.ndarray] = None
    params_per_latent: Optional[list] = None
    kernel_types: Optional[np.ndarray] = None
    A_matrices: Optional[np.ndarray] = None
    L_factors: Optional[np.ndarray] = None
    B: Optional[np.ndarray] = None
    Q: Optional[np.ndarray] = None
    Lambda: Optional[np.ndarray] = None
    alpha: Optional[np.ndarray] = None          # task-blocked [T * n]
    use_ard: bool = False
    lengthscales_per_dim: Optional[np.ndarray] = None
    mean_per_task: Optional[np.ndarray] = None
    var_diag: Optional[np.ndarray] = None
    iter_times_ms: Optional[np.ndarray] = None
    fixed_observation_noise: Optional[np.ndarray] = None
    cat_params_per_latent: Optional[list] = None       # constrained, per latent
    cat_param_names_per_latent: Optional[list] = None


def _leaves(node: KernelNode) -> list:
    if node.kernel_type is not None:
        return [node]
    out = _leaves(node.left) if node.left is not None else []
    return out + (_leaves(node.right) if node.right is not None else [])


def _mixed_layout(kernel: KernelNode, X: np.ndarray, latent: Optional[int] = None):
    """Categorical layout of one mixed latent (_configure_latent_kernels_for_fit,
    multi_output_gp.py:4136-4218): the leaves' {"levels", "kernel_type"} specs
    in tree order, their input columns, the continuous columns (the default
    dimensions of the latent's continuous leaves) and the categorical parameter
    names.  Columns must hold integer levels in [0, L).  latent: the LMC
    latent index (None: the ICM kernel), for the messages."""
    leaves = kernel.categorical_leaves()
    what = "kernel" if latent is None else f"latent {latent}"
    pure = ("Pure categorical kernels (all dimensions categorical, no continuous) are not "
            "supported" if latent is None else
            "Pure categorical latent kernels are not supported for MultiOutputLMCGP. "
            f"Latent kernel {latent} contains no continuous dimensions.")
    if all(lf.is_categorical() for lf in _leaves(kernel)):
        raise ValueError(pure)
    specs, cols, names = [], [], []
    for lf in leaves:
        col = int(lf.active_dims[0])
        if col >= X.shape[1]:
            raise ValueError(f"{what}: categorical column {col} out of range")
        v = X[:, col]
        L = int(lf.levels)
        if np.any(v != np.round(v)) or np.any(v < 0) or np.any(v >= L):
            raise ValueError(f"{what}: column {col} must hold integer levels in [0, {L})")
        specs.append({"levels": L, "kernel_type": lf.kernel_type.name.lower()})
        cols.append(col)
        names.extend(lf.get_param_names())
    cont = [c for c in range(X.shape[1]) if c not in set(cols)]
    if not cont:
        raise ValueError(pure)
    return specs, cols, cont, names


def _resolve_precond(rank: int, method: str, use_preconditioner: Optional[bool]):
    """resolve_preconditioner_settings for the LMC constructor: a disabled
    preconditioner is rank 0; 'auto' means greedy."""
    method = "greedy" if method == "auto" else method
    if method not in _PRECOND_METHODS:
        raise ValueError(f"preconditioner must be one of {sorted(_PRECOND_METHODS)} or 'auto'")
    rank = int(rank)
    if rank < 0:
        raise ValueError("preconditioner_rank must be >= 0")
    use = rank > 0 if use_preconditioner is None else bool(use_preconditioner)
    if not use:
        rank = 0
    return use, rank, method, _PRECOND_METHODS[method]


def _summarize(kernels, params_per_latent, use_ard: bool):
    """Lengthscale / outputscale summaries by parameter name
    (_summarize_lmc_kernel_params, multi_output_gp.py:177-228)."""
    ls_all, os_all, per_dim = [], [], []
    for k, p in zip(kernels, params_per_latent):
        lat = []
        for name, v in zip(k.get_param_names(), np.asarray(p, np.float32)):
            if name.endswith("_lengthscale") or "_ls_" in name:
                ls_all.append(float(v))
                if "_ls_" in name:
                    lat.append(float(v))
            if name.endswith("_outputscale"):
                os_all.append(float(v))
        if use_ard and lat:
            per_dim.append(np.asarray(lat, np.float32))
    lpd = None
    if use_ard and per_dim and len({len(v) for v in per_dim}) == 1:
        lpd = np.stack(per_dim).astype(np.float32)
    return np.asarray(ls_all, np.float32), np.asarray(os_all, np.float32), lpd


class MultiOutputLMCGP:
    """Linear Model of Coregionalization over R latent kernels."""

    def __init__(self, kernels: list, num_probes: int = 10, max_cg_iterations: int = 200,
                 cg_tolerance: float = 1.0, preconditioner_rank: int = 15,
                 precond_rebuild_threshold: float = 0.5, preconditioner: str = "greedy",
                 use_preconditioner: Optional[bool] = None, max_tridiag_iterations: int = 30,
                 ard: bool = False, init_mean: Optional[Union[float, np.ndarray]] = None):
        conv = []
        for k in kernels:
            if isinstance(k, str):
                if k.lower() not in _KERNEL_STRINGS:
                    raise NotImplementedError(
                        f"latent kernel {k!r} is outside the gfx950 engine "
                        f"(supported: {sorted(_KERNEL_STRINGS)})")
                k = _KERNEL_STRINGS[k.lower()]()
            if not isinstance(k, KernelNode):
                raise ValueError("All kernels must be KernelNode objects or valid kernel strings.")
            ncat = sum(lf.num_params() for lf in k.categorical_leaves())
            if not k.is_native_leaf() and (not k.is_tree_servable()
                                           or k.num_params() - ncat != k.engine_num_params()):
                raise NotImplementedError(f"latent kernel {k!r} is outside the gfx950 LMC "
                                          "engine (isotropic polynomial leaves are "
                                          "single-output only)")
            conv.append(k)
        if not conv:
            raise ValueError("MultiOutputLMCGP needs at least one latent kernel")
        self._original_kernels = [KernelNode.from_dict(k.to_dict()) for k in conv]
        self.kernels = conv
        self.num_latents = len(conv)
        self.num_probes = int(num_probes)
        self.max_cg_iter = int(max_cg_iterations)
        self.cg_tol = float(cg_tolerance)
        (self.use_preconditioner, self.precond_rank, self.precond,
         self.precond_method) = _resolve_precond(preconditioner_rank, preconditioner,
                                                 use_preconditioner)
        self.precond_rebuild_threshold = float(precond_rebuild_threshold)
        self.max_tridiag_iter = int(max_tridiag_iterations)
        self.ard = bool(ard)
        self.method = "materialized"
        self._init_mean = init_mean
        self._fitted_mean: Optional[np.ndarray] = None
        self._engine = None
        self._modules: Optional[list] = None
        self._provider_infos: Optional[list] = None
        self._is_trained = False
        self._X_train: Optional[np.ndarray] = None
        self._Y_train: Optional[np.ndarray] = None
        self._result: Optional[LMCTrainingResult] = None
        self._raw_result: Optional[dict] = None
        self._backend_train_info: Optional[dict] = None
        self._backend_predict_info: Optional[dict] = None
        self._backend_sample_info: Optional[dict] = None
        self._fixed_observation_noise: Optional[np.ndarray] = None
        # per latent: continuous columns of a mixed latent (None otherwise),
        # categorical specs and raw categorical parameters
        self._latent_cont_cols: list = [None] * len(conv)
        self._latent_cat_specs: list = [[] for _ in conv]
        self._latent_cat_raw: list = [np.zeros(0, np.float32) for _ in conv]
        self._latent_cat_cols: list = [[] for _ in conv]
        self._latent_cat_names: list = [[] for _ in conv]

    @property
    def has_mixed_latents(self) -> bool:
        return any(k.has_categorical() for k in self._original_kernels)

    # ------------------------------------------------------------ properties
    @property
    def is_trained(self) -> bool:
        return self._is_trained

    @property
    def training_result(self) -> Optional[LMCTrainingResult]:
        return self._result

    @property
    def backend_train_info(self) -> Optional[dict]:
        return self._backend_train_info

    @property
    def backend_predict_info(self) -> Optional[dict]:
        return self._backend_predict_info

    @property
    def backend_sample_info(self) -> Optional[dict]:
        return self._backend_sample_info

    @property
    def task_covariance(self) -> Optional[np.ndarray]:
        return None if self._result is None else self._result.B

    @property
    def num_tasks(self) -> Optional[int]:
        return None if self._result is None else self._result.num_tasks

    # ------------------------------------------------------------ providers
    def _destroy_providers(self) -> None:
        if self._provider_infos is not None and self._modules is not None:
            for mod, info in zip(self._modules, self._provider_infos):
                mod.destroy_provider(info)
        self._provider_infos = None

    def __del__(self):  # pragma: no cover - best effort
        try:
            self._destroy_providers()
        except Exception:
            pass

    def _build_providers(self, X: np.ndarray, params_per_latent, method: str) -> list:
        d = X.shape[1]
        self._modules = [_engine.load_kernel_module(k, False, d, default_dims=cc)
                         for k, cc in zip(self.kernels, self._latent_cont_cols)]
        infos = []
        for s, (mod, p) in enumerate(zip(self._modules, params_per_latent)):
            info = mod.init_provider(X, np.asarray(p, np.float32), 0.0)
            if self._latent_cat_specs[s]:
                kinds = [_engine.Engine._CAT_KIND[c["kernel_type"]]
                         for c in self._latent_cat_specs[s]]
                _engine._provider(info).set_categorical_params(kinds, self._latent_cat_raw[s])
            if method == "materialized":
                mod.materialize(info)
            infos.append(info)
        return infos

    def _ensure_providers(self) -> list:
        if self._provider_infos is None:
            params = [np.asarray(p, np.float32) for p in self._result.params_per_latent]
            self._provider_infos = self._build_providers(self._X_train, params, self.method)
        return self._provider_infos

    def _resolve_latents(self, X: np.ndarray) -> None:
        """Per-latent categorical layout for the training inputs X and the
        kernels as trained (ARD over the continuous columns of a mixed latent)."""
        d = X.shape[1]
        self._latent_cont_cols, self._latent_cat_specs = [], []
        self._latent_cat_names, self._latent_cat_cols = [], []
        kernels = []
        for s, k in enumerate(self._original_kernels):
            if k.has_categorical():
                specs, cols, cont, names = _mixed_layout(k, X, s)
                kernels.append(make_ard_kernel(k, len(cont)) if self.ard
                               else KernelNode.from_dict(k.to_dict()))
            else:
                specs, cols, cont, names = [], [], None, []
                kernels.append(make_ard_kernel(k, d) if self.ard
                               else KernelNode.from_dict(k.to_dict()))
            self._latent_cont_cols.append(cont)
            self._latent_cat_specs.append(specs)
            self._latent_cat_cols.append(cols)
            self._latent_cat_names.append(names)
        self.kernels = kernels

    def _latent_init(self, s: int) -> np.ndarray:
        """Initial parameters of latent s in its fit layout: the public layout
        for a continuous latent, the continuous (engine) parameters of a mixed
        one, whose categorical parameters train separately."""
        k = self.kernels[s]
        p = k.get_initial_params().astype(np.float32)
        return k.to_engine_params(p) if self._latent_cat_specs[s] else p

    def _latent_count(self, s: int) -> int:
        k = self.kernels[s]
        return k.engine_num_params() if self._latent_cat_specs[s] else k.num_params()

    # ------------------------------------------------------------ fit
    def fit(self, X, Y, max_iterations: int = 100, learning_rate: float = 0.05,
            method: str = "materialized", initial_lengthscales: Optional[np.ndarray] = None,
            initial_params: Optional[np.ndarray] = None, initial_noise: float = 0.1,
            initial_noise_per_task: Optional[np.ndarray] = None,
            fixed_observation_noise: Optional[np.ndarray] = None,
            input_dependent_noise: Optional[Any] = None, grouped_noise: Optional[Any] = None,
            verbose: bool = False, early_stop_tol: float = 1e-4, early_stop_patience: int = 15,
            use_fused_kernels: bool = True, observation_noise=None, observation_noise_fn=None,
            noise_model: str = "scalar", noise_group_train=None, group_noise=None,
            progress: Any = None, progress_stats: Optional[Any] = None,
            progress_interval: int = 1) -> LMCTrainingResult:
        if (observation_noise is not None or observation_noise_fn is not None
                or noise_model != "scalar" or noise_group_train is not None
                or group_noise is not None or input_dependent_noise is not None
                or grouped_noise is not None):
            raise NotImplementedError(
                "MultiOutputLMCGP supports scalar or per-task noise (plus fixed observation "
                "noise) only")
        method = normalize_fit_method(method)
        X = np.ascontiguousarray(X, dtype=np.float32)
        Y = np.ascontiguousarray(Y, dtype=np.float32)
        if X.ndim != 2:
            raise ValueError(f"X must be 2D [n, d], got shape {X.shape}")
        if Y.ndim != 2:
            raise ValueError(f"Y must be 2D [n, T], got shape {Y.shape}")
        if X.shape[0] != Y.shape[0]:
            raise ValueError(f"X has {X.shape[0]} samples, Y has {Y.shape[0]} -- must match")
        if not np.all(np.isfinite(X)):
            raise ValueError("X contains NaN or Inf values")
        if not np.all(np.isfinite(Y)):
            raise ValueError("Y contains NaN or Inf values")
        if initial_noise <= 0:
            raise ValueError(f"initial_noise must be > 0, got {initial_noise}")
        if learning_rate <= 0:
            raise ValueError(f"learning_rate must be > 0, got {learning_rate}")
        if max_iterations <= 0:
            raise ValueError(f"max_iterations must be > 0, got {max_iterations}")
        n, d = X.shape
        T = Y.shape[1]
        R = self.num_latents
        if fixed_observation_noise is not None:
            fixed_observation_noise = np.ascontiguousarray(fixed_observation_noise, np.float32)
            if fixed_observation_noise.shape != (n, T):
                raise ValueError(f"fixed_observation_noise must have shape ({n}, {T})")
            if not np.all(np.isfinite(fixed_observation_noise)) or np.any(
                    fixed_observation_noise < 0):
                raise ValueError("fixed_observation_noise must be finite and >= 0")
        if initial_noise_per_task is not None:
            noise0 = np.asarray(initial_noise_per_task, np.float32)
            if noise0.shape != (T,):
                raise ValueError(f"initial_noise_per_task must have shape ({T},)")
            if np.any(noise0 <= 0):
                raise ValueError("all initial_noise_per_task entries must be > 0")
        else:
            noise0 = np.full(T, initial_noise, np.float32)
        mixed = self.has_mixed_latents
        if mixed and fixed_observation_noise is not None:
            raise NotImplementedError(
                "fixed_observation_noise for mixed MultiOutputLMCGP is not yet supported; use "
                "continuous LMC or omit fixed observation noise.")
        self.method = method
        self._resolve_latents(X)
        counts = [self._latent_count(s) for s in range(R)]
        if initial_params is not None and initial_lengthscales is not None:
            raise ValueError("Provide either initial_params or initial_lengthscales for "
                             "MultiOutputLMCGP.fit(), not both.")
        if initial_params is not None:
            flat = np.ascontiguousarray(initial_params, np.float32).ravel()
            if flat.shape != (sum(counts),):
                raise ValueError(f"init_params must have shape ({sum(counts)},) "
                                 "[flat concat of per-latent params]")
        else:
            flat = np.concatenate([self._latent_init(s) for s in range(R)]).astype(np.float32)
            if initial_lengthscales is not None:
                flat = self._params_from_lengthscales(np.asarray(initial_lengthscales, np.float32))
        if self._init_mean is None:
            mean0 = np.mean(Y, axis=0).astype(np.float32)
        elif isinstance(self._init_mean, (int, float)):
            mean0 = np.full(T, float(self._init_mean), np.float32)
        else:
            mean0 = np.asarray(self._init_mean, np.float32)
        per_latent, off = [], 0
        for s, (c, k) in enumerate(zip(counts, self.kernels)):
            sl = flat[off:off + c]
            per_latent.append(sl.copy() if self._latent_cat_specs[s] else k.to_engine_params(sl))
            off += c
        self._destroy_providers()
        self._engine = _engine.load_engine()
        from .kernel import cat_default_raw_param
        cat0 = [np.asarray([cat_default_raw_param(lf.kernel_type, i, lf.levels)
                            for lf in k.categorical_leaves() for i in range(lf.num_params())],
                           np.float32) for k in self.kernels]
        self._latent_cat_raw = cat0
        infos = self._build_providers(X, per_latent, method)
        masks = [np.ones(c, bool) for c in counts]
        fixed_arg = (fixed_observation_noise if fixed_observation_noise is not None
                     else np.zeros((n, T), np.float32))
        try:
            if mixed:
                if early_stop_patience != 15 or early_stop_tol != 1e-4:
                    warnings.warn("early_stop_patience and early_stop_tol are not used: the "
                                  "engine handles convergence internally via max_iterations.",
                                  UserWarning, stacklevel=2)
                Cs = [np.ascontiguousarray(X[:, cols], np.int32).reshape(n, len(cols))
                      for cols in self._latent_cat_cols]
                raw = self._engine.train_lmc_mixed(
                    infos, per_latent, Y, T, Cs, self._latent_cat_specs, cat0,
                    int(max_iterations), float(learning_rate), bool(verbose), self.num_probes,
                    self.max_cg_iter, float(self.cg_tol), self.precond_rank,
                    self.precond_method, float(self.precond_rebuild_threshold),
                    self.max_tridiag_iter, noise0, fixed_arg, False, mean0,
                    1 if method == "materialized" else 0)
            else:
                raw = self._engine.train_lmc(
                    infos, per_latent, masks, Y, T, int(max_iterations), float(learning_rate),
                    bool(verbose), self.num_probes, self.max_cg_iter, float(self.cg_tol),
                    self.precond_rank, self.precond_method,
                    float(self.precond_rebuild_threshold), self.max_tridiag_iter, noise0,
                    fixed_arg, fixed_observation_noise is not None, mean0)
        except Exception:
            for mod, info in zip(self._modules, infos):
                mod.destroy_provider(info)
            raise
        self._provider_infos = infos
        if mixed:
            self._latent_cat_raw = [np.asarray(r, np.float32) for r in raw["cat_raw_per_latent"]]
        params = [np.asarray(p, np.float32) if self._latent_cat_specs[s]
                  else k.from_engine_params(np.asarray(p, np.float32))
                  for s, (k, p) in enumerate(zip(self.kernels, raw["params_per_latent"]))]
        public = [k.from_engine_params(np.asarray(p, np.float32))
                  for k, p in zip(self.kernels, raw["params_per_latent"])]
        ls, os_, lpd = _summarize(self.kernels, public, self.ard)
        A = np.asarray(raw["A_matrices"], np.float32)
        B = A.sum(axis=0).astype(np.float32)
        lam, Q = np.linalg.eigh(B.astype(np.float64))
        self._result = LMCTrainingResult(
            final_nll=float(raw["final_nll"]),
            nll_history=np.asarray(raw["nll_history"], np.float32),
            iterations=int(raw["iterations"]), converged=bool(raw["converged"]),
            num_latents=R, num_tasks=T,
            noise_per_task=np.asarray(raw["noise_per_task"], np.float32),
            lengthscales=ls, outputscales=os_, params_per_latent=[p.tolist() for p in params],
            kernel_types=np.asarray([k.native_kind() if k.is_native_leaf() else -1
                                     for k in self.kernels], np.int32),
            A_matrices=A, L_factors=np.asarray(raw["L_factors"], np.float32), B=B,
            Q=Q.astype(np.float32), Lambda=lam.astype(np.float32),
            alpha=np.asarray(raw["alpha"], np.float32), use_ard=self.ard,
            lengthscales_per_dim=lpd, mean_per_task=np.asarray(raw["mean_per_task"], np.float32),
            var_diag=np.asarray(raw["var_diag"], np.float32),
            iter_times_ms=np.asarray(raw["iter_times_ms"], np.float64),
            fixed_observation_noise=fixed_observation_noise,
            cat_params_per_latent=([np.asarray(c, np.float32) for c in
                                    raw["cat_params_per_latent"]] if mixed else None),
            cat_param_names_per_latent=(self._latent_cat_names if mixed else None))
        self._X_train, self._Y_train = X, Y
        self._fixed_observation_noise = fixed_observation_noise
        self._raw_result = raw
        self._backend_train_info = {
            k: raw[k] for k in ("training_route", "materialization_mode", "precond_rank",
                                "precond_method", "precond_rebuild_count",
                                "precond_rebuild_threshold", "max_tridiag_iter",
                                "uses_fixed_observation_noise", "iterations", "converged")}
        self._backend_train_info["use_preconditioner"] = bool(self.use_preconditioner)
        self._fitted_mean = self._result.mean_per_task
        self._is_trained = True
        self._backend_predict_info = None
        self._backend_sample_info = None
        return self._result

    def _params_from_lengthscales(self, values: np.ndarray) -> np.ndarray:
        """_build_lmc_initial_params_from_lengthscales (multi_output_gp.py:231-290)."""
        idx = [[i for i, nm in enumerate(k.get_param_names())
                if nm.endswith("_lengthscale") or "_ls_" in nm] for k in self.kernels]
        counts = [len(i) for i in idx]
        total = sum(counts)
        if values.shape == (len(self.kernels),) and all(c == 1 for c in counts):
            per = [values[s:s + 1] for s in range(len(self.kernels))]
        elif values.shape == (total,):
            per, off = [], 0
            for c in counts:
                per.append(values[off:off + c])
                off += c
        elif len(set(counts)) == 1 and values.shape == (len(self.kernels), counts[0]):
            per = [values[s] for s in range(len(self.kernels))]
        else:
            raise ValueError(f"initial_lengthscales has shape {values.shape}, incompatible "
                             f"with per-latent lengthscale counts {counts}")
        out = []
        for s, (k, ix, v) in enumerate(zip(self.kernels, idx, per)):
            p = k.get_initial_params().copy()
            p[ix] = v
            out.append(k.to_engine_params(p) if self._latent_cat_specs[s] else p)
        return np.concatenate(out).astype(np.float32)

    # ------------------------------------------------------------ predict
    def _check_test(self, X_test) -> np.ndarray:
        if not self._is_trained:
            raise RuntimeError("GP must be trained before prediction. Call fit() first.")
        X_test = np.ascontiguousarray(X_test, dtype=np.float32)
        if X_test.ndim != 2:
            raise ValueError(f"X_test must be 2D [m, d], got shape {X_test.shape}")
        if X_test.shape[1] != self._X_train.shape[1]:
            raise ValueError(f"X_test has {X_test.shape[1]} features, expected "
                             f"{self._X_train.shape[1]}")
        if not np.all(np.isfinite(X_test)):
            raise ValueError("X_test contains NaN or Inf values")
        return X_test

    def _solve_budget(self):
        """max(max_cg, 100) iterations, tolerance min(cg_tol, 1e-2)
        (multi_output_gp.py:4420-4423, 6480-6483)."""
        tol = min(self.cg_tol, 1e-2) if self.cg_tol > 0 else 1e-2
        return max(self.max_cg_iter, 100), tol

    def predict(self, X_test, return_var: bool = False, return_std: bool = False,
                variance_method: str = "love", progress: Any = None,
                progress_stats: Optional[Any] = None):
        valid = ("love", "exact", "mean_only")
        if variance_method not in valid:
            raise ValueError(f"variance_method must be one of {valid}, got '{variance_method}'")
        if self._fixed_observation_noise is not None and variance_method == "love":
            raise NotImplementedError(
                "MultiOutputLMCGP fixed_observation_noise supports exact prediction and "
                "pathwise sampling; use variance_method='exact' or 'mean_only'.")
        X_test = self._check_test(X_test)
        r = self._result
        R, T = r.num_latents, r.num_tasks
        infos = self._ensure_providers()
        params = [np.asarray(p, np.float32) for p in r.params_per_latent]
        noise = np.asarray(r.noise_per_task, np.float32)
        vm = {"mean_only": 0, "love": 1, "exact": 2}[variance_method]
        rank = _DEFAULT_PREDICT_LANCZOS_RANK
        if self.ard:
            rank = max(rank, _DEFAULT_ARD_PREDICT_LANCZOS_RANK)
        rank = max(rank, int(self.num_probes))
        res = self._engine.predict_lmc(
            infos, r.alpha, r.A_matrices, X_test, params, self._fitted_mean,
            self._X_train.shape[0], T, noise, 1 if vm == 1 else 0, self.max_cg_iter,
            float(self.cg_tol), self.precond_rank, rank)
        mean = res["mean"]
        variance = res.get("variance")
        route = "predict_lmc"
        var_route = "predict_lmc" if vm == 1 else None
        if vm == 2:
            max_cg, tol = self._solve_budget()
            if self.method == "materialized":
                # The reference factors the dense joint covariance on the host
                # here; the device block solve is run to a tight tolerance.
                max_cg, tol = max(max_cg, 1000), 1e-6
            variance = self.exact_variance(X_test, max_cg_iter=max_cg, cg_tol=tol)
            var_route = "predict_lmc_full_exact"
        if variance is not None:
            variance = np.maximum(variance, 1e-10).astype(np.float32)
        self._backend_predict_info = {
            "requested_method": self.method, "actual_prediction_route": route,
            "backend_prediction_used": True, "backend_variance_used": variance is not None,
            "variance_method": variance_method, "fallback_used": False,
            "actual_variance_route": var_route,
            "training_route": (self._backend_train_info or {}).get("training_route",
                                                                  self.method),
            "lanczos_rank_used": int(res.get("lanczos_rank_used", rank)),
            "precond_rank": self.precond_rank, "precond_method": self.precond_method}
        if return_var:
            return mean, variance
        if return_std:
            return mean, (np.sqrt(variance) if variance is not None else None)
        return MultiOutputPredictionResult(
            mean=mean, variance=variance,
            std=np.sqrt(variance) if variance is not None else None)

    def predict_latent(self, X_test, return_var: bool = False, return_std: bool = False,
                       variance_method: str = "love", **kwargs):
        """p(f_test | y_train) of every task (multi_output_gp.py:5558-5577)."""
        return self.predict(X_test, return_var=return_var, return_std=return_std,
                            variance_method=variance_method, **kwargs)

    def predict_observed(self, X_test, observation_noise=None, noise_group_test=None,
                         return_var: bool = False, return_std: bool = False,
                         variance_method: str = "love", **kwargs):
        """p(y_test | y_train) with explicit test-point noise variances [m, T];
        training noise is never reused for new points
        (multi_output_gp.py:5579-5609)."""
        latent = self.predict(X_test, variance_method=variance_method, **kwargs)
        noise = _resolve_observed_noise(latent.mean.shape[0], latent.mean.shape[1],
                                        observation_noise, noise_group_test, None)
        var = std = None
        if latent.variance is not None:
            var = np.ascontiguousarray(latent.variance + noise, dtype=np.float32)
            std = np.sqrt(var)
        if return_var:
            return latent.mean, var
        if return_std:
            return latent.mean, std
        return MultiOutputPredictionResult(mean=latent.mean, variance=var, std=std)

    def exact_variance(self, X_test, *, max_cg_iter: Optional[int] = None,
                       cg_tol: Optional[float] = None, block_points: int = 0) -> np.ndarray:
        """Exact joint posterior variance [m, T] with the task noise
        (multi_output_gp.py:4360-4515), all (point, task) right-hand sides of a
        block in one device solve."""
        import ctypes as C

        from . import _lib
        X_test = self._check_test(X_test)
        r = self._result
        mc, tol = self._solve_budget()
        mc = int(max_cg_iter) if max_cg_iter is not None else mc
        tol = float(cg_tol) if cg_tol is not None else tol
        infos = self._ensure_providers()
        provs = [_engine._provider(i) for i in infos]
        for p, prm in zip(provs, r.params_per_latent):
            p.update_params(np.asarray(prm, np.float32))
            p.update_noise(0.0)
        T = r.num_tasks
        A = np.ascontiguousarray(r.A_matrices, np.float32)
        noise = np.ascontiguousarray(r.noise_per_task, np.float32)
        fixed = None
        if self._fixed_observation_noise is not None:
            fixed = np.ascontiguousarray(self._fixed_observation_noise.T)
        m = X_test.shape[0]
        var = np.zeros((m, T), np.float32)
        its = C.c_int(0)
        _lib.call("mgp_lmc_exact_variance", _lib.handles(provs), len(provs), T, _lib.fptr(A),
                  _lib.fptr(noise), _lib.ofptr(fixed), _lib.fptr(X_test), m, mc, tol,
                  int(block_points), _lib.fptr(var), C.byref(its))
        self._last_exact_cg_iterations = int(its.value)
        return var

    def score(self, X_test, Y_test) -> dict:
        if not self._is_trained:
            raise RuntimeError("GP must be trained before scoring. Call fit() first.")
        Y_test = np.ascontiguousarray(Y_test, dtype=np.float32)
        pred = self.predict(X_test, variance_method="mean_only")
        mean = pred.mean if isinstance(pred, MultiOutputPredictionResult) else pred
        resid = Y_test - mean
        ss_res = np.sum(resid ** 2)
        ss_tot = np.sum((Y_test - np.mean(Y_test, axis=0)) ** 2)
        return {"rmse": float(np.sqrt(np.mean(resid ** 2))),
                "mae": float(np.mean(np.abs(resid))),
                "r2": float(1.0 - ss_res / (ss_tot + 1e-10)),
                "rmse_per_task": np.sqrt(np.mean(resid ** 2, axis=0))}

    # ------------------------------------------------------------ sampling
    def sample_posterior(self, X_test, n_samples: int = 1, method: str = "diagonal",
                         n_rff_features: int = 1024,
                         rng: Optional[np.random.Generator] = None) -> np.ndarray:
        if not self._is_trained:
            raise RuntimeError("GP must be trained before sampling. Call fit() first.")
        if method not in ("diagonal", "pathwise"):
            raise ValueError(f"method must be 'diagonal' or 'pathwise', got '{method}'")
        if rng is None:
            rng = np.random.default_rng()
        route = (self._backend_train_info or {}).get("training_route", self.method)
        if method == "pathwise":
            samples = self._sample_posterior_pathwise(X_test, int(n_samples),
                                                      int(n_rff_features), rng)
            self._backend_sample_info = {
                "requested_method": method, "actual_sampling_method": "pathwise",
                "actual_sampling_route": "provider_pathwise", "backend_sampling_used": True,
                "backend_correction_used": True,
                "backend_correction_route": "sample_lmc_pathwise", "training_route": route,
                "prior_sampler_family": "shared_feature_map",
                "n_rff_features": int(n_rff_features)}
            return samples
        mean, std = self.predict(X_test, return_std=True)
        z = rng.standard_normal((n_samples, mean.shape[0], mean.shape[1]))
        self._backend_sample_info = {
            "requested_method": method, "actual_sampling_method": "diagonal",
            "actual_sampling_route": "diagonal_from_predictive_std",
            "backend_sampling_used": True, "backend_correction_used": False,
            "training_route": route}
        return (mean[None] + std[None] * z).astype(np.float32)

    def _sample_posterior_pathwise(self, X_test, n_samples: int, n_rff_features: int,
                                   rng: np.random.Generator) -> np.ndarray:
        """Prior draws through shared RFF maps plus the exact LMC correction
        (multi_output_gp.py:6276-6598).  The Generator is consumed in the
        reference's order (feature maps per latent, then per sample: weights
        per latent, observation noise); all samples share one batched
        correction solve."""
        X_test = self._check_test(X_test)
        r = self._result
        R, T = r.num_latents, r.num_tasks
        X = self._X_train
        n, d = X.shape
        S = int(n_samples)
        if S < 1:
            raise ValueError("n_samples must be >= 1")
        y_c = (self._Y_train - np.asarray(self._fitted_mean, np.float32)[None, :]).astype(
            np.float32)
        noise = np.asarray(r.noise_per_task, np.float32)
        mean = np.asarray(self._fitted_mean, np.float32)
        fmaps, mix = [], []
        if not all(k.is_native_leaf() for k in self.kernels):
            raise NotImplementedError("pathwise samples need RBF / Matern latents (random "
                                      "Fourier features); composite trees have none")
        for s in range(R):
            fmaps.append(build_pathwise_feature_map(
                self.kernels[s].native_kind(), r.params_per_latent[s], input_dim=d,
                n_features=n_rff_features, rng=rng, ard=self.ard))
            A_s = np.asarray(r.A_matrices[s], np.float64)
            jitter = float(np.abs(np.diag(A_s)).mean()) * 1e-6 + 1e-8
            mix.append(np.linalg.cholesky(A_s + jitter * np.eye(T)))
        if self._fixed_observation_noise is not None:
            scale = np.sqrt(np.maximum(noise[None, :] + self._fixed_observation_noise,
                                       0.0)).astype(np.float32)
        else:
            scale = np.sqrt(np.maximum(noise, 0.0)).astype(np.float32)[None, :]
        weights = [[None] * R for _ in range(S)]
        eps = np.empty((S, n, T), np.float32)
        for c in range(S):
            for s in range(R):
                weights[c][s] = build_feature_weights(fmaps[s], T, rng)
            eps[c] = rng.standard_normal((n, T)).astype(np.float32)
        prior_train = np.zeros((S, n, T), np.float32)
        prior_test = np.zeros((S, X_test.shape[0], T), np.float32)
        for s in range(R):
            W = np.concatenate([weights[c][s] for c in range(S)], axis=0)   # [S*T, F]
            tr = sample_prior_values(fmaps[s], X, W).reshape(S, T, n)
            te = sample_prior_values(fmaps[s], X_test, W).reshape(S, T, -1)
            for c in range(S):
                prior_train[c] += np.einsum("ln,tl->nt", tr[c].astype(np.float64),
                                            mix[s]).astype(np.float32)
                prior_test[c] += np.einsum("ln,tl->nt", te[c].astype(np.float64),
                                           mix[s]).astype(np.float32)
        resid = np.ascontiguousarray(y_c[None] - (prior_train + eps * scale), np.float32)
        max_cg, tol = self._solve_budget()
        infos = self._ensure_providers()
        params = [np.asarray(p, np.float32) for p in r.params_per_latent]
        fixed = (self._fixed_observation_noise if self._fixed_observation_noise is not None
                 else np.zeros((0,), np.float32))
        raw = self._engine.sample_lmc_pathwise(infos, resid, r.A_matrices, X_test, params, noise,
                                               max_cg, tol, fixed)
        corr = np.asarray(raw["correction"], np.float32).reshape(S, X_test.shape[0], T)
        return (mean[None, None, :] + prior_test + corr).astype(np.float32)

    # ------------------------------------------------------------ persistence
    def save(self, path: str) -> None:
        """``<path>_config.json`` + ``<path>_arrays.npz`` (multi_output_gp.py:6638-6743)."""
        if not self._is_trained:
            raise RuntimeError("GP must be trained before saving. Call fit() first.")
        path = str(path)
        if path.endswith(".json") or path.endswith(".npz"):
            path = path.rsplit(".", 1)[0]
        from . import __version__
        tr = self._result
        cfg = {"schema_version": _MODEL_SCHEMA_VERSION, "mojogp_version": __version__,
               "wrapper": "MultiOutputLMCGP", "is_composite": True,
               "has_mixed_latents": self.has_mixed_latents, "ard": self.ard,
               "method": self.method,
               "num_probes": self.num_probes, "max_cg_iter": self.max_cg_iter,
               "cg_tol": self.cg_tol, "use_preconditioner": self.use_preconditioner,
               "precond_rank": self.precond_rank, "precond": self.precond,
               "precond_rebuild_threshold": self.precond_rebuild_threshold,
               "num_latents": tr.num_latents, "num_tasks": tr.num_tasks,
               "final_nll": float(tr.final_nll), "iterations": int(tr.iterations),
               "converged": bool(tr.converged), "use_ard": bool(tr.use_ard),
               "has_fixed_observation_noise": self._fixed_observation_noise is not None,
               "kernel_trees": [k.to_dict() for k in self._original_kernels],
               "kernel_mojo_type": self._original_kernels[0].to_mojo_type()}
        Path(path + "_config.json").write_text(json.dumps(cfg, indent=2, default=float))
        arrays = {"X_train": self._X_train, "Y_train": self._Y_train,
                  "lengthscales": tr.lengthscales, "outputscales": tr.outputscales,
                  "kernel_types": tr.kernel_types, "noise_per_task": tr.noise_per_task,
                  "A_matrices": tr.A_matrices, "L_factors": tr.L_factors, "B": tr.B, "Q": tr.Q,
                  "Lambda": tr.Lambda, "alpha": tr.alpha, "nll_history": tr.nll_history,
                  "mean_per_task": tr.mean_per_task, "fitted_mean": self._fitted_mean,
                  "var_diag": tr.var_diag, "iter_times_ms": tr.iter_times_ms,
                  "lengthscales_per_dim": tr.lengthscales_per_dim,
                  "fixed_observation_noise": self._fixed_observation_noise}
        for s, p in enumerate(tr.params_per_latent):
            arrays[f"params_latent_{s}"] = np.asarray(p, np.float32)
            if tr.cat_params_per_latent is not None:
                arrays[f"cat_params_latent_{s}"] = np.asarray(
                    tr.cat_params_per_latent[s], np.float32)
        np.savez(path + "_arrays.npz", **{k: v for k, v in arrays.items() if v is not None})

    @classmethod
    def load(cls, path: str, kernels: Optional[list] = None) -> "MultiOutputLMCGP":
        path = str(path)
        if path.endswith(".json") or path.endswith(".npz"):
            path = path.rsplit(".", 1)[0]
        cfg = json.loads(Path(path + "_config.json").read_text())
        if cfg.get("wrapper") != "MultiOutputLMCGP":
            raise ValueError("saved model is not a MultiOutputLMCGP")
        if int(cfg.get("schema_version", 0)) != _MODEL_SCHEMA_VERSION:
            raise ValueError("unsupported model schema version")
        arr = np.load(path + "_arrays.npz", allow_pickle=False)
        missing = [k for k in ("X_train", "Y_train", "noise_per_task", "A_matrices",
                               "nll_history") if k not in arr]
        if missing:
            raise ValueError("MultiOutputLMCGP artifact is missing required arrays: "
                             + ", ".join(missing))
        if kernels is None:
            kernels = [KernelNode.from_dict(k) for k in cfg["kernel_trees"]]
        gp = cls(kernels, num_probes=cfg["num_probes"], max_cg_iterations=cfg["max_cg_iter"],
                 cg_tolerance=cfg["cg_tol"], preconditioner_rank=cfg["precond_rank"],
                 precond_rebuild_threshold=cfg["precond_rebuild_threshold"],
                 preconditioner=cfg["precond"], use_preconditioner=cfg["use_preconditioner"],
                 ard=cfg["ard"])
        gp.method = cfg.get("method", "materialized")
        gp._X_train = np.ascontiguousarray(arr["X_train"], np.float32)
        gp._Y_train = np.ascontiguousarray(arr["Y_train"], np.float32)
        gp._resolve_latents(gp._X_train)
        R = int(cfg["num_latents"])
        mixed = bool(cfg.get("has_mixed_latents"))
        if mixed:
            # the file holds the constrained categorical parameters (as the
            # reference writes them); the tables come from their raw values
            miss = [f"cat_params_latent_{s}" for s in range(R)
                    if gp._latent_cat_specs[s] and f"cat_params_latent_{s}" not in arr]
            if miss:
                raise ValueError("MultiOutputLMCGP artifact is missing required arrays: "
                                 + ", ".join(miss))
            gp._latent_cat_raw = []
            for s in range(R):
                raw, off = [], 0
                theta = (np.asarray(arr[f"cat_params_latent_{s}"], np.float32)
                         if gp._latent_cat_specs[s] else np.zeros(0, np.float32))
                for lf in gp.kernels[s].categorical_leaves():
                    k = lf.num_params()
                    raw.append(cat_raw_from_constrained(lf.kernel_type, int(lf.levels),
                                                        theta[off:off + k]))
                    off += k
                if off != theta.size:
                    raise ValueError(f"cat_params_latent_{s} has {theta.size} values, the "
                                     f"latent's categorical leaves need {off}")
                gp._latent_cat_raw.append(np.concatenate(raw).astype(np.float32) if raw
                                          else np.zeros(0, np.float32))
        get = lambda k: arr[k] if k in arr else None  # noqa: E731
        fixed = get("fixed_observation_noise")
        gp._fixed_observation_noise = (np.ascontiguousarray(fixed, np.float32)
                                       if fixed is not None else None)
        gp._result = LMCTrainingResult(
            final_nll=float(cfg["final_nll"]), nll_history=arr["nll_history"],
            iterations=int(cfg["iterations"]), converged=bool(cfg["converged"]),
            num_latents=R, num_tasks=int(cfg["num_tasks"]),
            noise_per_task=arr["noise_per_task"], lengthscales=get("lengthscales"),
            outputscales=get("outputscales"),
            params_per_latent=[arr[f"params_latent_{s}"].tolist() for s in range(R)],
            kernel_types=get("kernel_types"), A_matrices=arr["A_matrices"],
            L_factors=get("L_factors"), B=get("B"), Q=get("Q"), Lambda=get("Lambda"),
            alpha=get("alpha"), use_ard=bool(cfg.get("use_ard", False)),
            lengthscales_per_dim=get("lengthscales_per_dim"),
            mean_per_task=get("mean_per_task"), var_diag=get("var_diag"),
            iter_times_ms=get("iter_times_ms"), fixed_observation_noise=gp._fixed_observation_noise,
            cat_params_per_latent=([np.asarray(arr[f"cat_params_latent_{s}"], np.float32)
                                    if gp._latent_cat_specs[s] else np.zeros(0, np.float32)
                                    for s in range(R)] if mixed else None),
            cat_param_names_per_latent=(gp._latent_cat_names if mixed else None))
        fm = get("fitted_mean")
        gp._fitted_mean = fm if fm is not None else gp._result.mean_per_task
        gp._backend_train_info = {"training_route": gp.method}
        gp._engine = _engine.load_engine()
        gp._is_trained = True
        return gp

    def __repr__(self) -> str:
        kinds = ", ".join(k.kernel_type.name.lower() if k.kernel_type is not None else repr(k)
                          for k in self._original_kernels)
        return (f"MultiOutputLMCGP(kernels=[{kinds}], num_latents={self.num_latents}, "
                f"trained={self._is_trained})")


# =============================================================================
# ICM multi-output GP
# =============================================================================

_ICM_PRESETS = {
    "fast": {"max_cg_iter": 50, "cg_tol": 5e-2, "num_probes": 5, "max_tridiag_iter": 15,
             "precond_rank": 5, "precond_rebuild_threshold": 0.75, "precond": "greedy"},
    "balanced": {"max_cg_iter": 200, "cg_tol": 1e-2, "num_probes": 10, "max_tridiag_iter": 30,
                 "precond_rank": 15, "precond_rebuild_threshold": 0.5, "precond": "greedy"},
    "accurate": {"max_cg_iter": 400, "cg_tol": 1e-2, "num_probes": 20, "max_tridiag_iter": 60,
                 "precond_rank": 20, "precond_rebuild_threshold": 0.25, "precond": "greedy"},
}
_PATHWISE_TEST_CHUNK = 512


@dataclass
class MultiOutputTrainingResult:
    """Trained ICM state (multi_output_gp.py:475-542)."""

    params: np.ndarray
    noise: float
    noise_per_task: np.ndarray
    final_nll: float
    iterations: int
    converged: bool
    num_tasks: int
    task_rank: int
    num_kernel_params: int
    B: np.ndarray                 # [T, T] outputscale * task covariance
    Q: np.ndarray                 # [T, T] eigenvectors of B
    Lambda: np.ndarray            # [T] eigenvalues of B, floored at 1e-6
    effective_scales: np.ndarray  # alias of Lambda
    W: np.ndarray
    raw_v: np.ndarray
    alpha_rotated: np.ndarray     # [n, T]
    mean_per_task: np.ndarray
    nll_history: np.ndarray
    param_names: list
    cat_params: Optional[np.ndarray] = None
    cat_param_names: list = field(default_factory=list)
    iter_times_ms: Optional[np.ndarray] = None

    @property
    def lengthscale(self) -> float:
        for i, name in enumerate(self.param_names):
            if "lengthscale" in name and "ls_" not in name:
                return float(self.params[i])
        return float(self.params[0])

    @property
    def outputscale(self) -> float:
        for i, name in enumerate(self.param_names):
            if "outputscale" in name:
                return float(self.params[i])
        return float(self.params[-1])

    @property
    def lengthscales(self) -> np.ndarray:
        idxs = [i for i, nm in enumerate(self.param_names) if "ls_" in nm]
        if idxs:
            return self.params[idxs]
        return np.array([self.lengthscale], dtype=np.float32)

    @property
    def dim(self) -> int:
        return len(self.lengthscales)


def _resolve_observed_noise(m: int, T: int, observation_noise=None, noise_group_test=None,
                            group_noise=None) -> np.ndarray:
    """Explicit test-point noise [m, T] (multi_output_gp.py:553-603)."""
    if observation_noise is not None and noise_group_test is not None:
        raise ValueError("Pass either observation_noise or noise_group_test for observed "
                         "prediction, not both")
    if observation_noise is not None:
        noise = np.ascontiguousarray(observation_noise, dtype=np.float32)
        if noise.shape != (m, T):
            raise ValueError(f"observation_noise must have shape ({m}, {T}), got {noise.shape}")
    elif noise_group_test is not None:
        if group_noise is None:
            raise ValueError("noise_group_test requires group_noise from fitted grouped noise "
                             "state")
        groups = np.ascontiguousarray(noise_group_test, dtype=np.int32)
        if groups.shape != (m,):
            raise ValueError(f"noise_group_test must have shape ({m},), got {groups.shape}")
        if np.any(groups < 0):
            raise ValueError("noise_group_test must contain non-negative group ids")
        if int(groups.max(initial=-1)) >= group_noise.shape[0]:
            raise ValueError("noise_group_test references a group id outside group_noise")
        noise = np.ascontiguousarray(group_noise[groups], dtype=np.float32)
    else:
        raise ValueError("Observed multi-output prediction requires explicit observation_noise "
                         "or noise_group_test; training noise is not reused for new points")
    if not np.all(np.isfinite(noise)):
        raise ValueError("observed prediction noise contains NaN or Inf values")
    if np.any(noise <= 0):
        raise ValueError("observed prediction noise values must be > 0")
    return noise


class MultiOutputGP:
    """ICM multi-output GP: K_full = os (B (x) K_X) + diag(noise_t),
    B = W W^T + diag(softplus(raw_v)) (mojogp/multi_output_gp.py:859-3402).

    Training runs the Kronecker-preconditioned BBMM loop of libmojogp_amd.so;
    prediction decomposes os B = Q diag(Lambda) Q^T into T independent
    single-output problems (mean from the rotated alpha, LOVE or exact
    variance per eigen-task).  Kernels: RBF / Matern-5/2, isotropic or ARD.
    """

    _PRESETS = _ICM_PRESETS

    def __init__(self, kernel: Union[str, KernelNode] = "rbf", task_rank: int = -1,
                 ard: bool = False, num_probes: Optional[int] = None,
                 max_cg_iterations: Optional[int] = None, cg_tolerance: Optional[float] = None,
                 preconditioner_rank: Optional[int] = None,
                 precond_rebuild_threshold: Optional[float] = None,
                 preconditioner: Optional[str] = None, use_preconditioner: Optional[bool] = None,
                 init_mean: Optional[Union[float, np.ndarray]] = None,
                 preset: Optional[str] = None, max_tridiag_iterations: Optional[int] = None):
        if preset is not None and preset not in self._PRESETS:
            raise ValueError(f"Unknown preset '{preset}'. Must be one of: "
                             f"{list(self._PRESETS)}")
        base = dict(self._PRESETS[preset or "balanced"])
        if num_probes is not None:
            base["num_probes"] = num_probes
        if max_cg_iterations is not None:
            base["max_cg_iter"] = max_cg_iterations
        if cg_tolerance is not None:
            base["cg_tol"] = cg_tolerance
        if max_tridiag_iterations is not None:
            base["max_tridiag_iter"] = max_tridiag_iterations
        rank = base["precond_rank"] if preconditioner_rank is None else preconditioner_rank
        (self.use_preconditioner, self.precond_rank, self.precond,
         self.precond_method) = _resolve_precond(rank, preconditioner or base["precond"],
                                                 use_preconditioner)
        self._preconditioner_explicitly_configured = (
            use_preconditioner is not None or preconditioner_rank is not None
            or preconditioner is not None)
        if isinstance(kernel, str):
            if kernel.lower() not in _KERNEL_STRINGS:
                raise NotImplementedError(
                    f"kernel {kernel!r} is outside the gfx950 engine "
                    f"(supported: {sorted(_KERNEL_STRINGS)})")
            kernel = _KERNEL_STRINGS[kernel.lower()]()
        if not isinstance(kernel, KernelNode):
            raise ValueError(f"kernel must be a string or KernelNode, got {type(kernel)}")
        if not kernel.is_native_leaf():
            # composite and mixed continuous x categorical trees run on the
            # kernel-tree products; the isotropic polynomial's hidden variance
            # slot is single-output only
            ncat = sum(lf.num_params() for lf in kernel.categorical_leaves())
            if (not kernel.is_tree_servable()
                    or kernel.num_params() - ncat != kernel.engine_num_params()):
                raise NotImplementedError(f"kernel {kernel!r} is outside the gfx950 ICM engine "
                                          "(isotropic polynomial leaves are single-output only)")
        self._is_composite = True
        self.kernel = kernel
        self._original_kernel = kernel
        self._compiled_kernel = kernel
        if int(task_rank) == 0 or int(task_rank) < -1:
            raise ValueError("task_rank must be -1 (full rank) or >= 1")
        self.task_rank = int(task_rank)
        self.ard = bool(ard)
        self.method = "materialized"
        self.num_probes = int(base["num_probes"])
        self.max_cg_iter = int(base["max_cg_iter"])
        self.cg_tol = float(base["cg_tol"])
        self.precond_rebuild_threshold = float(
            base["precond_rebuild_threshold"] if precond_rebuild_threshold is None
            else precond_rebuild_threshold)
        self.max_tridiag_iter = int(base["max_tridiag_iter"])
        self._init_mean = init_mean
        self._fitted_mean: Optional[np.ndarray] = None
        self._engine = None
        self._kernel_module = None
        self._dim: Optional[int] = None
        self._provider_info: Optional[dict] = None
        self._training_method: Optional[str] = None
        self._is_trained = False
        self._X_train: Optional[np.ndarray] = None
        self._Y_train: Optional[np.ndarray] = None
        self._observation_noise_train: Optional[np.ndarray] = None
        self._noise_group_train: Optional[np.ndarray] = None
        self._noise_group_values: Optional[np.ndarray] = None
        self._result: Optional[MultiOutputTrainingResult] = None
        self._raw_result: Optional[dict] = None
        self._backend_train_info: Optional[dict] = None
        self._backend_predict_info: Optional[dict] = None
        self._backend_sample_info: Optional[dict] = None
        # mixed continuous x categorical kernels: continuous columns, the
        # categorical leaves' specs / columns and their raw parameters
        self._cont_cols: Optional[list] = None
        self._cat_specs: list = []
        self._cat_cols: list = []
        self._cat_params_raw: Optional[np.ndarray] = None

    @property
    def _is_mixed(self) -> bool:
        return self._original_kernel.has_categorical()

    # ------------------------------------------------------------ properties
    @property
    def is_trained(self) -> bool:
        return self._is_trained

    @property
    def training_result(self) -> Optional[MultiOutputTrainingResult]:
        return self._result

    @property
    def backend_train_info(self) -> Optional[dict]:
        return self._backend_train_info

    @property
    def backend_predict_info(self) -> Optional[dict]:
        return self._backend_predict_info

    @property
    def backend_sample_info(self) -> Optional[dict]:
        return self._backend_sample_info

    @property
    def task_covariance(self) -> Optional[np.ndarray]:
        return None if self._result is None else self._result.B

    @property
    def num_tasks(self) -> Optional[int]:
        return None if self._result is None else self._result.num_tasks

    # ------------------------------------------------------------ provider
    def _destroy_persistent_provider(self) -> None:
        if self._provider_info is not None and self._kernel_module is not None:
            self._kernel_module.destroy_provider(self._provider_info)
        self._provider_info = None

    def __del__(self):  # pragma: no cover - best effort
        try:
            self._destroy_persistent_provider()
        except Exception:
            pass

    def _ensure_compiled(self, dim: int) -> None:
        self._engine = _engine.load_engine()
        self._kernel_module = _engine.load_kernel_module(
            self._compiled_kernel, False, dim,
            default_dims=self._cont_cols if self._is_mixed else None)
        self._dim = dim

    def _build_provider_info(self, X, params, noise) -> dict:
        info = self._kernel_module.init_provider(np.ascontiguousarray(X, np.float32),
                                                 np.ascontiguousarray(params, np.float32),
                                                 float(noise))
        if self._is_mixed and self._cat_params_raw is not None:
            kinds = [_engine.Engine._CAT_KIND[c["kernel_type"]] for c in self._cat_specs]
            _engine._provider(info).set_categorical_params(kinds, self._cat_params_raw)
        if self.method == "materialized":
            self._kernel_module.materialize(info)
        return info

    def _engine_params(self, params) -> np.ndarray:
        """Engine layout of result parameters: a mixed kernel's results are
        already its continuous (engine) parameters."""
        p = np.asarray(params, np.float32)
        return p if self._is_mixed else self._compiled_kernel.to_engine_params(p)

    def _continuous_param_names(self) -> list:
        """Names of the engine-layout parameters (the public names with the
        categorical slots dropped)."""
        k = self._compiled_kernel
        names = k.get_param_names()
        idx = np.rint(k.to_engine_params(np.arange(k.num_params(), dtype=np.float32) + 0.25)
                      - 0.25).astype(int)
        return [names[i] for i in idx]

    def _ensure_provider(self) -> dict:
        r = self._result
        if self._provider_info is None:
            if self._kernel_module is None:
                self._ensure_compiled(self._X_train.shape[1])
            self._provider_info = self._build_provider_info(
                self._X_train, self._engine_params(r.params), float(np.mean(r.noise_per_task)))
        return self._provider_info

    # ------------------------------------------------------------ fit
    def fit(self, X, Y, max_iterations: int = 100, learning_rate: float = 0.05,
            method: str = "materialized", initial_lengthscale: float = 1.0,
            initial_lengthscales: Optional[np.ndarray] = None,
            initial_params: Optional[np.ndarray] = None, initial_noise: float = 0.1,
            initial_noise_per_task: Optional[np.ndarray] = None,
            input_dependent_noise: Optional[Any] = None, grouped_noise: Optional[Any] = None,
            initial_outputscale: float = 1.0, verbose: bool = False,
            early_stop_tol: float = 1e-4, early_stop_patience: int = 15,
            use_fused_kernels: bool = True, lr_schedule: str = "constant",
            observation_noise: Optional[np.ndarray] = None, observation_noise_fn=None,
            noise_model: str = "scalar", noise_group_train=None, group_noise=None,
            progress: Any = None, progress_stats: Optional[Any] = None,
            progress_interval: int = 1) -> MultiOutputTrainingResult:
        """multi_output_gp.py:1431-1832 and _fit_composite 1834-2034."""
        if observation_noise_fn is not None or input_dependent_noise is not None:
            raise NotImplementedError(
                "MultiOutputGP input-dependent heteroskedastic noise is in development")
        if grouped_noise is not None:
            raise NotImplementedError("grouped_noise models are in development; use "
                                      "noise_model='grouped' with group_noise")
        if noise_model not in ("scalar", "fixed_vector", "grouped"):
            raise NotImplementedError(
                "MultiOutputGP currently supports scalar, per-task, fixed per-sample-task, and "
                "fixed grouped noise only")
        if noise_model == "fixed_vector" and observation_noise is None:
            raise ValueError("noise_model='fixed_vector' requires observation_noise with "
                             "shape [n, T]")
        if noise_model == "grouped" and observation_noise is not None:
            raise ValueError("noise_model='grouped' expands group_noise to observation_noise; "
                             "do not also pass observation_noise")
        if noise_model != "grouped" and (noise_group_train is not None
                                         or group_noise is not None):
            raise ValueError("noise_group_train and group_noise require noise_model='grouped'")
        self._destroy_persistent_provider()
        method = normalize_fit_method(method)
        self.method = method
        X = np.ascontiguousarray(X, dtype=np.float32)
        Y = np.ascontiguousarray(Y, dtype=np.float32)
        if X.ndim != 2:
            raise ValueError(f"X must be 2D [n, d], got shape {X.shape}")
        if Y.ndim != 2:
            raise ValueError(f"Y must be 2D [n, T], got shape {Y.shape}")
        if X.shape[0] != Y.shape[0]:
            raise ValueError(f"X has {X.shape[0]} samples, Y has {Y.shape[0]} -- must match")
        if not np.all(np.isfinite(X)):
            raise ValueError("X contains NaN or Inf values")
        if not np.all(np.isfinite(Y)):
            raise ValueError("Y contains NaN or Inf values")
        if initial_noise <= 0:
            raise ValueError(f"initial_noise must be > 0, got {initial_noise}")
        n, d = X.shape
        T = Y.shape[1]
        groups_arr = gnoise_arr = None
        if noise_model == "grouped":
            if noise_group_train is None:
                raise ValueError("noise_model='grouped' requires noise_group_train")
            if group_noise is None:
                raise ValueError("noise_model='grouped' requires group_noise")
            groups_arr = np.ascontiguousarray(noise_group_train, dtype=np.int32)
            if groups_arr.shape != (n,):
                raise ValueError(f"noise_group_train must have shape ({n},), got "
                                 f"{groups_arr.shape}")
            if np.any(groups_arr < 0):
                raise ValueError("noise_group_train must contain non-negative group ids")
            gnoise_arr = np.ascontiguousarray(group_noise, dtype=np.float32)
            if gnoise_arr.ndim != 2 or gnoise_arr.shape[1] != T:
                raise ValueError(f"group_noise must have shape [G, {T}], got "
                                 f"{gnoise_arr.shape}")
            if gnoise_arr.shape[0] == 0:
                raise ValueError("group_noise must contain at least one group")
            if not np.all(np.isfinite(gnoise_arr)):
                raise ValueError("group_noise contains NaN or Inf values")
            if np.any(gnoise_arr <= 0):
                raise ValueError("group_noise values must be > 0")
            if int(groups_arr.max(initial=-1)) >= gnoise_arr.shape[0]:
                raise ValueError("noise_group_train references a group id outside group_noise")
            observation_noise = gnoise_arr[groups_arr]
        obs = None
        if observation_noise is not None and self._is_mixed:
            raise NotImplementedError(
                "MultiOutputGP fixed per-sample-task observation_noise currently supports "
                "continuous kernels only; mixed heteroskedastic noise is in development")
        if observation_noise is not None:
            obs = np.ascontiguousarray(observation_noise, dtype=np.float32)
            if obs.shape != Y.shape:
                raise ValueError(f"observation_noise must have shape {Y.shape}, got {obs.shape}")
            if not np.all(np.isfinite(obs)):
                raise ValueError("observation_noise contains NaN or Inf values")
            if np.any(obs <= 0):
                raise ValueError("observation_noise values must be > 0")
            initial_noise_per_task = np.mean(obs, axis=0).astype(np.float32)
            self.use_preconditioner = False
            self.precond_rank = 0
        if learning_rate <= 0:
            raise ValueError(f"learning_rate must be > 0, got {learning_rate}")
        if max_iterations <= 0:
            raise ValueError(f"max_iterations must be > 0, got {max_iterations}")
        if int(progress_interval) < 1:
            raise ValueError("progress_interval must be >= 1")
        if lr_schedule not in ("constant", "cosine"):
            raise ValueError(f"lr_schedule must be 'constant' or 'cosine', got '{lr_schedule}'")
        if initial_noise_per_task is not None:
            initial_noise_per_task = np.asarray(initial_noise_per_task, dtype=np.float32)
            if initial_noise_per_task.shape != (T,):
                raise ValueError(f"initial_noise_per_task must have shape ({T},), got "
                                 f"{initial_noise_per_task.shape}")
            if np.any(initial_noise_per_task <= 0):
                raise ValueError("all initial_noise_per_task entries must be > 0")
        if self.task_rank > T:
            raise ValueError(f"task_rank={self.task_rank} exceeds num_tasks={T}")
        self._observation_noise_train = obs
        self._noise_group_train = groups_arr
        self._noise_group_values = gnoise_arr
        self._cat_params_raw = None
        if self._is_mixed:
            self._cat_specs, self._cat_cols, self._cont_cols, self._cat_names = _mixed_layout(
                self._original_kernel, X)
            cont_d = len(self._cont_cols)
            self._compiled_kernel = (make_ard_kernel(self._original_kernel, cont_d) if self.ard
                                     else KernelNode.from_dict(self._original_kernel.to_dict()))
            self.kernel = self._compiled_kernel
            if initial_lengthscales is not None or initial_lengthscale != 1.0:
                raise ValueError("initial_lengthscale(s) apply to single RBF / Matern kernels; "
                                 "pass initial_params for kernel trees")
            return self._fit_mixed(X, Y, T, max_iterations, learning_rate, initial_params,
                                   initial_noise, initial_noise_per_task, initial_outputscale,
                                   verbose, early_stop_tol, early_stop_patience,
                                   lr_schedule == "cosine", progress, progress_interval)
        self._cont_cols, self._cat_specs, self._cat_cols = None, [], []
        self._compiled_kernel = (make_ard_kernel(self._original_kernel, d) if self.ard
                                 else KernelNode.from_dict(self._original_kernel.to_dict()))
        self.kernel = self._compiled_kernel
        num_params = self._compiled_kernel.num_params()
        if not self._compiled_kernel.is_native_leaf() and (
                initial_lengthscales is not None or initial_lengthscale != 1.0
                or initial_outputscale != 1.0):
            raise ValueError("initial_lengthscale(s) / initial_outputscale apply to single "
                             "RBF / Matern kernels; pass initial_params for kernel trees")
        if initial_lengthscales is not None and len(initial_lengthscales) != num_params - 1:
            raise ValueError(f"initial_lengthscales must have shape ({num_params - 1},), got "
                             f"({len(initial_lengthscales)},)")
        if initial_params is None and (initial_lengthscale != 1.0 or initial_outputscale != 1.0
                                       or initial_lengthscales is not None):
            initial_params = np.ones(num_params, dtype=np.float32)
            if initial_lengthscales is not None:
                initial_params[:num_params - 1] = np.asarray(initial_lengthscales, np.float32)
            else:
                initial_params[:num_params - 1] = initial_lengthscale
            initial_params[-1] = initial_outputscale
        if initial_params is None:
            initial_params = np.ones(num_params, dtype=np.float32)
        initial_params = np.ascontiguousarray(initial_params, dtype=np.float32)
        if initial_params.shape != (num_params,):
            raise ValueError(f"init_params must have shape ({num_params},), got "
                             f"{initial_params.shape}")
        if self._init_mean is None:
            mean0 = np.mean(Y, axis=0).astype(np.float32)
        elif isinstance(self._init_mean, (int, float)):
            mean0 = np.full(T, float(self._init_mean), np.float32)
        else:
            mean0 = np.asarray(self._init_mean, np.float32)
        noise0 = (np.ascontiguousarray(initial_noise_per_task, np.float32)
                  if initial_noise_per_task is not None
                  else np.full(T, initial_noise, np.float32))
        self._ensure_compiled(d)
        engine_params = self._compiled_kernel.to_engine_params(initial_params)
        info = self._build_provider_info(X, engine_params, 0.0)
        self._provider_info = info
        self._training_method = method
        args = [info, Y, engine_params, np.ones(num_params, dtype=bool), noise0, 1.0, mean0,
                int(T), int(max_iterations), float(learning_rate), int(self.task_rank),
                bool(verbose), int(self.num_probes), int(self.max_cg_iter), float(self.cg_tol),
                int(self.precond_rank), int(self.precond_method),
                float(self.precond_rebuild_threshold), int(self.max_tridiag_iter),
                int(early_stop_patience), float(early_stop_tol), lr_schedule == "cosine", obs]
        if callable(progress):
            args.extend([progress, int(progress_interval)])
        try:
            raw = self._engine.train_multi_output(*args)
        except Exception:
            self._destroy_persistent_provider()
            raise
        noise_pt = np.asarray(raw["noise_per_task"], np.float32)
        mean_pt = np.asarray(raw["mean_per_task"], np.float32)
        params = self._compiled_kernel.from_engine_params(np.asarray(raw["params"], np.float32))
        os_ = float(raw["outputscale"])
        B_flat = np.asarray(raw["B_flat"], np.float32)
        B = B_flat.reshape(T, T) if B_flat.size == T * T else np.eye(T, dtype=np.float32)
        B_scaled = os_ * B
        eigvals, Q = np.linalg.eigh(B_scaled)
        Lam = np.maximum(eigvals, 1e-6).astype(np.float32)
        alpha_blocked = np.asarray(raw["alpha"], np.float32)
        alpha_rot = (alpha_blocked.reshape(T, n).T.astype(np.float64)
                     @ Q.astype(np.float64)).astype(np.float32)
        hist = np.asarray(raw["nll_history"], np.float32)
        self._result = MultiOutputTrainingResult(
            params=params, noise=float(np.mean(noise_pt)), noise_per_task=noise_pt,
            final_nll=float(raw["final_nll"]), iterations=int(raw["iterations"]),
            converged=bool(raw["converged"]), num_tasks=T, task_rank=int(raw["task_rank"]),
            num_kernel_params=len(params), B=B_scaled.astype(np.float32),
            Q=Q.astype(np.float32), Lambda=Lam, effective_scales=Lam,
            W=np.zeros((T, max(int(raw["task_rank"]), 1)), np.float32),
            raw_v=np.zeros(T, np.float32), alpha_rotated=alpha_rot, mean_per_task=mean_pt,
            nll_history=hist if hist.size else np.array([raw["final_nll"]], np.float32),
            param_names=self._compiled_kernel.get_param_names(),
            iter_times_ms=np.asarray(raw["iter_times_ms"], np.float64))
        self._X_train, self._Y_train = X, Y
        self._raw_result = raw
        self._backend_train_info = {
            k: raw[k] for k in ("training_route", "materialization_mode", "max_tridiag_iter",
                                "precond_rebuild_threshold", "precond_rebuild_count",
                                "precond_rank", "precond_method", "noise_mode",
                                "has_observation_noise_vector", "iter_times_ms")}
        self._backend_train_info["use_preconditioner"] = bool(self.use_preconditioner)
        self._is_trained = True
        self._fitted_mean = mean_pt.copy()
        self._backend_predict_info = None
        self._backend_sample_info = None
        return self._result

    def _fit_mixed(self, X, Y, T, max_iterations, learning_rate, initial_params, initial_noise,
                   initial_noise_per_task, initial_outputscale, verbose, early_stop_tol,
                   early_stop_patience, use_cosine_lr, progress, progress_interval):
        """_fit_mixed_composite (multi_output_gp.py:2036-2228): the kernel tree's
        continuous parameters (engine layout), the ICM outputscale, per-task
        noise and means, and the categorical leaves' raw parameters from their
        defaults, trained by the mixed ICM loop."""
        from .kernel import cat_default_raw_param
        n, d = X.shape
        k = self._compiled_kernel
        num_params = k.engine_num_params()
        if initial_params is None:
            initial_params = k.to_engine_params(k.get_initial_params())
        initial_params = np.ascontiguousarray(initial_params, dtype=np.float32)
        if initial_params.shape != (num_params,):
            raise ValueError(f"init_params must have shape ({num_params},), got "
                             f"{initial_params.shape}. Kernel {k.to_mojo_type()} has "
                             f"{num_params} continuous parameters: "
                             f"{self._continuous_param_names()}")
        if self._init_mean is None:
            mean0 = np.mean(Y, axis=0).astype(np.float32)
        elif isinstance(self._init_mean, (int, float)):
            mean0 = np.full(T, float(self._init_mean), np.float32)
        else:
            mean0 = np.asarray(self._init_mean, np.float32)
        noise0 = (np.ascontiguousarray(initial_noise_per_task, np.float32)
                  if initial_noise_per_task is not None
                  else np.full(T, initial_noise, np.float32))
        cat0 = np.asarray([cat_default_raw_param(lf.kernel_type, i, lf.levels)
                           for lf in k.categorical_leaves() for i in range(lf.num_params())],
                          np.float32)
        self._ensure_compiled(d)
        self._cat_params_raw = cat0
        info = self._build_provider_info(X, initial_params, 0.0)
        self._provider_info = info
        self._training_method = self.method
        C = np.ascontiguousarray(X[:, self._cat_cols], np.int32).reshape(n, len(self._cat_cols))
        args = [info, Y, initial_params, noise0, float(initial_outputscale), mean0, int(T), C,
                self._cat_specs, cat0, int(max_iterations), float(learning_rate),
                int(self.task_rank), bool(verbose), int(self.num_probes), int(self.max_cg_iter),
                float(self.cg_tol), int(self.precond_rank), int(self.precond_method),
                float(self.precond_rebuild_threshold),
                1 if self.method == "materialized" else 0, int(self.max_tridiag_iter),
                int(early_stop_patience), float(early_stop_tol), bool(use_cosine_lr)]
        if callable(progress):
            args.extend([progress, int(progress_interval)])
        try:
            raw = self._engine.train_multi_output_mixed(*args)
        except Exception:
            self._destroy_persistent_provider()
            raise
        noise_pt = np.asarray(raw["noise_per_task"], np.float32)
        mean_pt = np.asarray(raw["mean_per_task"], np.float32)
        params = np.asarray(raw["params"], np.float32)
        os_ = float(raw["outputscale"])
        self._cat_params_raw = np.asarray(raw["cat_params"], np.float32)
        B_flat = np.asarray(raw["B_flat"], np.float32)
        B = B_flat.reshape(T, T) if B_flat.size == T * T else np.eye(T, dtype=np.float32)
        B_scaled = os_ * B
        eigvals, Q = np.linalg.eigh(B_scaled)
        Lam = np.maximum(eigvals, 1e-6).astype(np.float32)
        alpha_blocked = np.asarray(raw["alpha"], np.float32)
        alpha_rot = (alpha_blocked.reshape(T, n).T.astype(np.float64)
                     @ Q.astype(np.float64)).astype(np.float32)
        hist = np.asarray(raw["nll_history"], np.float32)
        self._result = MultiOutputTrainingResult(
            params=params, noise=float(np.mean(noise_pt)), noise_per_task=noise_pt,
            final_nll=float(raw["final_nll"]), iterations=int(raw["iterations"]),
            converged=bool(raw["converged"]), num_tasks=T, task_rank=int(raw["task_rank"]),
            num_kernel_params=len(params), B=B_scaled.astype(np.float32),
            Q=Q.astype(np.float32), Lambda=Lam, effective_scales=Lam,
            W=np.zeros((T, max(int(raw["task_rank"]), 1)), np.float32),
            raw_v=np.zeros(T, np.float32), alpha_rotated=alpha_rot, mean_per_task=mean_pt,
            nll_history=hist if hist.size else np.array([raw["final_nll"]], np.float32),
            param_names=self._continuous_param_names(),
            cat_params=self._cat_params_raw if self._cat_params_raw.size else None,
            cat_param_names=list(self._cat_names),
            iter_times_ms=np.asarray(raw["iter_times_ms"], np.float64))
        self._X_train, self._Y_train = X, Y
        self._raw_result = raw
        self._backend_train_info = {
            k_: raw[k_] for k_ in ("training_route", "materialization_mode", "max_tridiag_iter",
                                   "precond_rebuild_threshold", "precond_rebuild_count",
                                   "precond_rank", "precond_method", "iter_times_ms")}
        self._backend_train_info["use_preconditioner"] = bool(self.use_preconditioner)
        self._backend_train_info["is_mixed"] = True
        self._is_trained = True
        self._fitted_mean = mean_pt.copy()
        self._backend_predict_info = None
        self._backend_sample_info = None
        return self._result

    # ------------------------------------------------------------ predict
    def _check_test(self, X_test) -> np.ndarray:
        if not self._is_trained:
            raise RuntimeError("GP must be trained before prediction. Call fit() first.")
        X_test = np.ascontiguousarray(X_test, dtype=np.float32)
        if X_test.ndim != 2:
            raise ValueError(f"X_test must be 2D [m, d], got shape {X_test.shape}")
        if X_test.shape[1] != self._X_train.shape[1]:
            raise ValueError(f"X_test has {X_test.shape[1]} features, expected "
                             f"{self._X_train.shape[1]}")
        if not np.all(np.isfinite(X_test)):
            raise ValueError("X_test contains NaN or Inf values")
        return X_test

    def _predict_rank(self) -> int:
        """_prediction_lanczos_rank (multi_output_gp.py:147-164)."""
        rank = max(int(self.max_tridiag_iter), _DEFAULT_PREDICT_LANCZOS_RANK)
        if self.ard:
            rank = max(rank, _DEFAULT_ARD_PREDICT_LANCZOS_RANK)
        return rank

    def predict(self, X_test, return_var: bool = False, return_std: bool = False,
                variance_method: str = "love", progress: Any = None,
                progress_stats: Optional[Any] = None):
        """multi_output_gp.py:2521-2691 with _predict_composite 2360-2519."""
        valid = ("love", "exact", "mean_only")
        if variance_method not in valid:
            raise ValueError(f"variance_method must be one of {valid}, got '{variance_method}'")
        X_test = self._check_test(X_test)
        r = self._result
        T = r.num_tasks
        vm = {"mean_only": 0, "love": 1, "exact": 2}[variance_method]
        info = self._ensure_provider()
        params = self._engine_params(r.params)
        noise = float(np.mean(r.noise_per_task))
        tol = min(float(self.cg_tol), 1e-2) if float(self.cg_tol) > 0.0 else 1e-2
        rank = self._predict_rank()
        res = self._engine.predict_multi_output(
            info, r.alpha_rotated, r.Q, r.effective_scales, X_test, params, noise, vm,
            self.max_cg_iter, tol, self.precond_rank, rank)
        mean = np.asarray(res["mean"], np.float32) + self._fitted_mean[None, :]
        variance = (np.maximum(np.asarray(res["variance"], np.float32), 0)
                    if vm and "variance" in res else None)
        self._backend_predict_info = {
            "requested_method": self.method, "actual_prediction_route": "predict_multi_output",
            "backend_prediction_used": True, "backend_variance_used": vm != 0,
            "variance_method": variance_method, "fallback_used": False,
            "actual_variance_route": "predict_multi_output" if vm else None,
            "training_route": (self._backend_train_info or {}).get("training_route",
                                                                  self.method),
            "precond_rank": self.precond_rank, "precond_method": self.precond_method,
            "lanczos_rank_used": int(res.get("lanczos_rank_used", rank))}
        if return_var:
            return mean, variance
        if return_std:
            return mean, (np.sqrt(variance) if variance is not None else None)
        return MultiOutputPredictionResult(mean=mean, variance=variance,
                                           std=np.sqrt(variance) if variance is not None
                                           else None)

    def predict_latent(self, X_test, return_var: bool = False, return_std: bool = False,
                       variance_method: str = "love", **kwargs):
        return self.predict(X_test, return_var=return_var, return_std=return_std,
                            variance_method=variance_method, **kwargs)

    def predict_observed(self, X_test, observation_noise=None, noise_group_test=None,
                         return_var: bool = False, return_std: bool = False,
                         variance_method: str = "love", **kwargs):
        """p(y_test | y_train) with explicit test noise (multi_output_gp.py:2714-2744)."""
        latent = self.predict(X_test, variance_method=variance_method, **kwargs)
        noise = _resolve_observed_noise(latent.mean.shape[0], latent.mean.shape[1],
                                        observation_noise, noise_group_test,
                                        self._noise_group_values)
        var = std = None
        if latent.variance is not None:
            var = np.ascontiguousarray(latent.variance + noise, dtype=np.float32)
            std = np.sqrt(var)
        if return_var:
            return latent.mean, var
        if return_std:
            return latent.mean, std
        return MultiOutputPredictionResult(mean=latent.mean, variance=var, std=std)

    def score(self, X_test, Y_test) -> dict:
        if not self._is_trained:
            raise RuntimeError("GP must be trained before scoring. Call fit() first.")
        Y_test = np.ascontiguousarray(Y_test, dtype=np.float32)
        pred = self.predict(X_test)
        resid = Y_test - pred.mean
        ss_res = np.sum(resid ** 2)
        ss_tot = np.sum((Y_test - np.mean(Y_test, axis=0)) ** 2)
        return {"rmse": float(np.sqrt(np.mean(resid ** 2))),
                "mae": float(np.mean(np.abs(resid))),
                "r2": float(1.0 - ss_res / (ss_tot + 1e-10)),
                "rmse_per_task": np.sqrt(np.mean(resid ** 2, axis=0))}

    # ------------------------------------------------------------ sampling
    def sample_posterior(self, X_test, n_samples: int = 1, method: str = "diagonal",
                         n_rff_features: int = 1024,
                         rng: Optional[np.random.Generator] = None) -> np.ndarray:
        """multi_output_gp.py:2790-2892."""
        if not self._is_trained:
            raise RuntimeError("GP must be trained before sampling. Call fit() first.")
        if method not in ("diagonal", "pathwise"):
            raise ValueError("MultiOutputGP only supports method='diagonal' or 'pathwise', "
                             f"got '{method}'.")
        if rng is None:
            rng = np.random.default_rng()
        route = (self._backend_train_info or {}).get("training_route",
                                                    self._training_method or self.method)
        if method == "pathwise":
            samples = self._sample_posterior_pathwise(X_test, int(n_samples),
                                                      int(n_rff_features), rng)
            self._backend_sample_info = {
                "requested_method": method, "actual_sampling_method": "pathwise",
                "actual_sampling_route": "provider_pathwise", "backend_sampling_used": True,
                "backend_correction_used": True,
                "backend_correction_route": "sample_multi_output_pathwise",
                "training_route": route, "prior_sampler_family": "shared_feature_map",
                "n_rff_features": int(n_rff_features)}
            return samples
        mean, std = self.predict(X_test, return_std=True)
        z = rng.standard_normal((n_samples, mean.shape[0], mean.shape[1]))
        self._backend_sample_info = {
            "requested_method": method, "actual_sampling_method": "diagonal",
            "actual_sampling_route": "diagonal_from_predictive_std",
            "backend_sampling_used": True, "backend_correction_used": False,
            "training_route": route}
        return (mean[None] + std[None] * z).astype(np.float32)

    def _sample_posterior_pathwise(self, X_test, n_samples: int, n_rff_features: int,
                                   rng: np.random.Generator) -> np.ndarray:
        """Shared RFF prior through the eigen-tasks of os B plus the exact
        Kronecker correction (multi_output_gp.py:2894-3102).  The Generator is
        consumed in the reference's order (feature map, then per sample: task
        weights, observation noise); all samples share one batched solve."""
        X_test = self._check_test(X_test)
        r = self._result
        T = r.num_tasks
        X = self._X_train
        n, d = X.shape
        m = X_test.shape[0]
        S = int(n_samples)
        if S < 1:
            raise ValueError("n_samples must be >= 1")
        params = np.asarray(r.params, np.float32)
        noise = np.ascontiguousarray(r.noise_per_task, np.float32)
        mean = np.asarray(self._fitted_mean if self._fitted_mean is not None
                          else r.mean_per_task, np.float32)
        y_c = (self._Y_train - mean[None, :]).astype(np.float32)
        if not self._compiled_kernel.is_native_leaf():
            raise NotImplementedError("pathwise samples need an RBF / Matern kernel (random "
                                      "Fourier features); composite trees have none")
        fmap = build_pathwise_feature_map(self._compiled_kernel.native_kind(), params,
                                          input_dim=d, n_features=n_rff_features, rng=rng,
                                          ard=self.ard)
        Qd = np.asarray(r.Q, np.float64)
        sc = np.sqrt(np.maximum(np.asarray(r.Lambda, np.float64), 1e-8))
        train_noise = np.sqrt(np.maximum(noise, 0.0)).astype(np.float32)
        Wts, eps = [], np.empty((S, n, T), np.float32)
        for c in range(S):
            Wts.append(build_feature_weights(fmap, T, rng))
            eps[c] = rng.standard_normal((n, T)).astype(np.float32)
        Wall = np.concatenate(Wts, axis=0)                       # [S*T, F]
        tr = sample_prior_values(fmap, X, Wall).reshape(S, T, n)
        resid = np.empty((S, n, T), np.float32)
        for c in range(S):
            prior = np.einsum("ln,tl,l->nt", tr[c].astype(np.float64), Qd, sc).astype(np.float32)
            resid[c] = y_c - (prior + eps[c] * train_noise[None, :])
        info = self._ensure_provider()
        eparams = self._compiled_kernel.to_engine_params(params)
        max_cg = max(int(self.max_cg_iter), 100)
        tol = min(float(self.cg_tol), 1e-2) if float(self.cg_tol) > 0.0 else 1e-2
        out = np.empty((S, m, T), np.float32)
        for start in range(0, m, _PATHWISE_TEST_CHUNK):
            end = min(start + _PATHWISE_TEST_CHUNK, m)
            te = sample_prior_values(fmap, X_test[start:end], Wall).reshape(S, T, end - start)
            raw = self._engine.sample_multi_output_pathwise(
                info, resid, np.ascontiguousarray(r.B, np.float32), X_test[start:end], eparams,
                noise, max_cg, tol)
            corr = np.asarray(raw["correction"], np.float32).reshape(S, end - start, T)
            for c in range(S):
                prior = np.einsum("ln,tl,l->nt", te[c].astype(np.float64), Qd,
                                  sc).astype(np.float32)
                out[c, start:end] = mean[None, :] + prior + corr[c]
        return out

    # ------------------------------------------------------------ persistence
    def save(self, path: str) -> None:
        """``<path>_config.json`` + ``<path>_arrays.npz`` (multi_output_gp.py:3104-3207)."""
        if not self._is_trained:
            raise RuntimeError("GP must be trained before saving. Call fit() first.")
        path = str(path)
        if path.endswith(".json") or path.endswith(".npz"):
            path = path.rsplit(".", 1)[0]
        from . import __version__
        tr = self._result
        cfg = {"schema_version": _MODEL_SCHEMA_VERSION, "mojogp_version": __version__,
               "wrapper": "MultiOutputGP", "kernel": self._original_kernel.to_mojo_type(),
               "kernel_tree": self._original_kernel.to_dict(), "is_composite": True,
               "task_rank": self.task_rank, "ard": self.ard, "method": self.method,
               "num_probes": self.num_probes, "max_cg_iter": self.max_cg_iter,
               "cg_tol": self.cg_tol, "use_preconditioner": self.use_preconditioner,
               "precond_rank": self.precond_rank, "precond": self.precond,
               "precond_rebuild_threshold": self.precond_rebuild_threshold, "dim": self._dim,
               "noise": float(tr.noise), "final_nll": float(tr.final_nll),
               "iterations": int(tr.iterations), "converged": bool(tr.converged),
               "num_tasks": int(tr.num_tasks), "task_rank_result": int(tr.task_rank),
               "training_method": self._training_method or self.method,
               "has_observation_noise_vector": self._observation_noise_train is not None,
               "has_noise_group_train": self._noise_group_train is not None,
               "has_group_noise": self._noise_group_values is not None,
               "result_type": "MultiOutputTrainingResult",
               "num_kernel_params": int(tr.num_kernel_params),
               "param_names": list(tr.param_names), "cat_param_names": list(tr.cat_param_names)}
        Path(path + "_config.json").write_text(json.dumps(cfg, indent=2))
        arrays = {"X_train": self._X_train, "Y_train": self._Y_train, "B": tr.B, "Q": tr.Q,
                  "Lambda": tr.Lambda, "W": tr.W, "raw_v": tr.raw_v,
                  "alpha_rotated": tr.alpha_rotated, "effective_scales": tr.effective_scales,
                  "noise_per_task": tr.noise_per_task, "nll_history": tr.nll_history,
                  "mean_per_task": tr.mean_per_task, "params": tr.params,
                  "X_train_cont": self._X_train}
        if tr.iter_times_ms is not None:
            arrays["iter_times_ms"] = tr.iter_times_ms
        if self._observation_noise_train is not None:
            arrays["observation_noise_train"] = self._observation_noise_train
        if self._noise_group_train is not None:
            arrays["noise_group_train"] = self._noise_group_train
        if self._noise_group_values is not None:
            arrays["group_noise"] = self._noise_group_values
        if self._fitted_mean is not None:
            arrays["fitted_mean"] = self._fitted_mean
        if self._is_mixed:
            # the reference's mixed artifact: raw categorical parameters, the
            # continuous and the integer categorical columns
            arrays["cat_params"] = self._cat_params_raw
            arrays["X_train_cont"] = np.ascontiguousarray(self._X_train[:, self._cont_cols])
            arrays["C_train"] = np.ascontiguousarray(self._X_train[:, self._cat_cols], np.int32)
        np.savez(path + "_arrays.npz", **arrays)

    @classmethod
    def load(cls, path: str, kernel: Optional[Union[str, KernelNode]] = None) -> "MultiOutputGP":
        """multi_output_gp.py:3210-3386."""
        path = str(path)
        if path.endswith(".json") or path.endswith(".npz"):
            path = path.rsplit(".", 1)[0]
        cfg = json.loads(Path(path + "_config.json").read_text())
        if cfg.get("wrapper") != "MultiOutputGP":
            raise ValueError("Saved model is not a MultiOutputGP artifact. Expected "
                             f"wrapper='MultiOutputGP', got {cfg.get('wrapper')!r}.")
        if int(cfg.get("schema_version", 0)) != _MODEL_SCHEMA_VERSION:
            raise ValueError(f"Unsupported MultiOutputGP schema_version="
                             f"{cfg.get('schema_version')}; expected {_MODEL_SCHEMA_VERSION}.")
        if cfg.get("result_type") != "MultiOutputTrainingResult":
            raise ValueError(f"Unsupported MultiOutputGP result_type={cfg.get('result_type')!r}")
        arr = np.load(path + "_arrays.npz", allow_pickle=False)
        if kernel is None:
            kernel = (KernelNode.from_dict(cfg["kernel_tree"]) if cfg.get("kernel_tree")
                      else cfg.get("kernel", "rbf"))
        gp = cls(kernel=kernel, task_rank=cfg["task_rank"], ard=cfg["ard"],
                 num_probes=cfg["num_probes"], max_cg_iterations=cfg["max_cg_iter"],
                 cg_tolerance=cfg["cg_tol"], use_preconditioner=cfg["use_preconditioner"],
                 preconditioner_rank=cfg["precond_rank"], preconditioner=cfg["precond"],
                 precond_rebuild_threshold=cfg["precond_rebuild_threshold"])
        gp.method = cfg["method"]
        gp._X_train = np.ascontiguousarray(arr["X_train"], np.float32)
        gp._Y_train = np.ascontiguousarray(arr["Y_train"], np.float32)
        get = lambda k: arr[k] if k in arr else None  # noqa: E731
        obs = get("observation_noise_train")
        gp._observation_noise_train = None if obs is None else np.ascontiguousarray(obs,
                                                                                    np.float32)
        grp = get("noise_group_train")
        gp._noise_group_train = None if grp is None else np.ascontiguousarray(grp, np.int32)
        gv = get("group_noise")
        gp._noise_group_values = None if gv is None else np.ascontiguousarray(gv, np.float32)
        gp._dim = cfg.get("dim")
        gp._training_method = cfg.get("training_method", gp.method)
        d = gp._X_train.shape[1]
        if gp._is_mixed:
            if "cat_params" not in arr:
                raise ValueError("mixed MultiOutputGP artifact is missing cat_params")
            (gp._cat_specs, gp._cat_cols, gp._cont_cols,
             gp._cat_names) = _mixed_layout(gp._original_kernel, gp._X_train)
            gp._cat_params_raw = np.ascontiguousarray(arr["cat_params"], np.float32)
            d = len(gp._cont_cols)
        gp._compiled_kernel = (make_ard_kernel(gp._original_kernel, d) if gp.ard
                               else gp._original_kernel)
        gp.kernel = gp._compiled_kernel
        gp._result = MultiOutputTrainingResult(
            params=np.asarray(arr["params"], np.float32), noise=float(cfg["noise"]),
            noise_per_task=np.asarray(arr["noise_per_task"], np.float32),
            final_nll=float(cfg["final_nll"]), iterations=int(cfg["iterations"]),
            converged=bool(cfg["converged"]), num_tasks=int(cfg["num_tasks"]),
            task_rank=int(cfg["task_rank_result"]),
            num_kernel_params=int(cfg["num_kernel_params"]),
            B=np.asarray(arr["B"], np.float32), Q=np.asarray(arr["Q"], np.float32),
            Lambda=np.asarray(arr["Lambda"], np.float32),
            effective_scales=np.asarray(arr["effective_scales"], np.float32),
            W=arr["W"], raw_v=arr["raw_v"],
            alpha_rotated=np.asarray(arr["alpha_rotated"], np.float32),
            mean_per_task=np.asarray(arr["mean_per_task"], np.float32),
            nll_history=arr["nll_history"], param_names=list(cfg["param_names"]),
            cat_params=gp._cat_params_raw,
            cat_param_names=list(cfg.get("cat_param_names", [])),
            iter_times_ms=get("iter_times_ms"))
        fm = get("fitted_mean")
        gp._fitted_mean = np.asarray(fm if fm is not None else arr["mean_per_task"], np.float32)
        gp._is_trained = True
        gp._backend_train_info = None
        return gp

    def __repr__(self) -> str:
        status = "trained" if self._is_trained else "untrained"
        tasks = f", tasks={self.num_tasks}" if self.num_tasks else ""
        ard = ", ard=True" if self.ard else ""
        return f"MultiOutputGP(kernel={self._original_kernel.to_mojo_type()}{tasks}{ard}, {status})"
