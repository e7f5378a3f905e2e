"""Random-Fourier-feature prior draws for pathwise posterior sampling.

The feature map of a stationary leaf follows mojogp/pathwise_prior.py:130-160
and :459-499: frequencies W [F, d] are standard normal for RBF and
independent Student-t with 5 degrees of freedom per dimension for Matern-5/2,
phases are uniform on [0, 2 pi), both drawn from the caller's NumPy Generator
in that order, and

    phi_f(x) = sqrt(os) sqrt(2 / F) cos((x / l) . W_f + phase_f).

Drawing uses the same Generator calls in the same order as the reference, so a
seeded run draws the same features and weights.  The evaluation
``weights @ phi(X)^T`` (n x F features, K draws) runs on the device in fp64
through ``mgp_rff_prior_values``; there is no host fallback.

For d > 1 the per-dimension t draws make the Matern-5/2 feature covariance the
product of one-dimensional Matern-5/2 kernels rather than the isotropic one;
this is the reference's construction and is kept as is.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import _lib
from ._provider import KIND_MATERN12, KIND_MATERN32, KIND_MATERN52, KIND_RBF


@dataclass(frozen=True)
class PathwiseFeatureMap:
    """Stationary RFF map of one latent kernel."""

    kind: int
    lengthscales: np.ndarray  # [d] float64
    outputscale: float
    W: np.ndarray             # [F, d] float64
    phase: np.ndarray         # [F] float64

    @property
    def size(self) -> int:
        return int(self.W.shape[0])


def build_pathwise_feature_map(kind: int, params, *, input_dim: int, n_features: int,
                               rng: np.random.Generator, ard: bool) -> PathwiseFeatureMap:
    """Feature map of an RBF / Matern leaf with public params [ls..., os]
    (pathwise_prior.py:130-160: Gaussian frequencies for RBF, Student-t with
    2 nu degrees of freedom per dimension for Matern-nu)."""
    p = np.asarray(params, dtype=np.float64).ravel()
    d = int(input_dim)
    if ard:
        if p.shape[0] != d + 1:
            raise ValueError(f"expected {d + 1} ARD params, got {p.shape[0]}")
        ls = p[:d].copy()
    else:
        if p.shape[0] != 2:
            raise ValueError(f"expected 2 params, got {p.shape[0]}")
        ls = np.full(d, float(p[0]))
    outputscale = float(p[-1])
    if kind == KIND_RBF:
        W = rng.standard_normal((n_features, d))
    elif kind == KIND_MATERN12:
        W = rng.standard_t(df=1, size=(n_features, d))
    elif kind == KIND_MATERN32:
        W = rng.standard_t(df=3, size=(n_features, d))
    elif kind == KIND_MATERN52:
        W = rng.standard_t(df=5, size=(n_features, d))
    else:
        raise ValueError(f"unsupported kernel kind {kind} for pathwise features")
    phase = rng.uniform(0.0, 2.0 * np.pi, size=n_features)
    return PathwiseFeatureMap(kind, ls, outputscale, np.ascontiguousarray(W, np.float64),
                              np.ascontiguousarray(phase, np.float64))


def build_feature_weights(feature_map: PathwiseFeatureMap, n_draws: int,
                          rng: np.random.Generator) -> np.ndarray:
    """Standard normal weights [n_draws, F] (float32, as the reference)."""
    return rng.standard_normal((n_draws, feature_map.size)).astype(np.float32)


def sample_prior_values(feature_map: PathwiseFeatureMap, X: np.ndarray,
                        weights: np.ndarray) -> np.ndarray:
    """Prior draws [K, n] = weights @ phi(X)^T, evaluated on the device (fp64,
    returned as float32)."""
    X = _lib.f32(X)
    if X.ndim != 2 or X.shape[1] != feature_map.lengthscales.shape[0]:
        raise ValueError("X must have shape (n, d) matching the feature map")
    w = np.ascontiguousarray(np.atleast_2d(weights), dtype=np.float64)
    if w.shape[1] != feature_map.size:
        raise ValueError("weights must have one column per feature")
    n, d = X.shape
    K = w.shape[0]
    out = np.zeros((K, n), dtype=np.float32)
    ls = np.ascontiguousarray(feature_map.lengthscales, np.float64)
    _lib.call("mgp_rff_prior_values", _lib.fptr(X), n, d, _lib.dptr(ls),
              _lib.dptr(feature_map.W), _lib.dptr(feature_map.phase), feature_map.size,
              float(feature_map.outputscale), _lib.dptr(w), K, _lib.fptr(out))
    return out
