"""float64 restatement of the categorical correlation kernels (test infrastructure).

Reference semantics (caspbian/mojogp):
  * GD   R_ij = exp(-theta) (i != j), 1 on the diagonal
         (kernels/categorical_kernel.mojo:33-57)
  * CR   R_ij = exp(-(theta_i + theta_j)) (i != j), 1 on the diagonal (:86-108)
  * hypersphere factor C from L(L-1)/2 angles in lower-triangular row order
    (1,0), (2,0), (2,1), ...: C[0,0] = 1, C[k,c] = cos(t_kc) prod_{m<c} sin(t_km),
    C[k,k] = prod_{m<k} sin(t_km)  (:143-205)
  * EHH  R_ij = exp(h (1 - (C C^T)_ij)) (i != j), h = log(1e-12) / 2  (:212-252)
  * HH   R = C C^T  (:410-437)
  * FE   angles then L diagonal parameters d:
         R_ij = exp(-(d_i + d_j + h ((C C^T)_ij - 1))) (i != j)  (:476-521)
  * raw -> constrained parameters: GD, CR and FE's d through softplus; EHH,
    HH and FE angles through pi * sigmoid (kernels/jit/jit_categorical_params.mojo:33-64)
  * default raw values: GD softplus^-1(0.5), CR softplus^-1(0.3), angles
    sigmoid^-1(0.25), FE d softplus^-1(0.3) (mojogp/kernel.py:84-101)

Derivatives dR/dtheta are central finite differences of these float64
formulas (step 1e-6 relative); pinned in tests/test_oracle_categorical.py by
closed forms (GD, CR), unit diagonals, symmetry, positive semi-definiteness
of the hypersphere matrices and the reference's default initialisation.
"""

from __future__ import annotations

import numpy as np

GD, CR, EHH, HH, FE = 0, 1, 2, 3, 4
NAMES = {"gd": GD, "cr": CR, "ehh": EHH, "hh": HH, "fe": FE}
_H = np.log(1e-12) / 2.0


def num_params(kind: int, L: int) -> int:
    return {GD: 1, CR: L, EHH: L * (L - 1) // 2, HH: L * (L - 1) // 2,
            FE: L * (L + 1) // 2}[kind]


def _is_angle(kind: int, L: int, k: int) -> bool:
    return kind in (EHH, HH) or (kind == FE and k < L * (L - 1) // 2)


def _sp(x):
    return np.logaddexp(0.0, x)


def _sig(x):
    return 1.0 / (1.0 + np.exp(-x))


def constrain(kind: int, L: int, raw) -> np.ndarray:
    raw = np.asarray(raw, np.float64)
    return np.array([np.pi * _sig(r) if _is_angle(kind, L, k) else _sp(r)
                     for k, r in enumerate(raw)])


def chain_derivative(kind: int, L: int, raw) -> np.ndarray:
    """d(constrained)/d(raw) per parameter."""
    raw = np.asarray(raw, np.float64)
    return np.array([np.pi * _sig(r) * (1 - _sig(r)) if _is_angle(kind, L, k) else _sig(r)
                     for k, r in enumerate(raw)])


def default_raw(kind: int, L: int) -> np.ndarray:
    def inv_sp(y):
        return np.log(np.expm1(y))

    def inv_sig(y):
        return np.log(y / (1 - y))

    return np.array([inv_sig(0.25) if _is_angle(kind, L, k)
                     else inv_sp(0.5 if kind == GD else 0.3)
                     for k in range(num_params(kind, L))])


def hypersphere_factor(angles, L: int) -> np.ndarray:
    C = np.zeros((L, L))
    C[0, 0] = 1.0
    idx = 0
    for k in range(1, L):
        s = 1.0
        for c in range(k):
            t = angles[idx]
            idx += 1
            C[k, c] = np.cos(t) * s
            s *= np.sin(t)
        C[k, k] = s
    return C


def correlation(kind: int, L: int, theta) -> np.ndarray:
    theta = np.asarray(theta, np.float64)
    off = ~np.eye(L, dtype=bool)
    R = np.eye(L)
    if kind == GD:
        R[off] = np.exp(-theta[0])
    elif kind == CR:
        E = np.exp(-(theta[:, None] + theta[None, :]))
        R[off] = E[off]
    else:
        na = L * (L - 1) // 2
        C = hypersphere_factor(theta[:na], L)
        D = C @ C.T
        if kind == HH:
            return D
        if kind == EHH:
            R[off] = np.exp(_H * (1.0 - D))[off]
        else:
            d = theta[na:]
            R[off] = np.exp(-(d[:, None] + d[None, :] + _H * (D - 1.0)))[off]
    return R


def correlation_gradients(kind: int, L: int, theta) -> np.ndarray:
    """dR/dtheta_k for every constrained parameter, shape (K, L, L)."""
    theta = np.asarray(theta, np.float64)
    out = np.zeros((theta.size, L, L))
    for k in range(theta.size):
        h = 1e-6 * max(abs(theta[k]), 1.0)
        tp, tm = theta.copy(), theta.copy()
        tp[k] += h
        tm[k] -= h
        out[k] = (correlation(kind, L, tp) - correlation(kind, L, tm)) / (2 * h)
    return out
