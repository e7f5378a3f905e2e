"""Pins of the learned per-sample noise restatement (oracle.engine
learned_noise_vector / learned_noise_grad / bbmm_step rowdot).

The gradient chain of every mode is checked against central finite
differences of the dense objective n * NLL(K + diag(noise(raw))) / n plus the
regulariser whose derivative the reference adds (reg log(noise/target)^2 /
(2 count), weight decay reg w^2 / (2 d) for the linear mode), with the exact
diagonal of the inverse in place of the probe estimate; the probe estimate
itself converges to that diagonal."""

import numpy as np
import pytest

from oracle import engine as oe
from oracle import kernels as ok


def _setup(n=24, d=2, seed=0):
    rng = np.random.default_rng(seed)
    X = rng.uniform(-1, 1, (n, d))
    y = np.sin(2 * X[:, 0]) + 0.1 * rng.normal(size=n)
    K = ok.kernel_matrix(ok.RBF, X, X, [0.7, 1.1], False)
    return X, y, K


def _objective(K, y, noise, reg, target, count_for_reg, extra=0.0):
    A = K + np.diag(noise)
    n = len(y)
    _, logdet = np.linalg.slogdet(A)
    nll = 0.5 * y @ np.linalg.solve(A, y) + 0.5 * logdet
    r = reg * np.sum(np.log(noise / target) ** 2) / (2 * count_for_reg)
    return nll / n + r + extra


def _exact_rowdot(K, y, noise):
    A = K + np.diag(noise)
    Ai = np.linalg.inv(A)
    a = Ai @ y
    return 0.5 * (np.diag(Ai) - a * a)


def _sp(x):
    return np.logaddexp(0.0, x)


@pytest.mark.parametrize("mode", [2, 3, 4])
def test_learned_noise_gradient_matches_finite_differences(mode):
    X, y, K = _setup()
    n, d = X.shape
    floor, reg, target = 1e-4, 0.05, 0.08
    rng = np.random.default_rng(mode)
    groups = np.arange(n) % 3
    if mode == 2:
        raw = rng.normal(-2.5, 0.3, n)
    elif mode == 3:
        raw = rng.normal(-2.5, 0.3, 3)
    else:
        raw = np.array([-2.5, 0.4, -0.3])

    def noise_of(r):
        if mode == 2:
            return _sp(r) + floor
        if mode == 3:
            return _sp(r[groups]) + floor
        return _sp(r[0] + X @ r[1:]) + floor

    def J(r):
        nz = noise_of(r)
        if mode == 3:
            gv = _sp(r) + floor      # the regulariser acts on group values
            A = K + np.diag(nz)
            _, ld = np.linalg.slogdet(A)
            nll = (0.5 * y @ np.linalg.solve(A, y) + 0.5 * ld) / n
            return nll + reg * np.sum(np.log(gv / target) ** 2) / (2 * 3)
        wd = reg * np.sum(r[1:] ** 2) / (2 * d) if mode == 4 else 0.0
        return _objective(K, y, nz, reg, target, n, wd)

    rd = _exact_rowdot(K, y, noise_of(raw))
    g = oe.learned_noise_grad(mode, raw, rd, floor, reg, target, groups, X)
    fd = np.zeros_like(raw)
    for k in range(raw.size):
        h = 1e-6
        rp, rm = raw.copy(), raw.copy()
        rp[k] += h
        rm[k] -= h
        fd[k] = (J(rp) - J(rm)) / (2 * h)
    np.testing.assert_allclose(g, fd, rtol=1e-5, atol=1e-9)


def test_noise_vector_from_state():
    X, _, _ = _setup()
    raw = np.array([-1.0, 0.5, 2.0], np.float32)
    v = oe.learned_noise_vector(4, raw, 1e-3, X=X)
    ref = np.logaddexp(0.0, -1.0 + X.astype(np.float32) @ raw[1:]) + 1e-3
    np.testing.assert_allclose(v, ref, rtol=1e-5)   # fp32 state, fp64 reference
    g = np.array([0, 2, 1, 2])
    np.testing.assert_allclose(oe.learned_noise_vector(3, raw, 0.0, groups=g),
                               np.logaddexp(0.0, raw[g]), rtol=1e-6)


def test_probe_rowdot_estimates_exact_diagonal():
    """The probe estimate (0.5/T) sum_j (A^-1 z_j)_i (z_j)_i converges to
    0.5 diag(A^-1)_i; with T = 4000 probes the error is a few percent."""
    X, y, K = _setup(n=30)
    noise = np.full(30, 0.1)
    A = K + np.diag(noise)
    r = oe.bbmm_step(ok.RBF, False, X, y, [0.7, 1.1], 0.0, None, 4000, 200, 0, 1e-10, 0,
                     noise_vec=noise)
    exact = _exact_rowdot(K, y, noise)
    assert np.abs(r["rowdot"] - exact).max() <= 0.05 * np.abs(exact).max()
