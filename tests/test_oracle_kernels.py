"""Pins the float64 kernel oracle (oracle/kernels.py) against independent facts:
scikit-learn kernels, the reference's clamp guards, SymPy derivatives and finite
differences.  CPU only."""

import numpy as np
import pytest

from oracle import kernels as ok


def _sk_kernel(kind, ls):
    from sklearn.gaussian_process.kernels import RBF, Matern
    if kind == ok.RBF:
        return RBF(length_scale=ls)
    nu = {ok.MATERN12: 0.5, ok.MATERN32: 1.5, ok.MATERN52: 2.5}[kind]
    return Matern(length_scale=ls, nu=nu)


@pytest.mark.parametrize("kind", ok.KINDS)
@pytest.mark.parametrize("ard", [False, True])
def test_matches_sklearn_in_unclamped_region(kind, ard, rng):
    d = 4
    X1 = rng.uniform(-1, 1, size=(30, d))
    X2 = rng.uniform(-1, 1, size=(25, d))
    ls = rng.uniform(0.5, 2.0, size=d) if ard else np.array([0.9])
    os = 1.7
    params = np.concatenate([ls, [os]])
    K = ok.kernel_matrix(kind, X1, X2, params, ard)
    sk = _sk_kernel(kind, ls if ard else float(ls[0]))(X1, X2) * os
    np.testing.assert_allclose(K, sk, rtol=1e-10, atol=1e-13)


def test_rbf_clamp_tail_is_exact_e_minus_20():
    # 0.5 r^2 = 50 > 20: the reference clamps the exponent to -20.
    X1 = np.zeros((1, 2))
    X2 = np.array([[10.0, 0.0]])
    K = ok.kernel_matrix(ok.RBF, X1, X2, [1.0, 2.5], False)
    assert K[0, 0] == pytest.approx(2.5 * np.exp(-20.0), rel=1e-14)


def test_matern_clamp_tail_keeps_polynomial():
    # sqrt5 r = 30 > 20: exp clamps at -20 but the polynomial still grows.
    r = 30.0 / np.sqrt(5.0)
    X1 = np.zeros((1, 1))
    X2 = np.array([[r]])
    K = ok.kernel_matrix(ok.MATERN52, X1, X2, [1.0, 1.0], False)
    expect = (1 + 30.0 + (5.0 / 3.0) * r * r) * np.exp(-20.0)
    assert K[0, 0] == pytest.approx(expect, rel=1e-12)


@pytest.mark.parametrize("kind", ok.KINDS)
def test_diagonal_is_outputscale(kind, rng):
    X = rng.normal(size=(10, 3))
    K = ok.kernel_matrix(kind, X, X, [0.7, 0.3, 1.1, 2.0], True)
    np.testing.assert_allclose(np.diag(K), 2.0, rtol=1e-9)


@pytest.mark.parametrize("kind", ok.KINDS)
@pytest.mark.parametrize("ard", [False, True])
def test_gradients_match_finite_differences(kind, ard, rng):
    d = 3
    X1 = rng.uniform(-1, 1, size=(8, d))
    X2 = rng.uniform(-1, 1, size=(7, d))
    params = np.concatenate([rng.uniform(0.6, 1.5, size=d if ard else 1), [1.3]])
    G = ok.kernel_gradients(kind, X1, X2, params, ard)
    assert G.shape == (params.size, 8, 7)
    h = 1e-6
    for p in range(params.size):
        up = params.copy(); up[p] += h
        dn = params.copy(); dn[p] -= h
        fd = (ok.kernel_matrix(kind, X1, X2, up, ard) - ok.kernel_matrix(kind, X1, X2, dn, ard)) / (2 * h)
        np.testing.assert_allclose(G[p], fd, rtol=1e-6, atol=1e-9)


def test_matern_gradient_matches_sympy():
    sp = pytest.importorskip("sympy")
    l0, l1, os, a0, a1 = sp.symbols("l0 l1 os a0 a1", positive=True)
    r = sp.sqrt((a0 / l0) ** 2 + (a1 / l1) ** 2)
    k = os * (1 + sp.sqrt(5) * r + sp.Rational(5, 3) * r**2) * sp.exp(-sp.sqrt(5) * r)
    vals = {l0: 0.8, l1: 1.3, os: 1.7, a0: 0.4, a1: -0.9}
    X1 = np.array([[0.4, -0.9]])
    X2 = np.zeros((1, 2))
    G = ok.kernel_gradients(ok.MATERN52, X1, X2, [0.8, 1.3, 1.7], True)
    for p, sym in enumerate([l0, l1, os]):
        ref = float(sp.diff(k, sym).subs(vals))
        assert G[p, 0, 0] == pytest.approx(ref, rel=1e-12)


@pytest.mark.parametrize("kind,nu_k", [(ok.MATERN12, "exp"), (ok.MATERN32, "m32")])
def test_low_order_matern_gradient_matches_sympy(kind, nu_k):
    """Matern-1/2 and 3/2 lengthscale derivatives of the forward expressions
    with the reference's r = sqrt(sum (a/l)^2 + 1e-20), as SymPy gives them."""
    sp = pytest.importorskip("sympy")
    l0, l1, os, a0, a1 = sp.symbols("l0 l1 os a0 a1", positive=True)
    r = sp.sqrt((a0 / l0) ** 2 + (a1 / l1) ** 2 + sp.Float(1e-20))
    if nu_k == "exp":
        k = os * sp.exp(-r)
    else:
        k = os * (1 + sp.sqrt(3) * r) * sp.exp(-sp.sqrt(3) * r)
    vals = {l0: 0.8, l1: 1.3, os: 1.7, a0: 0.4, a1: -0.9}
    G = ok.kernel_gradients(kind, np.array([[0.4, -0.9]]), np.zeros((1, 2)), [0.8, 1.3, 1.7], True)
    for p, sym in enumerate([l0, l1, os]):
        assert G[p, 0, 0] == pytest.approx(float(sp.diff(k, sym).subs(vals)), rel=1e-12)
    # coincident points: finite (the floored r), zero lengthscale derivative
    G0 = ok.kernel_gradients(kind, np.zeros((1, 2)), np.zeros((1, 2)), [0.8, 1.3, 1.7], True)
    assert np.all(np.isfinite(G0)) and G0[0, 0, 0] == 0.0
    assert G0[2, 0, 0] == pytest.approx(1.0, abs=1e-9)


def test_forward_matvec_matches_dense(rng):
    X = rng.normal(size=(60, 5))
    V = rng.normal(size=(3, 60))
    params = [0.9, 1.1, 0.8, 1.2, 1.0, 1.4]
    K = ok.kernel_matrix(ok.MATERN52, X, X, params, True)
    out = ok.forward_matvec(ok.MATERN52, X, V, params, 0.05, True, block=17)
    np.testing.assert_allclose(out, V @ K.T + 0.05 * V, rtol=1e-12)
    rows = np.array([3, 17, 59])
    part = ok.forward_matvec(ok.MATERN52, X, V, params, 0.05, True, rows=rows)
    np.testing.assert_allclose(part, out[:, rows], rtol=1e-12)


def test_gradient_matvec_layout(rng):
    X = rng.normal(size=(12, 2))
    V = rng.normal(size=(2, 12))
    params = [0.9, 1.2, 1.5]
    G = ok.kernel_gradients(ok.RBF, X, X, params, True)
    out = ok.gradient_matvec(ok.RBF, X, V, params, True)
    for p in range(3):
        np.testing.assert_allclose(out[p], V @ G[p].T, rtol=1e-12)
