"""Pins of the composite-kernel-tree restatement (oracle.kernels.TreeKernel)
and of the host-side tree compiler (KernelNode.to_tree_spec / evaluate).

Independent checks: scikit-learn kernels for every leaf family (RBF, Matern
nu = 1/2, 3/2, 5/2, RationalQuadratic, ExpSineSquared), Sum / Product /
ConstantKernel compositions on column slices, scikit-learn's analytic
log-parameter gradients, and central finite differences of the tree gradients."""

import numpy as np
import pytest
from sklearn.gaussian_process import kernels as sk

from mojogp_amd import (RBF, RQ, Linear, Matern12, Matern32, Matern52, Periodic, Polynomial,
                        make_ard_kernel)
from mojogp_amd.kernel import KernelNode
from oracle import kernels as ok


def _tree(node: KernelNode, d: int) -> ok.TreeKernel:
    return ok.TreeKernel(node.to_dict(), d)


def _rng_X(seed, n, d, scale=1.0):
    return np.random.default_rng(seed).normal(scale=scale, size=(n, d))


@pytest.mark.parametrize("node,skk", [
    (RBF(), lambda l: sk.RBF(l)),
    (Matern12(), lambda l: sk.Matern(l, nu=0.5)),
    (Matern32(), lambda l: sk.Matern(l, nu=1.5)),
    (Matern52(), lambda l: sk.Matern(l, nu=2.5)),
])
def test_radial_leaves_match_sklearn(node, skk):
    X = _rng_X(0, 30, 3)
    Y = _rng_X(1, 20, 3)
    T = _tree(node, 3)
    K = T.matrix(X, Y, [1.3, 0.7])
    np.testing.assert_allclose(K, 0.7 * skk(1.3)(X, Y), rtol=1e-12, atol=1e-14)


def test_rq_leaf_matches_sklearn():
    X, Y = _rng_X(2, 25, 2), _rng_X(3, 15, 2)
    T = _tree(RQ(), 2)
    K = T.matrix(X, Y, [0.9, 2.5, 1.7])
    ref = 1.7 * sk.RationalQuadratic(length_scale=0.9, alpha=2.5)(X, Y)
    np.testing.assert_allclose(K, ref, rtol=1e-12)
    # ARD: sklearn's isotropic RQ on inputs pre-divided by the lengthscales
    ls = np.array([0.6, 1.8])
    Ta = _tree(make_ard_kernel(RQ(), 2), 2)
    Ka = Ta.matrix(X, Y, [*ls, 0.8, 1.1])
    refa = 1.1 * sk.RationalQuadratic(length_scale=1.0, alpha=0.8)(X / ls, Y / ls)
    np.testing.assert_allclose(Ka, refa, rtol=1e-12)


def test_periodic_leaf_matches_sklearn():
    """The engine divides the summed sin^2 terms by the lengthscale itself
    (codegen_engine/expressions.py:242-285), i.e. sklearn's ExpSineSquared
    with length_scale = sqrt(l); over several dimensions the sum becomes a
    product of per-dimension ExpSineSquared kernels."""
    X, Y = _rng_X(4, 20, 2, 2.0), _rng_X(5, 18, 2, 2.0)
    l, per, os = 1.6, 2.3, 0.9
    K = _tree(Periodic(), 2).matrix(X, Y, [l, per, os])
    ref = os * np.ones((20, 18))
    for q in range(2):
        ref *= sk.ExpSineSquared(length_scale=np.sqrt(l), periodicity=per)(X[:, [q]], Y[:, [q]])
    np.testing.assert_allclose(K, ref, rtol=1e-11)
    ls = np.array([0.7, 2.2])
    Ka = _tree(make_ard_kernel(Periodic(), 2), 2).matrix(X, Y, [*ls, per, os])
    refa = os * np.ones((20, 18))
    for q in range(2):
        refa *= sk.ExpSineSquared(length_scale=np.sqrt(ls[q]), periodicity=per)(X[:, [q]],
                                                                               Y[:, [q]])
    np.testing.assert_allclose(Ka, refa, rtol=1e-11)


def test_composition_on_active_dims_matches_sklearn():
    X, Y = _rng_X(6, 24, 4), _rng_X(7, 11, 4)
    node = (RBF(active_dims=[0]) + 2.0 * Matern52(active_dims=[1, 3])) * RQ(active_dims=[2])
    p = np.array([1.2, 0.8, 0.9, 1.4, 2.0, 0.7, 1.5, 1.3])
    K = _tree(node, 4).matrix(X, Y, p)
    a = 0.8 * sk.RBF(1.2)(X[:, [0]], Y[:, [0]])
    b = 2.0 * 1.4 * sk.Matern(0.9, nu=2.5)(X[:, [1, 3]], Y[:, [1, 3]])
    c = 1.3 * sk.RationalQuadratic(0.7, 1.5)(X[:, [2]], Y[:, [2]])
    np.testing.assert_allclose(K, (a + b) * c, rtol=1e-12)
    # a composite's active_dims restrict every leaf inside it
    node2 = (RBF() * Periodic()).with_active_dims([1, 2]) + Matern32(active_dims=[0])
    p2 = np.array([1.1, 0.9, 0.6, 2.0, 1.2, 0.8, 0.5])
    K2 = _tree(node2, 4).matrix(X, Y, p2)
    cols = [1, 2]
    per = 1.2 * np.ones((24, 11))
    for q in cols:
        per *= sk.ExpSineSquared(np.sqrt(0.6), 2.0)(X[:, [q]], Y[:, [q]])
    ref2 = 0.9 * sk.RBF(1.1)(X[:, cols], Y[:, cols]) * per + 0.5 * sk.Matern(
        0.8, nu=1.5)(X[:, [0]], Y[:, [0]])
    np.testing.assert_allclose(K2, ref2, rtol=1e-12)


def test_rq_gradients_match_sklearn_log_gradients():
    X = _rng_X(8, 15, 2)
    l, a, os = 0.9, 1.7, 1.3
    # d/dlog theta, hyperparameters in name order: alpha, then length_scale
    _, G = sk.RationalQuadratic(length_scale=l, alpha=a)(X, eval_gradient=True)
    Gt = _tree(RQ(), 2).gradients(X, X, [l, a, os])
    np.testing.assert_allclose(Gt[0] * l, os * G[:, :, 1], rtol=1e-10, atol=1e-13)
    np.testing.assert_allclose(Gt[1] * a, os * G[:, :, 0], rtol=1e-10, atol=1e-13)


def test_periodic_gradients_match_sklearn_log_gradients():
    X = _rng_X(9, 15, 1, 2.0)
    l, per, os = 1.4, 1.9, 0.8
    _, G = sk.ExpSineSquared(length_scale=np.sqrt(l), periodicity=per)(X, eval_gradient=True)
    Gt = _tree(Periodic(), 1).gradients(X, X, [l, per, os])
    # d/dlog(sqrt l) = 2 d/dlog l
    np.testing.assert_allclose(Gt[0] * l * 2.0, os * G[:, :, 0], rtol=1e-10, atol=1e-13)
    np.testing.assert_allclose(Gt[1] * per, os * G[:, :, 1], rtol=1e-10, atol=1e-13)


TREES = [
    lambda: RBF(active_dims=[0]) * Periodic(active_dims=[1]) + RQ(active_dims=[0, 2]),
    lambda: 1.5 * (Matern52() + Matern12(active_dims=[2])) * Matern32(active_dims=[1]),
    lambda: make_ard_kernel(RQ() * Periodic(active_dims=[0, 1]) + 0.5 * RBF(), 3),
]


@pytest.mark.parametrize("mk", TREES)
def test_tree_gradients_match_finite_differences(mk):
    node = mk()
    T = _tree(node, 3)
    rng = np.random.default_rng(10)
    X, Y = rng.uniform(-1, 1, (12, 3)), rng.uniform(-1, 1, (9, 3))
    p = rng.uniform(0.6, 1.6, T.nparams)
    G = T.gradients(X, Y, p)
    assert G.shape == (T.nparams, 12, 9)
    for q in range(T.nparams):
        h = 1e-6 * p[q]
        pp, pm = p.copy(), p.copy()
        pp[q] += h
        pm[q] -= h
        fd = (T.matrix(X, Y, pp) - T.matrix(X, Y, pm)) / (2 * h)
        np.testing.assert_allclose(G[q], fd, rtol=2e-6, atol=1e-8)


@pytest.mark.parametrize("mk", TREES)
def test_host_evaluate_matches_oracle(mk):
    node = mk()
    T = _tree(node, 3)
    rng = np.random.default_rng(11)
    X = rng.normal(size=(16, 3))
    p = rng.uniform(0.6, 1.6, T.nparams)
    assert node.num_params() == T.nparams
    np.testing.assert_allclose(node.evaluate(X, params=p), T.matrix(X, X, p), rtol=2e-6)
    assert T.diag(p) == pytest.approx(float(T.matrix(X[:1], X[:1], p)[0, 0]), rel=1e-12)


def test_tree_spec_layout():
    node = (RBF(active_dims=[0]) + 2.0 * Matern52(active_dims=[1, 2])) * RQ()
    spec = node.to_tree_spec(3)
    # header, leaves (code, ard, ndim, p0, dims), nodes (code, a, b; root last)
    assert spec == [3, 8, 3, 6,
                    0, 0, 1, 0, 0,
                    1, 0, 2, 2, 1, 2,
                    4, 0, 3, 5, 0, 1, 2,
                    0, 0, 0,
                    0, 1, 0,
                    3, 1, 4,
                    1, 0, 2,
                    0, 2, 0,
                    2, 3, 4]
    ard = make_ard_kernel(node, 3)
    s = ard.to_tree_spec(3)
    assert s[:4] == [3, 11, 3, 6]
    assert s[4:9] == [0, 1, 1, 0, 0]          # RBF ARD on [0]: 1 ls at p0 = 0
    assert s[9:15] == [1, 1, 2, 2, 1, 2]      # Matern52 ARD on [1, 2] at p0 = 2
    assert s[15:22] == [4, 1, 3, 6, 0, 1, 2]  # RQ ARD: 3 ls, alpha, os at p0 = 6


def test_tree_spec_rejects_unserved():
    with pytest.raises(ValueError):    # non-integer polynomial degree
        Polynomial(degree=2.5).to_tree_spec(2)
    with pytest.raises(ValueError):
        RBF(active_dims=[3]).to_tree_spec(2)
    with pytest.raises(NotImplementedError):
        node = RBF()
        for _ in range(8):
            node = node + RBF()
        node.to_tree_spec(2)


def test_linear_and_polynomial_leaves_match_sklearn():
    """Linear os*var*x.x' and polynomial os*(var*x.x' + offset)^D against
    scikit-learn's DotProduct (sigma_0 = 0, resp. sqrt(offset)) and its
    Exponentiation; the engine's polynomial layout carries a hidden variance
    and an unread degree slot (kernel.py:462-606)."""
    X, Y = _rng_X(12, 14, 3), _rng_X(13, 9, 3)
    K = _tree(Linear(), 3).matrix(X, Y, [0.7, 1.3])
    np.testing.assert_allclose(K, 1.3 * 0.7 * sk.DotProduct(sigma_0=0.0)(X, Y), rtol=1e-12)
    T = _tree(Polynomial(degree=3), 3)
    assert T.nparams == 4
    K = T.matrix(X, Y, [1.0, 2.7, 0.5, 1.2])   # degree slot 2.7 is not read
    ref = 1.2 * sk.Exponentiation(sk.DotProduct(sigma_0=np.sqrt(0.5)), 3)(X, Y)
    np.testing.assert_allclose(K, ref, rtol=1e-12)
    node = Polynomial(degree=2) * RBF()
    p_pub = np.array([2.0, 0.4, 1.1, 0.9, 1.3])
    np.testing.assert_allclose(node.evaluate(X, Y, p_pub),
                               _tree(node, 3).matrix(X, Y, node.to_engine_params(p_pub)),
                               rtol=2e-6)


@pytest.mark.parametrize("mk", [
    lambda: Linear() * RBF() + Polynomial(degree=2),
    lambda: make_ard_kernel(Linear(ard=True), 3),
    lambda: make_ard_kernel(Polynomial(degree=3, ard=True), 3),
])
def test_nonstationary_gradients_match_finite_differences(mk):
    node = mk()
    T = _tree(node, 3)
    rng = np.random.default_rng(14)
    X, Y = rng.uniform(-1, 1, (10, 3)), rng.uniform(-1, 1, (8, 3))
    p = rng.uniform(0.6, 1.4, T.nparams)
    G = T.gradients(X, Y, p)
    for q in range(T.nparams):
        h = 1e-6 * p[q]
        pp, pm = p.copy(), p.copy()
        pp[q] += h
        pm[q] -= h
        fd = (T.matrix(X, Y, pp) - T.matrix(X, Y, pm)) / (2 * h)
        np.testing.assert_allclose(G[q], fd, rtol=2e-6, atol=1e-8)
