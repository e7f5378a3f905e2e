"""GPU parity of composite kernel trees (sums, products and scales of RBF,
Matern, RQ and periodic leaves on dimension subsets) against the float64
tree restatement: forward / cross products on the direct and materialized
routes, pivoted Cholesky, one BBMM evaluation (NLL and every tree-parameter
gradient), a fit on the restatement's trajectory, prediction and
persistence.  Bars as for single kernels: products 1e-5, NLL / mean / std
1e-4."""

import ctypes as C

import numpy as np
import pytest

from mojogp_amd import (RBF, RQ, Linear, Matern12, Matern32, Matern52, Periodic, Polynomial,
                        make_ard_kernel)
from mojogp_amd import _lib
from mojogp_amd._provider import NativeProvider
from oracle import engine as oe
from oracle import kernels as ok

pytestmark = pytest.mark.gpu


def _rel(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


TREES = {
    "rbf+m52": (lambda: RBF() + Matern52(), 3),
    "rbf[0]*m32[1]": (lambda: RBF(active_dims=[0]) * Matern32(active_dims=[1]), 2),
    "2*rbf_ard": (lambda: make_ard_kernel(2.0 * RBF(ard=True), 4), 4),
    "rq_ard+per[1]": (lambda: make_ard_kernel(RQ(ard=True), 3) + Periodic(active_dims=[1]), 3),
    "(m12+rbf[2])*per": (lambda: (Matern12(active_dims=[0, 1]) + RBF(active_dims=[2]))
                         * Periodic(period=2.0), 3),
}


def _setup(name, n, seed):
    mk, d = TREES[name]
    node = mk()
    rng = np.random.default_rng(seed)
    X = rng.uniform(-2, 2, size=(n, d)).astype(np.float32)
    T = ok.TreeKernel(node.to_dict(), d)
    params = rng.uniform(0.6, 1.5, T.nparams).astype(np.float32)
    return node, T, X, params, rng


@pytest.mark.parametrize("name", list(TREES))
def test_tree_products_match_oracle(name):
    n, t = 1100, 20    # 20 right-hand sides: two column passes
    node, T, X, params, rng = _setup(name, n, 1)
    V = rng.normal(size=(t, n)).astype(np.float32)
    Xs = rng.uniform(-2.5, 2.5, size=(150, X.shape[1])).astype(np.float32)
    print(f"tree products {name} n={n} t={t}", flush=True)
    p = NativeProvider(None, False, X, params, 0.2, tree_spec=node.to_tree_spec(X.shape[1]))
    try:
        fwd = p.forward_matvec(V)
        cr = p.cross_matvec(Xs, V)
        p.materialize()
        mat = p.forward_matvec(V)
    finally:
        p.close()
    ref = ok.forward_matvec(T, X, V, params, 0.2, False)
    refc = ok.cross_matvec(T, Xs, X, V, params, False)
    print(f"  forward {_rel(fwd, ref):.2e} cross {_rel(cr, refc):.2e} "
          f"materialized {_rel(mat, ref):.2e} matrix-free vs materialized "
          f"{_rel(fwd, mat):.2e}", flush=True)
    assert _rel(fwd, ref) <= 1e-5
    assert _rel(cr, refc) <= 1e-5
    assert _rel(mat, ref) <= 1e-5
    # the compiled product and the dense fill evaluate the same arithmetic
    # (data spread over 3-6 lengthscales): they differ by the product
    # rounding only (fp32 / fp16-split MFMA sums)
    assert _rel(fwd, mat) <= 5e-6


@pytest.mark.parametrize("name", ["rbf+m52", "rq_ard+per[1]"])
def test_tree_products_multi_tile_splits(name):
    """n = 15003 (not a multiple of 8) and 20 right-hand sides: each column
    split of the tree product covers several 128-column tiles (LDS re-staging,
    fp32 part reset, fp64 carry), trailing splits may be empty, the last chunk
    is partial, and both the 16-column and the 4-column pass run.  Checked on
    192 sampled rows of the forward product and on a 300-row cross product."""
    n, t = 15003, 20
    node, T, X, params, rng = _setup(name, n, 5)
    V = rng.normal(size=(t, n)).astype(np.float32)
    Xs = rng.uniform(-2.5, 2.5, size=(300, X.shape[1])).astype(np.float32)
    rows = np.sort(rng.choice(n, 192, replace=False))
    rows[-1] = n - 1
    print(f"tree multi-tile {name} n={n} t={t}", flush=True)
    p = NativeProvider(None, False, X, params, 0.2, tree_spec=node.to_tree_spec(X.shape[1]))
    try:
        fwd = p.forward_matvec(V)
        cr = p.cross_matvec(Xs, V)
    finally:
        p.close()
    ref = ok.forward_matvec(T, X, V, params, 0.2, False, rows=rows, block=64)
    refc = ok.cross_matvec(T, Xs, X, V, params, False)
    e1, e2 = _rel(fwd[:, rows], ref), _rel(cr, refc)
    print(f"  forward (sampled rows) {e1:.2e} cross {e2:.2e}", flush=True)
    assert e1 <= 1e-5
    assert e2 <= 1e-5


@pytest.mark.parametrize("name,rank", [("rbf+m52", 30), ("rq_ard+per[1]", 40),
                                       ("(m12+rbf[2])*per", 0)])
def test_tree_pivoted_cholesky_and_bbmm(name, rank):
    n, probes = 500, 12
    node, T, X, params, rng = _setup(name, n, 2)
    y = (np.sin(X).sum(1) + 0.1 * rng.normal(size=n)).astype(np.float32)
    noise = 0.08 if rank else 0.2   # unpreconditioned: noise as for single kernels
    mean, it = 0.05, 3
    print(f"tree bbmm {name} rank={rank}", flush=True)
    p = NativeProvider(None, False, X, params, noise, tree_spec=node.to_tree_spec(X.shape[1]))
    g = np.zeros(params.size + 1, np.float32)
    nll, iq, ld, ci, pl = C.c_float(), C.c_float(), C.c_float(), C.c_int(), C.c_float()
    L = np.zeros((max(rank, 1), n), np.float32)
    rk, lpd = C.c_int(), C.c_float()
    try:
        if rank:
            _lib.call("mgp_pivoted_cholesky", p.handle, rank, 0, 0.0, 0.01, 42, _lib.fptr(L),
                      C.byref(rk), C.byref(lpd))
        _lib.call("mgp_bbmm_eval", p.handle, _lib.fptr(y), mean, probes, 100, 30, 1e-2, it, rank,
                  C.byref(nll), C.byref(iq), C.byref(ld), _lib.fptr(g), C.byref(ci), C.byref(pl),
                  None)
    finally:
        p.close()
    P = None
    if rank:
        K = T.matrix(X, X, params)
        Lr, kr = oe.pivoted_cholesky(K, rank)
        assert rk.value == kr
        assert np.abs(L[:kr].T - Lr).max() <= 1e-4 * np.abs(Lr).max()
        P = oe.Precond(Lr, noise)
    y_c = (y - np.float32(mean)).astype(np.float64)
    r = oe.bbmm_step(T, False, X, y_c, params.astype(np.float64), noise, P, probes, 100, 30,
                     1e-2, it)
    print(f"  nll {nll.value:.7f} vs {r['nll']:.7f}; cg {ci.value} vs {r['cg_iterations']}; "
          f"grad relerr {_rel(g, r['grads']):.2e}", flush=True)
    if rank:
        assert ci.value == r["cg_iterations"]
    assert nll.value == pytest.approx(r["nll"], rel=1e-4)
    assert iq.value == pytest.approx(r["inv_quad"], rel=1e-4)
    assert _rel(g, r["grads"]) <= 1e-3


def test_tree_fit_predict_save_load(tmp_path):
    from mojogp_amd import SingleOutputGP
    rng = np.random.default_rng(3)
    n = 400
    X = np.stack([np.linspace(-3, 3, n), rng.uniform(-1, 1, n)], 1).astype(np.float32)
    y = (np.sin(2 * X[:, 0]) * (1 + 0.3 * X[:, 1]) + 0.05 * rng.normal(size=n)).astype(np.float32)
    Xs = np.stack([np.linspace(-4, 4, 64), np.linspace(-1, 1, 64)], 1).astype(np.float32)
    kernel = RBF(active_dims=[0]) * Matern52(active_dims=[1]) + 0.5 * RQ()
    init = kernel.get_initial_params()
    gp = SingleOutputGP(kernel)
    tr = gp.fit(X, y, max_iterations=12, method="matrix_free")
    T = ok.TreeKernel(gp.kernel.to_dict(), 2)
    ref = oe.train(T, False, X, y, init, 0.1, max_iterations=12, num_probes=10, max_cg=100,
                   cg_tol=1e-2, precond_rank=0, max_tridiag=30)
    print(f"tree fit: params {tr.params} vs {ref['params']}; noise {tr.noise} vs "
          f"{ref['noise']}", flush=True)
    assert _rel(tr.params, ref["params"]) <= 1e-3
    assert tr.noise == pytest.approx(ref["noise"], rel=1e-3)
    mean_t, std_t = gp.predict(Xs, return_std=True, cg_tolerance=1e-6)
    pr = tr.params.astype(np.float64)
    mu_t, var_t, _ = oe.predict(T, False, X, y, Xs, pr, tr.noise, tr.mean, max_cg=300, tol=1e-6,
                                lanczos_rank=100)
    print(f"  predict mean relerr {_rel(mean_t, mu_t):.2e} LOVE std relerr "
          f"{_rel(std_t, np.sqrt(var_t)):.2e}", flush=True)
    assert _rel(mean_t, mu_t) <= 1e-4
    assert _rel(std_t, np.sqrt(var_t)) <= 1e-4
    _, var_e = gp.predict(Xs, return_var=True, variance_method="exact", cg_tolerance=1e-6,
                          max_cg_iterations=1000)
    ve, _, _ = oe.exact_variance(T, False, X, Xs, pr, tr.noise, max_cg=1000, tol=1e-6)
    print(f"  exact std relerr {_rel(np.sqrt(var_e), np.sqrt(ve)):.2e}", flush=True)
    assert _rel(np.sqrt(var_e), np.sqrt(ve)) <= 1e-4
    gp.save(tmp_path / "tree")
    gp2 = SingleOutputGP.load(str(tmp_path / "tree"))
    m2, s2 = gp2.predict(Xs, return_std=True, cg_tolerance=1e-6)
    np.testing.assert_allclose(m2, mean_t, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(s2, std_t, rtol=1e-5, atol=1e-6)


NONSTAT = {
    "linear*rbf+poly2": (lambda: Linear() * RBF()
                         + Polynomial(degree=2), 3),
    "linear_ard+rbf": (lambda: make_ard_kernel(Linear(ard=True) + RBF(), 3), 3),
    "poly3_ard+m52": (lambda: make_ard_kernel(Polynomial(degree=3, ard=True)
                                              + Matern52(), 2), 2),
}


@pytest.mark.parametrize("name", list(NONSTAT))
def test_nonstationary_tree_products_and_bbmm(name):
    """Linear / polynomial leaves: products, per-point diagonals (pivoted
    Cholesky start, extract_diagonal), and one preconditioned BBMM."""
    mk, d = NONSTAT[name]
    node = mk()
    rng = np.random.default_rng(21)
    n = 500
    X = rng.uniform(-1.5, 1.5, size=(n, d)).astype(np.float32)
    T = ok.TreeKernel(node.to_dict(), d)
    params = rng.uniform(0.5, 1.2, T.nparams).astype(np.float32)
    V = rng.normal(size=(3, n)).astype(np.float32)
    y = (np.sin(X).sum(1) + 0.1 * rng.normal(size=n)).astype(np.float32)
    print(f"non-stationary tree {name}", flush=True)
    p = NativeProvider(None, False, X, params, 0.2, tree_spec=node.to_tree_spec(d))
    g = np.zeros(params.size + 1, np.float32)
    nll, iq, ld, ci, pl = C.c_float(), C.c_float(), C.c_float(), C.c_int(), C.c_float()
    L = np.zeros((20, n), np.float32)
    rk, lpd = C.c_int(), C.c_float()
    diag = np.zeros(n, np.float32)
    try:
        fwd = p.forward_matvec(V)
        _lib.call("mgp_extract_diagonal", p.handle, _lib.fptr(diag))
        _lib.call("mgp_pivoted_cholesky", p.handle, 20, 0, 0.0, 0.01, 42, _lib.fptr(L),
                  C.byref(rk), C.byref(lpd))
        _lib.call("mgp_bbmm_eval", p.handle, _lib.fptr(y), 0.0, 10, 100, 30, 1e-2, 2, 20,
                  C.byref(nll), C.byref(iq), C.byref(ld), _lib.fptr(g), C.byref(ci), C.byref(pl),
                  None)
    finally:
        p.close()
    K = T.matrix(X, X, params)
    assert _rel(fwd, ok.forward_matvec(T, X, V, params, 0.2, False)) <= 1e-5
    np.testing.assert_allclose(diag, np.diag(K), rtol=1e-5, atol=1e-6)
    Lr, kr = oe.pivoted_cholesky(K, 20)
    assert rk.value == kr
    assert np.abs(L[:kr].T - Lr).max() <= 1e-4 * np.abs(Lr).max()
    r = oe.bbmm_step(T, False, X, y.astype(np.float64), params.astype(np.float64), 0.2,
                     oe.Precond(Lr, 0.2), 10, 100, 30, 1e-2, 2)
    print(f"  nll {nll.value:.7f} vs {r['nll']:.7f}; grads {_rel(g, r['grads']):.2e}", flush=True)
    assert nll.value == pytest.approx(r["nll"], rel=1e-4)
    assert _rel(g, r["grads"]) <= 1e-3


def test_nonstationary_fit_predict():
    """Linear x RBF + polynomial fit on the restatement's trajectory; LOVE and
    exact variances with per-test-point prior diagonals."""
    from mojogp_amd import SingleOutputGP
    rng = np.random.default_rng(8)
    n = 300
    X = rng.uniform(-2, 2, size=(n, 2)).astype(np.float32)
    y = (0.8 * X[:, 0] + np.sin(2 * X[:, 1]) + 0.1 * rng.normal(size=n)).astype(np.float32)
    kernel = Linear() * RBF() + Polynomial(degree=2)
    gp = SingleOutputGP(kernel)
    tr = gp.fit(X, y, max_iterations=8, method="matrix_free", learning_rate=0.02)
    T = ok.TreeKernel(gp.kernel.to_dict(), 2)
    init = gp.kernel.to_engine_params(gp.kernel.get_initial_params())
    ref = oe.train(T, False, X, y, init, 0.1, max_iterations=8, learning_rate=0.02,
                   num_probes=10, max_cg=100, cg_tol=1e-2, precond_rank=0, max_tridiag=30)
    eng_trained = ref["params"]
    print(f"nonstationary fit: noise {tr.noise} vs {ref['noise']}", flush=True)
    assert tr.noise == pytest.approx(ref["noise"], rel=1e-3)
    # public params report the structural degree; compare the engine slots the
    # public layout keeps (kernel.py:570-606)
    pub_ref = gp.kernel.from_engine_params(eng_trained)
    assert _rel(tr.params, pub_ref) <= 1e-3
    Xs = rng.uniform(-2.5, 2.5, size=(40, 2)).astype(np.float32)
    mean_t, std_t = gp.predict(Xs, return_std=True, cg_tolerance=1e-6)
    pe = gp.kernel.to_engine_params(tr.params).astype(np.float64)
    mu, var, _ = oe.predict(T, False, X, y, Xs, pe, tr.noise, tr.mean, max_cg=300, tol=1e-6,
                            lanczos_rank=100)
    # var = k(x*, x*) - |V|^2 cancels: polynomial priors reach ~100 here
    # against posterior variances ~0.05, so fp32 rounding of the prior term
    # alone is ~2e-7 * prior / var relative; the bar scales with that factor.
    prior = oe._kdiag(T, pe, Xs)
    cancel = float(np.max(prior / var))
    bar = max(1e-4, 2e-7 * cancel)
    print(f"  predict mean {_rel(mean_t, mu):.2e} std {_rel(std_t, np.sqrt(var)):.2e} "
          f"(prior / variance up to {cancel:.0f}, bar {bar:.1e})", flush=True)
    assert _rel(mean_t, mu) <= 1e-4
    assert _rel(std_t, np.sqrt(var)) <= bar
    _, var_e = gp.predict(Xs, return_var=True, variance_method="exact", cg_tolerance=1e-6,
                          max_cg_iterations=1000)
    ve, _, _ = oe.exact_variance(T, False, X, Xs, pe, tr.noise, max_cg=1000, tol=1e-6)
    print(f"  exact std {_rel(np.sqrt(var_e), np.sqrt(ve)):.2e}", flush=True)
    assert _rel(np.sqrt(var_e), np.sqrt(ve)) <= bar
