"""GPU parity of the Matern-1/2 and Matern-3/2 kernels against the float64
oracle: products (training, cross, materialized), gradient products, pivoted
Cholesky, one BBMM evaluation, a short fit, and their use as LMC / ICM
latents.  Matern-3/2 runs on the Gram-form tile kernel; Matern-1/2 always on
the per-dimension-difference path (its slope in the squared distance is
unbounded at 0).  Bars as for RBF / Matern-5/2: products 1e-5, NLL 1e-4,
gradients 1e-3."""

import ctypes as C

import numpy as np
import pytest

from mojogp_amd import _lib
from mojogp_amd._provider import NativeProvider
from oracle import engine as oe
from oracle import kernels as ok
from oracle import lmc as ol

pytestmark = pytest.mark.gpu

TOL = 1e-5
M12, M32 = ok.MATERN12, ok.MATERN32


def _rel(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def _params(rng, d, ard, lo=0.6, hi=1.6, os=1.3):
    ls = rng.uniform(lo, hi, size=d if ard else 1)
    return np.concatenate([ls, [os]]).astype(np.float32)


CASES = [
    # kind, ard, d, n, t
    (M32, True, 8, 3000, 16),
    (M32, False, 2, 1500, 1),
    (M32, True, 16, 2000, 40),
    (M12, True, 4, 2000, 16),
    (M12, False, 1, 2500, 3),
    (M12, True, 20, 700, 1),
]


@pytest.mark.parametrize("kind,ard,d,n,t", CASES)
def test_forward_matvec_parity(kind, ard, d, n, t):
    rng = np.random.default_rng(2000 + 7 * d + n + kind)
    print(f"forward kind={kind} ard={ard} d={d} n={n} t={t}", flush=True)
    X = rng.normal(size=(n, d)).astype(np.float32)
    if d == 1:  # dense 1-D data with exact duplicates: the Matern-1/2 cusp
        idx = np.arange(0, n - 1, 7)
        X[idx] = X[idx + 1]
    V = rng.normal(size=(t, n)).astype(np.float32)
    params = _params(rng, d, ard)
    ref = ok.forward_matvec(kind, X, V, params, 0.05, ard)
    p = NativeProvider(kind, ard, X, params, 0.05)
    try:
        got = p.forward_matvec(V)
        direct = p.direct_matvec(V)
    finally:
        p.close()
    print(f"  relerr fused {_rel(got, ref):.2e} direct {_rel(direct, ref):.2e}", flush=True)
    assert _rel(got, ref) <= TOL
    assert _rel(direct, ref) <= TOL


@pytest.mark.parametrize("kind,ard,d,t", [(M32, True, 6, 16), (M12, False, 3, 5), (M32, False, 1, 1)])
def test_cross_matvec_parity(kind, ard, d, t):
    rng = np.random.default_rng(70 + d + kind)
    X = rng.normal(size=(1500, d)).astype(np.float32)
    Xs = rng.normal(size=(333, d)).astype(np.float32)
    V = rng.normal(size=(t, 1500)).astype(np.float32)
    params = _params(rng, d, ard)
    p = NativeProvider(kind, ard, X, params, 0.0)
    try:
        got = p.cross_matvec(Xs, V)
    finally:
        p.close()
    ref = ok.cross_matvec(kind, Xs, X, V, params, ard)
    print(f"cross kind={kind}: relerr {_rel(got, ref):.2e}", flush=True)
    assert _rel(got, ref) <= TOL


@pytest.mark.parametrize("kind", [M12, M32])
def test_materialized_route_parity(kind):
    rng = np.random.default_rng(90 + kind)
    X = rng.normal(size=(2000, 3)).astype(np.float32)
    V = rng.normal(size=(8, 2000)).astype(np.float32)
    params = _params(rng, 3, True)
    p = NativeProvider(kind, True, X, params, 0.1)
    try:
        p.materialize()
        got = p.forward_matvec(V)
    finally:
        p.close()
    ref = ok.forward_matvec(kind, X, V, params, 0.1, True)
    print(f"materialized kind={kind}: relerr {_rel(got, ref):.2e}", flush=True)
    assert _rel(got, ref) <= TOL


@pytest.mark.parametrize("kind,ard,d", [(M12, True, 3), (M12, False, 2), (M32, True, 4),
                                        (M32, False, 1)])
def test_gradient_matvec_parity(kind, ard, d):
    rng = np.random.default_rng(60 + d + kind)
    X = rng.normal(size=(800, d)).astype(np.float32)
    V = rng.normal(size=(3, 800)).astype(np.float32)
    params = _params(rng, d, ard)
    p = NativeProvider(kind, ard, X, params, 0.05)
    try:
        got = p.gradient_matvec(V)
    finally:
        p.close()
    ref = ok.gradient_matvec(kind, X, V, params, ard)
    got = got.reshape(ref.shape)
    errs = [_rel(got[q], ref[q]) for q in range(ref.shape[0])]
    print(f"gradient kind={kind} ard={ard} d={d}: max relerr {max(errs):.2e}", flush=True)
    assert np.all(np.isfinite(got))
    assert max(errs) <= TOL


@pytest.mark.parametrize("kind,ard,d,rank", [(M12, True, 3, 40), (M32, False, 2, 30)])
def test_pivoted_cholesky_and_bbmm_match_oracle(kind, ard, d, rank):
    rng = np.random.default_rng(10 + d + kind)
    n, probes = 500, 12
    X = rng.uniform(-2, 2, size=(n, d)).astype(np.float32)
    y = (np.sin(X).sum(1) + 0.1 * rng.normal(size=n)).astype(np.float32)
    params = np.concatenate([rng.uniform(0.7, 1.3, d if ard else 1), [1.1]]).astype(np.float32)
    noise, mean, it = 0.08, 0.05, 3
    print(f"bbmm kind={kind} ard={ard} d={d} rank={rank}", flush=True)
    p = NativeProvider(kind, ard, X, params, noise)
    g = np.zeros(params.size + 1, np.float32)
    nll, iq, ld, ci, pl = C.c_float(), C.c_float(), C.c_float(), C.c_int(), C.c_float()
    L = np.zeros((rank, n), np.float32)
    rk, lpd = C.c_int(), C.c_float()
    try:
        _lib.call("mgp_pivoted_cholesky", p.handle, rank, 0, 0.0, 0.01, 42, _lib.fptr(L),
                  C.byref(rk), C.byref(lpd))
        _lib.call("mgp_bbmm_eval", p.handle, _lib.fptr(y), mean, probes, 100, 30, 1e-2, it, rank,
                  C.byref(nll), C.byref(iq), C.byref(ld), _lib.fptr(g), C.byref(ci), C.byref(pl),
                  None)
    finally:
        p.close()
    K = ok.kernel_matrix(kind, X, X, params, ard)
    Lr, kr = oe.pivoted_cholesky(K, rank)
    assert rk.value == kr
    assert np.abs(L[:kr].T - Lr).max() <= 1e-4 * np.abs(Lr).max()
    P = oe.Precond(Lr, noise)
    y_c = (y - np.float32(mean)).astype(np.float64)
    r = oe.bbmm_step(kind, ard, X, y_c, params.astype(np.float64), noise, P, probes, 100, 30,
                     1e-2, it)
    print(f"  nll {nll.value:.7f} vs {r['nll']:.7f}; cg {ci.value} vs {r['cg_iterations']}; "
          f"grad relerr {_rel(g, r['grads']):.2e}", flush=True)
    assert ci.value == r["cg_iterations"]
    assert nll.value == pytest.approx(r["nll"], rel=1e-4)
    assert iq.value == pytest.approx(r["inv_quad"], rel=1e-4)
    assert _rel(g, r["grads"]) <= 1e-3


@pytest.mark.parametrize("kernel,kind", [("Matern32", M32), ("Matern12", M12)])
def test_fit_then_predict_matches_oracle(kernel, kind):
    import mojogp_amd
    rng = np.random.default_rng(3)
    n = 400
    X = np.linspace(-3, 3, n, dtype=np.float32)[:, None]
    y = (np.sin(2 * X[:, 0]) + 0.05 * rng.normal(size=n)).astype(np.float32)
    Xs = np.linspace(-4, 4, 64, dtype=np.float32)[:, None]
    gp = mojogp_amd.SingleOutputGP(getattr(mojogp_amd, kernel)())
    tr = gp.fit(X, y, max_iterations=15, method="matrix_free", initial_params=[0.5, 1.0])
    ref = oe.train(kind, False, X, y, [0.5, 1.0], 0.1, max_iterations=15, num_probes=10,
                   max_cg=100, cg_tol=1e-2, precond_rank=0, max_tridiag=30)
    print(f"{kernel}: params {tr.params} vs {ref['params']}; noise {tr.noise} vs "
          f"{ref['noise']}", flush=True)
    assert _rel(tr.params, ref["params"]) <= 1e-3
    assert tr.noise == pytest.approx(ref["noise"], rel=1e-3)
    mean_t, std_t = gp.predict(Xs, return_std=True, cg_tolerance=1e-6)
    mu_t, var_t, _ = oe.predict(kind, False, X, y, Xs, tr.params.astype(np.float64), tr.noise,
                                tr.mean, max_cg=300, tol=1e-6, lanczos_rank=100)
    print(f"  predict mean relerr {_rel(mean_t, mu_t):.2e} std relerr "
          f"{_rel(std_t, np.sqrt(var_t)):.2e}", flush=True)
    assert _rel(mean_t, mu_t) <= 1e-4
    assert _rel(std_t, np.sqrt(var_t)) <= 1e-4


def test_lmc_with_low_order_matern_latents():
    """One Matern-3/2 (fused, mixing folded into the reduction) and one
    Matern-1/2 latent (difference path + separate mixing) in one product."""
    rng = np.random.default_rng(5)
    n, d, T, Cc = 900, 3, 3, 4
    X = rng.uniform(0, 1, size=(n, d)).astype(np.float32)
    params = [np.array([0.4, 1.1], np.float32), np.array([0.3, 0.5, 0.7, 0.9], np.float32)]
    kinds, ards = [M32, M12], [False, True]
    A = []
    for _ in range(2):
        Lm = rng.normal(size=(T, T)) * 0.6
        A.append(Lm @ Lm.T + 0.1 * np.eye(T))
    A = np.asarray(A, np.float32)
    noise = rng.uniform(0.03, 0.1, size=T).astype(np.float32)
    V = rng.normal(size=(Cc, T * n)).astype(np.float32)
    provs = [NativeProvider(k, a, X, p, 0.0) for k, a, p in zip(kinds, ards, params)]
    out = np.zeros_like(V)
    try:
        _lib.call("mgp_lmc_forward_matvec", _lib.handles(provs), 2, T, _lib.fptr(A),
                  _lib.fptr(noise), None, _lib.fptr(V), Cc, _lib.fptr(out))
    finally:
        for p in provs:
            p.close()
    ref = ol.forward_matvec(kinds, ards, X, params, A, noise, V)
    errs = [_rel(out[c], ref[c]) for c in range(Cc)]
    print(f"lmc M32+M12 max column relerr {max(errs):.2e}", flush=True)
    assert max(errs) <= TOL


def test_icm_matern32_surface():
    from mojogp_amd import MultiOutputGP
    rng = np.random.default_rng(7)
    n, T = 800, 2
    X = rng.normal(size=(n, 2)).astype(np.float32)
    Y = np.stack([np.sin(X[:, 0] + 0.5 * t) + 0.1 * rng.normal(size=n) for t in range(T)],
                 axis=1).astype(np.float32)
    gp = MultiOutputGP(kernel="matern32")
    res = gp.fit(X, Y, max_iterations=20, learning_rate=0.1, early_stop_tol=0.0)
    h = np.asarray(res.nll_history)
    print(f"icm matern32 nll {h[0]:.4f} -> {h[-1]:.4f}", flush=True)
    assert np.all(np.isfinite(h)) and np.mean(h[-3:]) < np.mean(h[:3])
    mean, var = gp.predict(X[:50], return_var=True, variance_method="exact")
    assert np.all(var > 0) and gp.score(X[:200], Y[:200])["r2"] > 0.8
