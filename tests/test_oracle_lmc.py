"""Pins of the LMC oracle (oracle/lmc.py) by independent mathematics (CPU)."""

import numpy as np
import pytest

from oracle import engine as oe
from oracle import kernels as ok
from oracle import lmc as ol


def _setup(rng, n=12, d=2, T=2, R=2):
    X = rng.uniform(0, 1, size=(n, d))
    kinds = [ok.RBF, ok.MATERN52][:R] + [ok.RBF] * max(0, R - 2)
    ards = [False, True][:R] + [False] * max(0, R - 2)
    params = []
    for s in range(R):
        k = d if ards[s] else 1
        params.append(np.concatenate([rng.uniform(0.3, 0.9, size=k), [rng.uniform(0.5, 1.5)]]))
    A = []
    for s in range(R):
        L = rng.normal(size=(T, T)) * 0.5
        A.append(L @ L.T + 0.1 * np.eye(T))
    noise = rng.uniform(0.05, 0.2, size=T)
    return X, kinds, ards, params, np.array(A), noise


def test_operator_entrywise_layout():
    """K_full[t n + i, t' n + j] = sum_s A_s[t, t'] K_s[i, j] + delta (noise_t + fixed)."""
    rng = np.random.default_rng(0)
    X, kinds, ards, params, A, noise = _setup(rng, n=7, T=3, R=2)
    n, T = X.shape[0], 3
    fixed = rng.uniform(0, 0.1, size=(T, n))
    Ks = ol.latent_kernels(kinds, ards, X, params)
    Kf = ol.dense_operator(Ks, A, noise, fixed)
    for t in range(T):
        for tp in range(T):
            for i in range(n):
                for j in range(n):
                    want = sum(A[s, t, tp] * Ks[s][i, j] for s in range(2))
                    if t == tp and i == j:
                        want += noise[t] + fixed[t, i]
                    assert Kf[t * n + i, tp * n + j] == pytest.approx(want, rel=1e-12, abs=1e-14)


def test_operator_reduces_to_single_output():
    rng = np.random.default_rng(1)
    X = rng.normal(size=(20, 3))
    p = np.array([0.7, 1.3])
    V = rng.normal(size=(2, 20))
    got = ol.forward_matvec([ok.MATERN52], [False], X, [p], np.array([[[1.0]]]), [0.1], V)
    ref = ok.forward_matvec(ok.MATERN52, X, V, p, 0.1, False)
    np.testing.assert_allclose(got, ref, rtol=1e-12)


def test_precond_structure_and_logdet():
    """U U^T = sum_s A_s (x) L_s L_s^T and log|P| by the determinant lemma."""
    rng = np.random.default_rng(2)
    X, kinds, ards, params, A, noise = _setup(rng, n=15, T=2, R=2)
    Ks = ol.latent_kernels(kinds, ards, X, params)
    P = ol.Precond(Ks, A, noise, rank=4)
    want = sum(np.kron(A[s], P.L[s] @ P.L[s].T) for s in range(2))
    np.testing.assert_allclose(P.U @ P.U.T, want, rtol=1e-10, atol=1e-12)
    Dinv = 1.0 / P.D
    M = np.eye(P.K) + P.U.T @ (Dinv[:, None] * P.U)
    lemma = np.sum(np.log(P.D)) + np.linalg.slogdet(M)[1]
    assert P.logdet == pytest.approx(lemma, rel=1e-10)
    # Woodbury apply against the dense solve
    r = rng.normal(size=(P.n * P.T, 3))
    w = Dinv[:, None] * r
    wood = w - Dinv[:, None] * (P.U @ np.linalg.solve(M, P.U.T @ w))
    np.testing.assert_allclose(P.apply(r), wood, rtol=1e-8, atol=1e-10)


def test_precond_probe_covariance():
    """Probes D^1/2 eps + U w have covariance P (sample moments)."""
    rng = np.random.default_rng(3)
    X, kinds, ards, params, A, noise = _setup(rng, n=5, T=2, R=2)
    Ks = ol.latent_kernels(kinds, ards, X, params)
    P = ol.Precond(Ks, A, noise, rank=3)
    Z = P.sample(40000, 7)
    cov = Z @ Z.T / Z.shape[1]
    scale = np.sqrt(np.outer(np.diag(P.P), np.diag(P.P)))
    assert np.max(np.abs(cov - P.P) / scale) < 0.03


def _exact(Kf, y):
    al = np.linalg.solve(Kf, y)
    N = len(y)
    nll = (0.5 * y @ al + 0.5 * np.linalg.slogdet(Kf)[1] + 0.5 * N * np.log(2 * np.pi)) / N
    return nll, al


def test_bbmm_gradients_converge_to_exact():
    """With many probes and tight CG the estimator reaches the exact
    gradients: d/dA_s[i, j] (independent entries), d/dnoise_t, kernel params."""
    rng = np.random.default_rng(4)
    X, kinds, ards, params, A, noise = _setup(rng, n=10, T=2, R=2)
    n, T, R = 10, 2, 2
    y = rng.normal(size=n * T)
    ev = ol.bbmm(kinds, ards, X, params, A, noise, y, num_probes=3000, max_cg=200,
                 max_tridiag=60, tol=1e-10)
    Ks = ol.latent_kernels(kinds, ards, X, params)
    Kf = ol.dense_operator(Ks, A, noise)
    nll, al = _exact(Kf, y)
    Kinv = np.linalg.inv(Kf)
    N = n * T
    assert ev["inv_quad"] == pytest.approx(y @ al, rel=1e-8)
    assert ev["nll"] == pytest.approx(nll, rel=0.02)
    ab = al.reshape(T, n)
    Pn = 3000

    def tol(dK):
        """4 standard deviations of the Gaussian Hutchinson estimate of
        0.5 tr(K^-1 dK) / N with Pn probes."""
        M = Kinv @ dK
        Ms = 0.5 * (M + M.T)
        return 4.0 * 0.5 * np.sqrt(2.0 * np.sum(Ms * Ms) / Pn) / N + 1e-9

    for s in range(R):
        for i in range(T):
            for j in range(T):
                E = np.zeros((T, T))
                E[i, j] = 1.0
                dK = np.kron(E, Ks[s])
                g = (-0.5 * al @ dK @ al + 0.5 * np.trace(Kinv @ dK)) / N
                assert ev["G_A"][s, i, j] == pytest.approx(g, abs=tol(dK))
                # data term is exact in the estimator's own algebra
                assert (-ab[i] @ Ks[s] @ ab[j]) == pytest.approx(-al @ dK @ al, rel=1e-10)
    for t in range(T):
        Et = np.zeros(N)
        Et[t * n:(t + 1) * n] = 1.0
        g = (-0.5 * al @ (Et * al) + 0.5 * np.sum(np.diag(Kinv) * Et)) / N
        assert ev["noise_grads"][t] == pytest.approx(g, abs=tol(np.diag(Et)))
    q = 0
    for s in range(R):
        for G in ok.kernel_gradients(kinds[s], X, X, params[s], ards[s]):
            dK = np.kron(A[s], G)
            g = (-0.5 * al @ dK @ al + 0.5 * np.trace(Kinv @ dK)) / N
            assert ev["kernel_grads"][q] == pytest.approx(g, abs=tol(dK))
            q += 1


def test_exact_gradient_formula_by_finite_differences():
    """The exact-gradient expressions used above match central differences of
    the exact NLL (pins the trace term's sign and the 1/N scaling)."""
    rng = np.random.default_rng(5)
    X, kinds, ards, params, A, noise = _setup(rng, n=8, T=2, R=2)
    y = rng.normal(size=16)
    Ks = ol.latent_kernels(kinds, ards, X, params)
    Kinv = np.linalg.inv(ol.dense_operator(Ks, A, noise))
    al = Kinv @ y
    h = 1e-6
    for s, i, j in [(0, 0, 1), (1, 1, 1), (1, 1, 0)]:
        Ap, Am = A.copy(), A.copy()
        Ap[s, i, j] += h
        Am[s, i, j] -= h
        fd = (_exact(ol.dense_operator(Ks, Ap, noise), y)[0]
              - _exact(ol.dense_operator(Ks, Am, noise), y)[0]) / (2 * h)
        E = np.zeros((2, 2))
        E[i, j] = 1.0
        dK = np.kron(E, Ks[s])
        g = (-0.5 * al @ dK @ al + 0.5 * np.trace(Kinv @ dK)) / 16
        assert g == pytest.approx(fd, rel=1e-5, abs=1e-9)


def test_bbmm_with_preconditioner_matches_without():
    """The preconditioner changes the probes but not the solution: with tight
    CG both routes reach the dense solve (to the pAp < 1e-10 guard of the
    reference's CG, which freezes a column once its normalised residual is
    ~1e-5)."""
    rng = np.random.default_rng(6)
    X, kinds, ards, params, A, noise = _setup(rng, n=14, T=2, R=2)
    y = rng.normal(size=28)
    ex = np.linalg.solve(ol.dense_operator(ol.latent_kernels(kinds, ards, X, params), A, noise), y)
    for rank in (0, 5):
        a = ol.bbmm(kinds, ards, X, params, A, noise, y, num_probes=4, max_cg=300, tol=1e-10,
                    precond_rank=rank)
        assert np.max(np.abs(a["alpha"] - ex)) <= 1e-5 * np.max(np.abs(ex))
        assert a["inv_quad"] == pytest.approx(y @ ex, rel=1e-5)


def test_pathwise_correction_and_prior():
    """Correction = LMC cross product of K_full^{-1} r; RFF covariance -> kernel."""
    rng = np.random.default_rng(7)
    X, kinds, ards, params, A, noise = _setup(rng, n=9, T=2, R=2)
    Xs = rng.uniform(0, 1, size=(4, 2))
    r = rng.normal(size=18)
    got = ol.pathwise_correction(kinds, ards, X, Xs, params, A, noise, r, max_cg=500, tol=1e-12)
    Kf = ol.dense_operator(ol.latent_kernels(kinds, ards, X, params), A, noise)
    beta = np.linalg.solve(Kf, r).reshape(2, 9)
    want = np.zeros((4, 2))
    for s in range(2):
        Kx = ok.kernel_matrix(kinds[s], Xs, X, params[s], ards[s])
        for t in range(2):
            for tp in range(2):
                want[:, t] += A[s, t, tp] * (Kx @ beta[tp])
    # the reference CG's pAp < 1e-10 guard ends the solve near 1e-5 relative
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-6)
    # RFF features: phi phi^T -> k for RBF (any d) and Matern-5/2 (d = 1)
    F = 20000
    for kind, d in [(ok.RBF, 3), (ok.MATERN52, 1)]:
        Z = rng.uniform(0, 1, size=(6, d))
        ls = np.full(d, 0.6)
        W = rng.standard_normal((F, d)) if kind == ok.RBF else rng.standard_t(5, size=(F, d))
        ph = rng.uniform(0, 2 * np.pi, size=F)
        feats = np.sqrt(2.0 / F) * np.cos((Z / ls) @ W.T + ph)
        cov = 1.7 * feats @ feats.T
        ref = ok.kernel_matrix(kind, Z, Z, np.array([0.6, 1.7]), False)
        assert np.max(np.abs(cov - ref)) < 0.06
        # the oracle's prior values are weights @ features^T
        w = rng.standard_normal((3, F)).astype(np.float32)
        vals = ol.rff_prior_values(Z, ls, W, ph, 1.7, w)
        np.testing.assert_allclose(vals, (w.astype(np.float64) @ (np.sqrt(1.7) * feats).T),
                                   rtol=1e-5, atol=1e-5)


def test_train_oracle_smoke():
    """Three oracle training steps run, keep A_s symmetric positive definite
    and report finite NLLs."""
    rng = np.random.default_rng(8)
    X, kinds, ards, params, A, noise = _setup(rng, n=10, T=2, R=2)
    Y = rng.normal(size=(2, 10))
    res = ol.train(kinds, ards, X, Y.reshape(-1), [p.astype(np.float32) for p in params],
                   np.full(2, 0.1, np.float32), np.zeros(2, np.float32), max_iterations=3,
                   num_probes=4, precond_rank=3)
    assert np.all(np.isfinite(res["nll_history"]))
    for s in range(2):
        np.testing.assert_allclose(res["A"][s], res["A"][s].T, rtol=1e-6)
        assert np.all(np.linalg.eigvalsh(res["A"][s].astype(np.float64)) > 0)
