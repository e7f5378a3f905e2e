"""Pins of the ICM oracle (oracle/icm.py) by independent mathematics (CPU)."""

import numpy as np
import pytest

from oracle import engine as oe
from oracle import icm as oi
from oracle import kernels as ok


def _setup(rng, n=12, d=2, T=3, ard=False, kind=ok.RBF):
    X = rng.uniform(0, 1, size=(n, d))
    k = d if ard else 1
    params = np.concatenate([rng.uniform(0.3, 0.9, size=k), [rng.uniform(0.5, 1.5)]])
    W = rng.normal(size=(T, T)) * 0.4
    B = (W @ W.T + 0.3 * np.eye(T)).astype(np.float32)
    noise = rng.uniform(0.05, 0.2, size=T).astype(np.float32)
    return X, kind, ard, params, B, noise


def test_init_w_known_values():
    """W = 0.1 + 0.4 u, u from the 31-bit LCG of seed ^ (i * 2654435761).
    i = 0: 42 * 1103515245 + 12345 = 46347652635 = 21 * 2^31 + 1250496027,
    u = 1250496027 / (2^31 - 1); i = 1: 42 ^ 2654435761 = 2654435803,
    whose product with 1103515245 plus 12345 is reduced mod 2^31 in Python
    integers below."""
    W = oi.init_w(3, 2)
    assert W.shape == (3, 2)
    assert W[0, 0] == pytest.approx(0.1 + 0.4 * 1250496027 / 2147483647, abs=1e-7)
    s1 = ((42 ^ 2654435761) * 1103515245 + 12345) % 2 ** 31
    assert W[0, 1] == pytest.approx(0.1 + 0.4 * s1 / 2147483647, abs=1e-7)
    assert np.all((W >= 0.1) & (W <= 0.5))
    assert len(np.unique(W)) == W.size


def test_task_b_is_wwt_plus_softplus_diag():
    W = np.array([[0.3, 0.2], [0.1, 0.4]], np.float32)
    v = np.array([0.0, -1.0], np.float32)
    B = oi.task_b(W, v)
    want = W.astype(np.float64) @ W.T + np.diag(np.log1p(np.exp(v.astype(np.float64))))
    np.testing.assert_allclose(B, want, rtol=1e-6)


@pytest.mark.parametrize("k", [1, 2, 5, 15])
def test_jacobi_matches_eigh(k):
    rng = np.random.default_rng(k)
    G = rng.normal(size=(k, k))
    A = (G @ G.T + 0.1 * np.eye(k)).astype(np.float32)
    e, V = oi.jacobi_eigen(A)
    ref = np.linalg.eigvalsh(A.astype(np.float64))
    np.testing.assert_allclose(e, ref, rtol=1e-5, atol=1e-6)
    assert np.all(np.diff(e) >= 0)
    np.testing.assert_allclose(V.T.astype(np.float64) @ V, np.eye(k), atol=1e-5)
    np.testing.assert_allclose((V * e) @ V.T, A, rtol=1e-4, atol=1e-5)


def test_kron_precond_apply_and_logdet_match_dense():
    """Eigenbasis Woodbury apply == solve(P, .) and log|P| == slogdet(P),
    P = os (B + 1e-6 D) (x) L L^T + D (x) I."""
    rng = np.random.default_rng(3)
    X, kind, ard, params, B, noise = _setup(rng, n=30, T=3)
    K = ok.kernel_matrix(kind, X, X, params, ard)
    P = oi.KronPrecond(K, 1.7, B, noise, rank=6)
    assert P.r == 6
    R = rng.normal(size=(90, 4))
    np.testing.assert_allclose(P.apply(R), np.linalg.solve(P.P, R), rtol=2e-4, atol=1e-5)
    assert P.logdet == pytest.approx(np.linalg.slogdet(P.P)[1], rel=1e-5)


def test_kron_precond_probe_factor_and_covariance():
    rng = np.random.default_rng(4)
    X, kind, ard, params, B, noise = _setup(rng, n=6, T=2)
    K = ok.kernel_matrix(kind, X, X, params, ard)
    os_ = 0.8
    P = oi.KronPrecond(K, os_, B, noise, rank=3)
    Cb = P.Cb.astype(np.float64)
    want = os_ * (B.astype(np.float64) + 1e-6 * np.diag(noise.astype(np.float64)))
    np.testing.assert_allclose(Cb @ Cb.T, want, rtol=2e-5, atol=1e-6)
    # explicit assembly from the two streams
    C, seed = 3, 11
    Z = P.sample(C, seed)
    N = 12
    zn = oe.gaussian(N * C, seed + 12345).astype(np.float64).reshape(C, N)
    zr = oe.gaussian(P.r * 2 * C, seed).astype(np.float64).reshape(2, C, P.r)
    for c in range(C):
        w = np.concatenate([zr[t, c] for t in range(2)])
        ds = np.sqrt(noise).astype(np.float64)          # fp32 D^1/2, as the reference
        want_c = np.repeat(ds, 6) * zn[c] + np.kron(Cb, P.L) @ w
        np.testing.assert_allclose(Z[:, c], want_c, rtol=1e-10, atol=1e-12)
    Zb = P.sample(40000, 5)
    cov = Zb @ Zb.T / Zb.shape[1]
    scale = np.sqrt(np.outer(np.diag(P.P), np.diag(P.P)))
    assert np.max(np.abs(cov - P.P) / scale) < 0.03


def _exact(Kf, y):
    al = np.linalg.solve(Kf, y)
    N = len(y)
    return (0.5 * y @ al + 0.5 * np.linalg.slogdet(Kf)[1] + 0.5 * N * np.log(2 * np.pi)) / N


def test_icm_gradients_match_finite_differences():
    """dNLL/d(os), G_B / os (= dNLL/dA at A = os B) and dNLL/dnoise of the
    estimator (many probes) against central differences of the exact NLL."""
    rng = np.random.default_rng(6)
    X, kind, ard, params, B, noise = _setup(rng, n=10, T=2)
    os_ = 1.3
    n, T = 10, 2
    N = n * T
    y = rng.normal(size=N)
    Pn = 3000
    ev = oi.bbmm(kind, ard, X, params, os_, B, noise, y, num_probes=Pn, max_cg=200,
                 max_tridiag=60, tol=1e-10)
    K = ok.kernel_matrix(kind, X, X, params, ard)

    def full(o, Bm, nz):
        return o * np.kron(np.asarray(Bm, np.float64), K) + np.diag(np.repeat(nz, n))

    Kf = full(os_, B, noise)
    Kinv = np.linalg.inv(Kf)

    def tol(dK):
        M = Kinv @ dK
        Ms = 0.5 * (M + M.T)
        return 4.0 * 0.5 * np.sqrt(2.0 * np.sum(Ms * Ms) / Pn) / N + 1e-9

    h = 1e-6
    fd_os = (_exact(full(os_ + h, B, noise), y) - _exact(full(os_ - h, B, noise), y)) / (2 * h)
    assert ev["grad_outputscale"] == pytest.approx(fd_os, abs=tol(np.kron(B, K)))
    for i, j in [(0, 0), (0, 1), (1, 1)]:
        Bp, Bm = B.astype(np.float64).copy(), B.astype(np.float64).copy()
        Bp[i, j] += h
        Bm[i, j] -= h
        fd = (_exact(full(os_, Bp, noise), y) - _exact(full(os_, Bm, noise), y)) / (2 * h)
        E = np.zeros((T, T))
        E[i, j] = 1.0
        # G_B[i, j] = os * dNLL/dA[i, j] = dNLL/dB[i, j] for independent entries
        assert ev["grad_B"][i, j] == pytest.approx(fd, abs=os_ * tol(np.kron(E, K)))
    for t in range(T):
        npl, nmi = noise.astype(np.float64).copy(), noise.astype(np.float64).copy()
        npl[t] += h
        nmi[t] -= h
        fd = (_exact(full(os_, B, npl), y) - _exact(full(os_, B, nmi), y)) / (2 * h)
        Et = np.zeros(N)
        Et[t * n:(t + 1) * n] = 1.0
        assert ev["noise_grads"][t] == pytest.approx(fd, abs=tol(np.diag(Et)))


def test_bbmm_with_kron_precond_matches_exact_nll():
    """Preconditioned evaluation: log|K| = log|P| + SLQ(P^-1 K) reaches the
    exact value with many probes."""
    rng = np.random.default_rng(7)
    X, kind, ard, params, B, noise = _setup(rng, n=20, T=2, kind=ok.MATERN52)
    y = rng.normal(size=40)
    ev = oi.bbmm(kind, ard, X, params, 0.9, B, noise, y, num_probes=2000, max_cg=200,
                 max_tridiag=60, tol=1e-10, precond_rank=5)
    K = ok.kernel_matrix(kind, X, X, params, ard)
    Kf = 0.9 * np.kron(B.astype(np.float64), K) + np.diag(np.repeat(noise.astype(np.float64), 20))
    assert ev["inv_quad"] == pytest.approx(y @ np.linalg.solve(Kf, y), rel=1e-8)
    assert ev["logdet"] == pytest.approx(np.linalg.slogdet(Kf)[1], rel=0.02)


def test_rotated_prediction_matches_joint_posterior():
    """With equal task noise the eigen-task decomposition of os B is exact:
    mean and variance equal the dense joint posterior of the latent."""
    rng = np.random.default_rng(8)
    X, kind, ard, params, B, _ = _setup(rng, n=15, T=3, ard=True)
    Xs = rng.uniform(0, 1, size=(5, 2))
    os_, sig2, n, T = 1.2, 0.07, 15, 3
    K = ok.kernel_matrix(kind, X, X, params, ard)
    Kx = ok.kernel_matrix(kind, Xs, X, params, ard)
    Bs = os_ * B.astype(np.float64)
    Kf = np.kron(Bs, K) + sig2 * np.eye(n * T)
    y = rng.normal(size=n * T)
    alpha = np.linalg.solve(Kf, y)
    Q, lam, arot = oi.rotate(os_, B, alpha, n)
    mean, var = oi.predict(kind, ard, X, Xs, params, arot, Q, lam, sig2)
    want_mean = (np.kron(Bs, Kx) @ alpha).reshape(T, -1).T
    np.testing.assert_allclose(mean, want_mean, rtol=1e-8, atol=1e-10)
    kss = params[-1]
    for t in range(T):
        for i in range(Xs.shape[0]):
            c = np.kron(Bs[:, t], Kx[i])
            v = Bs[t, t] * kss - c @ np.linalg.solve(Kf, c)
            assert var[i, t] == pytest.approx(v, rel=1e-6, abs=1e-9)


def test_train_oracle_improves_nll():
    rng = np.random.default_rng(9)
    n, T = 40, 2
    X = rng.uniform(-1, 1, size=(n, 2))
    Y = np.stack([np.sin(3 * X[:, 0]), np.sin(3 * X[:, 0] + 0.5)]) + 0.1 * rng.normal(size=(T, n))
    res = oi.train(ok.RBF, False, X, Y.reshape(-1), [1.0, 1.0], [0.1, 0.1], 1.0,
                   Y.mean(axis=1), max_iterations=15, learning_rate=0.1, num_probes=8,
                   precond_rank=5, early_stop_tol=0.0)
    h = res["nll_history"]
    assert np.all(np.isfinite(h)) and len(h) == 15
    assert np.mean(h[-3:]) < np.mean(h[:3])
    assert res["final_nll"] == pytest.approx(float(np.min(h)))


def test_unpreconditioned_logdet_fp32_floor():
    """The GPU ICM BBMM test's unpreconditioned tolerance-1e-5 cases
    (test_gpu_icm.py) run by the restatement with its CG in fp64 and in fp32:
    the SLQ log-determinant moves by 1.0e-4 and 1.4e-4 and the CG count from 70
    to 100 / 120, while inv_quad stays within 1e-6.  This is the floor any
    fp32 implementation sits at, and why the GPU bar is 3e-4 there."""
    import sys
    import os
    sys.path.insert(0, os.path.dirname(__file__))
    from test_gpu_icm import _problem
    F32 = np.float32
    orig = oe.batched_cg

    def cg32(A, rhs, P, max_iter, max_tridiag, tol, x0=None):
        x, it, conv, dd, oo = orig(A.astype(F32), rhs.astype(F32), P, max_iter, max_tridiag,
                                   tol, None if x0 is None else x0.astype(F32))
        return x.astype(np.float64), it, conv, dd, oo

    gaps = []
    for fixed in (False, True):
        n, d, T, os_ = 180, 2, 3, 1.3
        rng, X, params, B, noise = _problem(11, n, d, T, False)
        noise = rng.uniform(0.1, 0.3, size=T).astype(np.float32)
        y = (np.sin(4 * X[:, :1]) * np.array([[1.0, -0.5, 0.3]]) + 0.1 * rng.normal(size=(n, T)))
        y = np.ascontiguousarray(y.T.reshape(-1), dtype=np.float64)
        fx = rng.uniform(0.1, 0.3, size=(T, n)).astype(np.float32) if fixed else None
        op_noise = np.zeros(T, np.float32) if fixed else noise
        kw = dict(fixed=fx, num_probes=8, max_cg=500, max_tridiag=30, tol=1e-5, iteration=2,
                  precond_rank=0)
        ref = oi.bbmm(ok.MATERN52, False, X, params.astype(np.float64), os_, B, op_noise, y, **kw)
        oe.batched_cg = cg32
        try:
            r32 = oi.bbmm(ok.MATERN52, False, X, params.astype(np.float64), os_, B, op_noise, y,
                          **kw)
        finally:
            oe.batched_cg = orig
        assert abs(r32["inv_quad"] - ref["inv_quad"]) <= 1e-6 * abs(ref["inv_quad"])
        assert r32["cg_iterations"] > ref["cg_iterations"]
        gaps.append(abs(r32["logdet"] - ref["logdet"]) / abs(ref["logdet"]))
    print(f"fp32-CG log-determinant gaps {gaps}")
    assert 5e-5 < max(gaps) < 3e-4
