"""Pins the CPU restatement of the engine (oracle/engine.py) against facts that do
not depend on it: library solvers, closed forms, exact identities and
statistical properties.  CPU only, small n."""

import numpy as np
import pytest
from scipy import stats

from oracle import engine as oe
from oracle import kernels as ok


def _spd(rng, n, d=3, noise=0.1, kind=ok.MATERN52):
    X = rng.normal(size=(n, d))
    params = np.concatenate([rng.uniform(0.7, 1.5, d), [1.3]])
    K = ok.kernel_matrix(kind, X, X, params, True)
    return X, params, K, K + noise * np.eye(n)


# ------------------------------------------------------------------ RNG
def test_gaussian_moments_and_normality():
    z = oe.gaussian(200_000, 42).astype(np.float64)
    assert abs(z.mean()) < 0.01
    assert abs(z.var() - 1.0) < 0.01
    assert stats.kstest(z[:20000], "norm").pvalue > 1e-3


def test_gaussian_deterministic_and_seed_dependent():
    a = oe.gaussian(1000, 7)
    assert np.array_equal(a, oe.gaussian(1000, 7))
    assert not np.array_equal(a, oe.gaussian(1000, 8))
    assert np.array_equal(oe.gaussian(1000, 7)[:10], oe.gaussian(10, 7))


def test_gaussian_integer_hash_with_python_ints():
    """Same uniforms from arbitrary-precision integers reduced mod 2^64."""
    M = (1 << 64) - 1
    seed = 104729 * 3 + 42
    out = oe.gaussian(5, seed)
    for idx in range(5):
        k = idx + 1
        s1 = (k * 6364136223846793005 + seed) & M
        s1 ^= s1 >> 33
        s1 = (s1 * 0xFF51AFD7ED558CCD) & M
        s1 ^= s1 >> 33
        s2 = (k * 1442695040888963407 + seed + 0xBEEF) & M
        s2 ^= s2 >> 33
        s2 = (s2 * 0xC4CEB9FE1A85EC53) & M
        s2 ^= s2 >> 33
        u1 = ((s1 & 0x7FFFFF) + 1) / 8388608.0
        u2 = (s2 & 0xFFFFFF) / 16777216.0
        z = np.sqrt(-2 * np.log(u1)) * np.cos(2 * 3.14159265 * u2)
        assert out[idx] == pytest.approx(z, rel=2e-6, abs=2e-6)


# ------------------------------------------------------------------ preconditioner
def test_pivoted_cholesky_exact_on_low_rank():
    rng = np.random.default_rng(1)
    B = rng.normal(size=(60, 5))
    K = B @ B.T
    L, k = oe.pivoted_cholesky(K, 5, dtype=np.float64)
    assert k == 5
    np.testing.assert_allclose(L @ L.T, K, atol=1e-9)
    L2, k2 = oe.pivoted_cholesky(K, 12, dtype=np.float64)  # stops once the residual vanishes
    assert k2 == 5


def test_pivoted_cholesky_full_rank_and_monotone_error():
    rng = np.random.default_rng(2)
    _, _, K, _ = _spd(rng, 40)
    errs = []
    for r in (1, 5, 10, 20, 40):
        L, _ = oe.pivoted_cholesky(K, r, dtype=np.float64)
        errs.append(np.trace(K - L @ L.T))
    assert all(a >= b - 1e-12 for a, b in zip(errs, errs[1:]))
    L, _ = oe.pivoted_cholesky(K, 40, dtype=np.float64)
    np.testing.assert_allclose(L @ L.T, K, atol=1e-8)
    L32, _ = oe.pivoted_cholesky(K, 40)
    np.testing.assert_allclose(L32 @ L32.T, K, atol=1e-4)


def test_fp32_residual_ties_pick_lowest_index():
    # Rows 2 and 3 are far from the first pivot (row 0): their fp32 residual
    # diagonal rounds to exactly 1.0, so the second pivot is row 2 (lowest
    # index), although row 3 is farther away in exact arithmetic.
    K = np.eye(4)
    K[0, 1] = K[1, 0] = 0.5
    K[0, 2] = K[2, 0] = 1e-5
    K[0, 3] = K[3, 0] = 1e-9
    L32, _ = oe.pivoted_cholesky(K, 2)
    L64, _ = oe.pivoted_cholesky(K, 2, dtype=np.float64)
    assert np.argmax(np.abs(L32[:, 1])) == 2
    assert np.argmax(np.abs(L64[:, 1])) == 3


def test_sampled_pivots_exact_on_low_rank():
    # rpcholesky / nystrom on a rank-5 K: every draw lands on a point with
    # positive residual, and the factor is exact once the residual vanishes.
    rng = np.random.default_rng(4)
    B = rng.normal(size=(80, 5))
    K = B @ B.T
    for method in (1, 2):
        L, k = oe.pivoted_cholesky(K, 12, dtype=np.float64, method=method, error_tol=0.0,
                                   adaptive_tol=0.0, noise=0.1, diag_value=1.0)
        assert k == 5
        np.testing.assert_allclose(L @ L.T, K, atol=1e-8)


def test_sampled_pivot_frequencies_follow_residual_diagonal():
    # First pivot over a diagonal K: drawn with probability d_i / sum d
    # (chi-square over 4000 seeds).
    w = np.array([0.5, 1.0, 2.0, 4.0, 0.0, 2.5])
    K = np.diag(w)
    counts = np.zeros(w.size)
    for seed in range(1, 4001):
        L, _ = oe.pivoted_cholesky(K, 1, method=1, error_tol=0.0, seed=seed, diag_value=1.0)
        counts[int(np.argmax(np.abs(L[:, 0])))] += 1
    assert counts[4] == 0
    expected = w / w.sum() * counts.sum()
    keep = expected > 0
    chi2 = ((counts[keep] - expected[keep]) ** 2 / expected[keep]).sum()
    assert stats.chi2.sf(chi2, keep.sum() - 1) > 1e-3


def test_nystrom_adaptive_rank_stops_at_noise_floor():
    rng = np.random.default_rng(5)
    X = rng.normal(size=(300, 3))
    params = np.array([0.8, 1.3])
    K = ok.kernel_matrix(ok.RBF, X, X, params, False)
    n, noise, tol = 300, 0.05, 0.01
    L, k = oe.pivoted_cholesky(K, 300, method=2, adaptive_tol=tol, noise=noise,
                               diag_value=1.3)
    assert 1 < k < 300
    thr = tol * n * noise
    # The first k pivots reproduce the run; its residual trace is below the
    # floor and the (k-1)-pivot residual is not (fp32 run, small margin).
    tr_k = np.trace(K - L @ L.T)
    tr_km1 = np.trace(K - L[:, :k - 1] @ L[:, :k - 1].T)
    assert tr_k < thr * (1 + 1e-4)
    assert tr_km1 >= thr * (1 - 1e-4)


def test_rpcholesky_relative_trace_stop():
    rng = np.random.default_rng(6)
    X = rng.normal(size=(200, 2))
    params = np.array([1.1, 1.0])
    K = ok.kernel_matrix(ok.MATERN52, X, X, params, False)
    L, k = oe.pivoted_cholesky(K, 200, method=1, error_tol=1e-2, diag_value=1.0)
    assert 1 < k < 200
    assert np.trace(K - L @ L.T) / 1.0 < 1e-2 * (1 + 1e-4)
    assert np.trace(K - L[:, :k - 1] @ L[:, :k - 1].T) >= 1e-2 * (1 - 1e-4)


def test_pivot_order_is_greedy_lowest_index():
    K = np.diag([1.0, 3.0, 3.0, 2.0])
    L, k = oe.pivoted_cholesky(K, 2)
    assert np.argmax(np.abs(L[:, 0])) == 1     # tie 3.0 at rows 1, 2 -> row 1
    assert np.argmax(np.abs(L[:, 1])) == 2


def test_woodbury_and_logdet_match_dense():
    rng = np.random.default_rng(3)
    _, _, K, _ = _spd(rng, 50)
    L, _ = oe.pivoted_cholesky(K, 15)
    P = oe.Precond(L, 0.05)
    Pm = L @ L.T + 0.05 * np.eye(50)
    V = rng.normal(size=(50, 4))
    np.testing.assert_allclose(P.apply(V), np.linalg.solve(Pm, V), rtol=1e-8, atol=1e-10)
    assert P.logdet == pytest.approx(np.linalg.slogdet(Pm)[1], rel=1e-10)


def test_precond_samples_have_covariance_P():
    rng = np.random.default_rng(4)
    _, _, K, _ = _spd(rng, 12)
    L, _ = oe.pivoted_cholesky(K, 4)
    P = oe.Precond(L, 0.2)
    Z = P.sample(40000, 42)
    cov = Z @ Z.T / Z.shape[1]
    Pm = L @ L.T + 0.2 * np.eye(12)
    assert np.abs(cov - Pm).max() < 0.06 * np.abs(Pm).max()


# ------------------------------------------------------------------ CG / SLQ
@pytest.mark.parametrize("use_pc", [False, True])
def test_batched_cg_matches_solve(use_pc):
    rng = np.random.default_rng(5)
    _, _, K, A = _spd(rng, 80)
    P = oe.Precond(oe.pivoted_cholesky(K, 10)[0], 0.1) if use_pc else None
    rhs = rng.normal(size=(80, 3))
    x, iters, conv, _, _ = oe.batched_cg(A, rhs, P, 1000, 30, 1e-12)
    np.testing.assert_allclose(x, np.linalg.solve(A, rhs), rtol=1e-6, atol=1e-9)
    assert iters >= 30


def test_cg_stops_only_on_check_iterations():
    rng = np.random.default_rng(6)
    _, _, _, A = _spd(rng, 60)
    rhs = rng.normal(size=(60, 2))
    rhs /= np.linalg.norm(rhs, axis=0)
    _, iters, conv, _, _ = oe.batched_cg(A, rhs, None, 100, 5, 1e-2)
    assert conv and iters % 10 == 0 and iters >= 10


def test_slq_full_lanczos_equals_quadratic_form_of_log():
    """With n CG steps the probe tridiagonal carries the exact spectral measure:
    sum_i V0i^2 log(lambda_i) = z^T log(A) z for a unit probe z."""
    rng = np.random.default_rng(7)
    n = 24
    _, _, _, A = _spd(rng, n, noise=0.5)
    z = rng.normal(size=(n, 1))
    z /= np.linalg.norm(z)
    _, _, _, diags, offs = oe.batched_cg(A, z, None, n, n, 1e-30)
    est = oe.slq_logdet(diags, offs, 1)
    w, U = np.linalg.eigh(A)
    exact = float((z[:, 0] @ U) ** 2 @ np.log(w))
    assert est == pytest.approx(exact, rel=1e-6)


def test_slq_scaled_identity_closed_form():
    n, c = 30, 3.5
    z = np.ones((n, 2)) / np.sqrt(n)
    _, _, _, diags, offs = oe.batched_cg(c * np.eye(n), z, None, 5, 5, 1e-30)
    assert oe.slq_logdet(diags, offs, n) == pytest.approx(n * np.log(c), rel=1e-12)


# ------------------------------------------------------------------ BBMM
def test_bbmm_converges_to_exact_nll_and_gradient():
    rng = np.random.default_rng(8)
    n, d = 120, 2
    X = rng.uniform(-2, 2, size=(n, d))
    params = np.array([0.9, 1.3, 1.1])
    noise = 0.2
    y = np.sin(X.sum(1)) + 0.1 * rng.normal(size=n)
    A = ok.kernel_matrix(ok.RBF, X, X, params, True) + noise * np.eye(n)
    r = oe.bbmm_step(ok.RBF, True, X, y, params, noise, None, 400, n, n, 1e-10, 0)
    a = np.linalg.solve(A, y)
    nll = (0.5 * y @ a + 0.5 * np.linalg.slogdet(A)[1] + 0.5 * n * np.log(2 * np.pi)) / n
    assert r["nll"] == pytest.approx(nll, rel=2e-2)
    assert r["inv_quad"] == pytest.approx(y @ a, rel=1e-8)
    Ainv = np.linalg.inv(A)
    G = list(ok.kernel_gradients(ok.RBF, X, X, params, True)) + [np.eye(n)]
    exact = np.array([(-0.5 * a @ g @ a + 0.5 * np.trace(Ainv @ g)) / n for g in G])
    assert np.linalg.norm(r["grads"] - exact) < 0.1 * np.linalg.norm(exact)


# ------------------------------------------------------------------ prediction
def test_solve_alpha_matches_solve():
    rng = np.random.default_rng(9)
    _, _, _, A = _spd(rng, 70)
    b = rng.normal(size=70)
    # The absolute pAp < 1e-10 guard ends the solve once p is tiny, so the
    # achievable accuracy is limited by that guard rather than by tol.
    np.testing.assert_allclose(oe.solve_alpha(A, b, 500, 1e-12), np.linalg.solve(A, b), rtol=1e-4)
    np.testing.assert_allclose(oe.solve_alpha(A, 1e4 * b, 500, 1e-12),
                               np.linalg.solve(A, 1e4 * b), rtol=1e-8)


def test_lanczos_full_rank_root_inverts():
    rng = np.random.default_rng(10)
    n = 30
    _, _, _, A = _spd(rng, n, noise=0.3)
    S = oe.lanczos_inv_root(A, n)
    np.testing.assert_allclose(S @ S.T, np.linalg.inv(A), rtol=1e-6, atol=1e-8)


def test_love_full_rank_equals_exact_variance():
    rng = np.random.default_rng(11)
    n, d = 40, 2
    X = rng.uniform(-1, 1, size=(n, d))
    Xs = rng.uniform(-1.2, 1.2, size=(9, d))
    y = np.cos(X).sum(1)
    params = np.array([0.8, 1.2])
    mu, var, _ = oe.predict(ok.MATERN52, False, X, y, Xs, params, 0.3, 0.1, max_cg=500,
                            tol=1e-12, lanczos_rank=n)
    A = ok.kernel_matrix(ok.MATERN52, X, X, params, False) + 0.3 * np.eye(n)
    Ks = ok.kernel_matrix(ok.MATERN52, Xs, X, params, False)
    np.testing.assert_allclose(mu, Ks @ np.linalg.solve(A, y - 0.1) + 0.1, rtol=1e-5)
    exact = 1.2 - np.sum(Ks * np.linalg.solve(A, Ks.T).T, axis=1)
    np.testing.assert_allclose(var, exact, rtol=1e-6, atol=1e-9)


def test_love_fp32_full_rank_equals_exact_variance_to_fp32_rounding():
    """The fp32 restatement at full rank on a well-conditioned problem is the
    exact posterior variance to fp32 rounding (a dropped or transposed term
    would not be)."""
    rng = np.random.default_rng(12)
    n, d = 48, 2
    X = rng.uniform(-1, 1, size=(n, d))
    Xs = rng.uniform(-1.2, 1.2, size=(9, d))
    params = np.array([0.8, 1.2])
    var32 = oe.love_variance_fp32(ok.RBF, False, X, Xs, params, 0.5, lanczos_rank=n)
    assert var32.dtype == np.float32
    A = ok.kernel_matrix(ok.RBF, X, X, params, False) + 0.5 * np.eye(n)
    Ks = ok.kernel_matrix(ok.RBF, Xs, X, params, False)
    exact = 1.2 - np.sum(Ks * np.linalg.solve(A, Ks.T).T, axis=1)
    np.testing.assert_allclose(var32, exact, rtol=2e-5, atol=2e-6)


def test_love_fp32_floor_on_config1():
    """Config 1 (N = 2000, 1-D RBF, LOVE rank 100 at 128 test points) at the
    fitted hyperparameters: LOVE in the reference's fp32 arithmetic lands
    ~1.2e-4 (norm-wise) from the float64 LOVE on the predictive std.  Inside
    the data var ~2e-4 k**, so var = k** - ||K* S||^2 cancels ~5000-fold and
    the fp32 Lanczos root's rounding (~2e-6 k** in var) is ~1e-4 of std: no
    fp32 implementation of the method, the reference's included, can be held
    to 1e-4 of the float64 std there."""
    rng = np.random.default_rng(0)
    n = 2000
    X = np.linspace(-3, 3, n, dtype=np.float32)[:, None]
    y = (np.sin(2 * X[:, 0]) + 0.05 * rng.normal(size=n)).astype(np.float32)
    Xs = np.linspace(-4, 4, 128, dtype=np.float32)[:, None]
    # the config-1 fit's hyperparameters (oracle.engine.train, 50 iterations)
    params, noise, mean = np.array([1.0559015, 1.2796385]), 0.06235869, -0.005485322
    _, var, _ = oe.predict(ok.RBF, False, X, y, Xs, params, noise, mean, max_cg=300,
                           tol=1e-8, lanczos_rank=100)
    var32 = oe.love_variance_fp32(ok.RBF, False, X, Xs, params, noise, lanczos_rank=100)
    s, s32 = np.sqrt(var), np.sqrt(var32.astype(np.float64))
    floor = float(np.linalg.norm(s32 - s) / np.linalg.norm(s))
    print(f"config-1 LOVE std: fp32 reference-order vs float64 {floor:.3e}")
    assert floor >= 1e-4
    assert float(np.max(np.abs(var32 - var))) / params[-1] < 1e-5


def test_train_reduces_nll():
    rng = np.random.default_rng(12)
    n = 150
    X = np.linspace(-3, 3, n)[:, None]
    y = np.sin(2 * X[:, 0]) + 0.05 * rng.normal(size=n)
    res = oe.train(ok.RBF, False, X, y, [0.5, 1.0], 0.1, max_iterations=15, num_probes=8)
    h = res["nll_history"]
    assert np.all(np.isfinite(h)) and h[-1] < h[0]
    assert np.all(res["params"] > 0) and res["noise"] > 0

# ------------------------------------------------------------------ exact variance
def test_exact_variance_matches_dense_formula():
    rng = np.random.default_rng(8)
    X = rng.uniform(-2, 2, size=(150, 2))
    Xs = rng.uniform(-2.5, 2.5, size=(40, 2))
    params = np.array([0.9, 1.1, 1.3])
    noise = 0.04
    A = ok.kernel_matrix(ok.MATERN52, X, X, params, True) + noise * np.eye(150)
    Ks = ok.kernel_matrix(ok.MATERN52, X, Xs, params, True)
    dense = 1.3 - np.sum(Ks * np.linalg.solve(A, Ks), axis=0)
    for rank, block in ((0, 0), (20, 16)):
        var, k, iters = oe.exact_variance(ok.MATERN52, True, X, Xs, params, noise, max_cg=400,
                                          tol=1e-8, precond_rank=rank, block_cols=block)
        np.testing.assert_allclose(var, dense, rtol=1e-6, atol=1e-7)
        assert len(iters) == (1 if block == 0 else 3)
    # The Nystrom preconditioner cuts the iteration count.
    _, _, it0 = oe.exact_variance(ok.MATERN52, True, X, Xs, params, noise, tol=1e-6,
                                  precond_rank=0)
    _, _, it1 = oe.exact_variance(ok.MATERN52, True, X, Xs, params, noise, tol=1e-6,
                                  precond_rank=60)
    assert it1[0] < it0[0]



def test_precond_noise_vector_woodbury_logdet_and_probes():
    """P = L L^T + diag(d): apply == solve(P, .), log|P| == slogdet(P), and the
    probes L z_rank + sqrt(d) z_noise have covariance P (noise mode 1)."""
    rng = np.random.default_rng(21)
    n, r = 40, 6
    L = rng.normal(size=(n, r)) * 0.5
    d = rng.uniform(0.05, 0.4, size=n)
    P = oe.Precond(L, d)
    Pd = L @ L.T + np.diag(d)
    V = rng.normal(size=(n, 3))
    np.testing.assert_allclose(P.apply(V), np.linalg.solve(Pd, V), rtol=1e-9, atol=1e-12)
    assert P.logdet == pytest.approx(np.linalg.slogdet(Pd)[1], rel=1e-12)
    Z = P.sample(40000, 3)
    cov = Z @ Z.T / Z.shape[1]
    scale = np.sqrt(np.outer(np.diag(Pd), np.diag(Pd)))
    assert np.max(np.abs(cov - Pd) / scale) < 0.03


def test_bbmm_noise_vector_reaches_exact_nll():
    """With a fixed noise vector the BBMM NLL and kernel gradients converge to
    the exact values of K + diag(d) (many probes, tight CG)."""
    rng = np.random.default_rng(22)
    n = 30
    X = rng.uniform(-1, 1, size=(n, 2))
    y = np.sin(2 * X[:, 0]) + 0.1 * rng.normal(size=n)
    params = np.array([0.7, 1.2])
    d = rng.uniform(0.05, 0.3, size=n)
    r = oe.bbmm_step(ok.MATERN52, False, X, y, params, 123.0, None, 3000, 200, 60, 1e-10, 0,
                     noise_vec=d)
    A = ok.kernel_matrix(ok.MATERN52, X, X, params, False) + np.diag(d)
    al = np.linalg.solve(A, y)
    exact = (0.5 * y @ al + 0.5 * np.linalg.slogdet(A)[1] + 0.5 * n * np.log(2 * np.pi)) / n
    assert r["inv_quad"] == pytest.approx(y @ al, rel=1e-8)
    assert r["nll"] == pytest.approx(exact, rel=0.02)
    G = ok.kernel_gradients(ok.MATERN52, X, X, params, False)
    Ainv = np.linalg.inv(A)
    for q, g in enumerate(G):
        ex = (-0.5 * al @ g @ al + 0.5 * np.trace(Ainv @ g)) / n
        assert r["grads"][q] == pytest.approx(ex, abs=0.05 * abs(ex) + 2e-3)
