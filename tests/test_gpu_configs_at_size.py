"""The benchmark configurations at their stated sizes,
end to end through the public surface, checked against the float64
restatement on sampled rows and through size-independent properties.

The restatement cannot solve these systems densely (config 3 is a
250 000-point system), so each test checks what the oracle can evaluate at
full size:
* kernel products on sampled rows (oracle.kernels.forward_matvec / cross_matvec
  in float64) at the north star's 1e-5;
* the predictive mean given the engine's own alpha, on sampled test points;
* the residual ||(K + s^2 I) alpha - (y - mu)|| of the prediction solve on
  sampled rows, against the solve's tolerance;
* finite NLL histories, CG counts within max_cg, a decreasing NLL;
* variances in (0, outputscale], LOVE >= exact variance (the Lanczos
  approximation Q T^-1 Q^T of A^-1 is a projection, so it never exceeds A^-1),
  and exact variance agreeing across independent routes.
Every case prints its progress so a long run shows where it is.
"""

import sys
import time

import numpy as np
import pytest

from mojogp_amd import RBF, Matern52, MultiOutputLMCGP, SingleOutputGP
from mojogp_amd import _engine, _lib
from mojogp_amd._provider import KIND_RBF, NativeProvider
from oracle import kernels as ok
from oracle import lmc as ol

pytestmark = pytest.mark.gpu


def _log(msg):
    print(msg, flush=True)
    sys.__stderr__.write(msg + "\n")
    sys.__stderr__.flush()


def _rel(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def _progress(tag):
    t0 = time.perf_counter()

    def cb(ev):
        st = ev.get("stats", {})
        if ev.get("current", 0) % 5 == 0 or ev.get("current") == ev.get("total"):
            _log(f"  {tag} iter {ev.get('current')}/{ev.get('total')} nll {st.get('nll')} "
                 f"cg {st.get('cg_iter')} t {time.perf_counter() - t0:.1f}s")
    return cb


def _alpha_residual(kind, ard, X, y, mean, params, noise, alpha, rows):
    """||(K + s^2 I) alpha - (y - mu)|| / ||y - mu|| over the sampled rows (float64)."""
    Ka = ok.forward_matvec(kind, X, alpha[None, :], params, noise, ard, rows=rows, block=64)[0]
    b = y[rows].astype(np.float64) - mean
    return float(np.linalg.norm(Ka - b) / np.linalg.norm(b))


def _mean_check(kind, ard, Xs, X, alpha, params, mu, mean, tag):
    """Predictive mean given the engine's alpha against float64 K(X*, X) alpha + mu.
    The bar is relative to K(X*, X)|alpha| (kernel values are positive): the
    rounding of a sum of n fp32 products scales with the sum of their
    magnitudes, which a cancelling alpha (small noise) makes much larger than
    the result itself."""
    ref = ok.cross_matvec(kind, Xs, X, alpha[None, :], params, ard)[0] + mu
    mag = ok.cross_matvec(kind, Xs, X, np.abs(alpha)[None, :], params, ard)[0]
    plain = _rel(mean, ref)
    scaled = float(np.linalg.norm(np.asarray(mean, np.float64) - ref) / np.linalg.norm(mag))
    _log(f"  {tag}: mean on {len(Xs)} test points vs float64: {plain:.2e} relative, "
         f"{scaled:.2e} of ||K*|alpha|||")
    assert scaled <= 1e-5


def _fit_checks(tr, info, iters, max_cg):
    h = np.asarray(tr.nll_history, np.float64)
    cg = np.asarray(info["cg_iterations_history"])
    assert len(h) == iters and np.all(np.isfinite(h))
    assert cg.size == iters and cg.max() <= max_cg and cg.min() >= 1
    assert h[-1] < h[0]
    return h, cg


# ----------------------------------------------------------------- config 3
def _c3_data():
    """Config 3: X ~ N(0, I) [250000 x 16]; y an RBF random-Fourier-feature draw
    (1024 features, lengthscale 2) + 0.05 N(0, 1); 10 000 test points."""
    rng = np.random.default_rng(0)
    n, d = 250_000, 16
    X = rng.normal(size=(n, d)).astype(np.float32)
    W = rng.normal(size=(1024, d)) / 2.0
    b = rng.uniform(0, 2 * np.pi, size=1024)
    w = rng.normal(size=1024)

    def f(Z):
        return np.sqrt(2.0 / 1024) * np.cos(Z @ W.T + b) @ w

    y = (f(X) + 0.05 * rng.normal(size=n)).astype(np.float32)
    Xs = rng.normal(size=(10_000, d)).astype(np.float32)
    return X, y, Xs, f


def test_config3_fit_and_love_predict_at_size():
    X, y, Xs, f = _c3_data()
    n = X.shape[0]
    _log("config 3: Matern-5/2 ARD N=250000 d=16, 50 iterations, 15 probes, rank 200")
    gp = SingleOutputGP(Matern52(ard=True))
    t0 = time.perf_counter()
    tr = gp.fit(X, y, method="matrix_free", max_iterations=50, num_probes=15,
                cg_tolerance=1e-2, preconditioner_rank=200, progress=_progress("c3"))
    fit_s = time.perf_counter() - t0
    info = gp.backend_train_info
    assert info["precond_rank"] == 200 and info["use_preconditioner"] is True
    h, cg = _fit_checks(tr, info, 50, 100)
    _log(f"  fit {fit_s:.1f}s, NLL {h[0]:.5f} -> {h[-1]:.5f}, CG total {cg.sum()}")

    t0 = time.perf_counter()
    mean, var = gp.predict(Xs, return_var=True, variance_method="love")
    pinfo = gp.backend_predict_info
    _log(f"  LOVE predict {time.perf_counter() - t0:.1f}s, alpha CG "
         f"{pinfo['alpha_cg_iterations']} iterations, rank {pinfo['max_root_decomposition_size']}")
    params = np.asarray(gp.kernel.to_engine_params(np.asarray(tr.params, np.float32)),
                        np.float64)
    os_ = float(params[-1])
    mu = float(gp._engine_predict_mean if gp._engine_predict_mean is not None else tr.mean)
    assert np.all(np.isfinite(mean)) and np.all(var > 0) and np.all(var <= os_ * (1 + 1e-6))
    alpha = np.asarray(gp._cached_alpha, np.float64)
    rng = np.random.default_rng(11)

    # predictive mean given the engine's alpha: float64 K(X*, X) alpha + mu
    sub = np.sort(rng.choice(Xs.shape[0], size=256, replace=False))
    _mean_check(ok.MATERN52, True, Xs[sub], X, alpha, params, mu, mean[sub], "config 3")

    # the prediction solve's residual on sampled rows
    rows = np.sort(rng.choice(n, size=192, replace=False))
    res = _alpha_residual(ok.MATERN52, True, X, y, mu, params, tr.noise, alpha, rows)
    _log(f"  alpha residual on 192 rows: {res:.2e} (tolerance {pinfo['cg_tolerance']})")
    if pinfo["alpha_cg_iterations"] < pinfo["max_cg_iterations"]:
        assert res <= 2.0 * pinfo["cg_tolerance"]

    # LOVE against the exact variance on 64 test points
    sub64 = sub[:64]
    t0 = time.perf_counter()
    _, var_ex = gp.predict(Xs[sub64], return_var=True, variance_method="exact")
    einfo = gp.backend_predict_info
    gap = (var[sub64] - var_ex) / var_ex
    _log(f"  exact variance on 64 points {time.perf_counter() - t0:.1f}s "
         f"({einfo.get('exact_cg_total_iterations')} CG iterations); LOVE - exact relative: "
         f"min {gap.min():.2e} max {gap.max():.2e} median {np.median(gap):.2e}")
    assert np.all(var_ex > 0) and np.all(var_ex <= os_ * (1 + 1e-6))
    # LOVE at rank 200 on a 250k-point system keeps 15%-130% of the variance
    # reduction the exact solve removes (measured): the Krylov space of a
    # fixed start vector holds only part of each k*; the one-sided bound is
    # what the method guarantees
    assert gap.min() >= -1e-3
    rmse = float(np.sqrt(np.mean((mean - f(Xs)) ** 2)))
    _log(f"  test RMSE against the noiseless draw: {rmse:.4f} (std of f: {np.std(f(Xs)):.4f})")


# ----------------------------------------------------------------- config 2
def test_config2_forward_product_sampled_rows(monkeypatch):
    """Config 2's forward product at size (N = 50 000, d = 8, RBF ARD, t = 16):
    the automatic route is the symmetric kernel (98 blocks of 512 points, an
    even count, so the last delta step pairs half the blocks) -- shown by its
    output equalling the forced symmetric route's bit for bit -- and it and
    the one-sided tile route each match float64 on 192 sampled rows at 1e-5,
    at the fit's starting hyperparameters and at shorter lengthscales."""
    rng = np.random.default_rng(0)
    n, d, t = 50_000, 8, 16
    X = rng.uniform(size=(n, d)).astype(np.float32)
    V = rng.normal(size=(t, n)).astype(np.float32)
    rows = np.sort(np.random.default_rng(5).choice(n, size=192, replace=False))
    for params in (np.concatenate([np.ones(d), [1.0]]),
                   np.concatenate([rng.uniform(0.3, 0.8, d), [1.3]])):
        params = params.astype(np.float32)
        _log(f"config 2 forward product, lengthscales {np.round(params[:d], 3)}")
        ref = ok.forward_matvec(ok.RBF, X, V, params, 0.1, True, rows=rows, block=64)
        p = NativeProvider(ok.RBF, True, X, params, 0.1)
        try:
            monkeypatch.delenv("MGP_SYM_MATVEC", raising=False)
            auto = p.forward_matvec(V)
            monkeypatch.setenv("MGP_SYM_MATVEC", "1")
            sym = p.forward_matvec(V)
            monkeypatch.setenv("MGP_SYM_MATVEC", "0")
            one = p.forward_matvec(V)
            monkeypatch.delenv("MGP_SYM_MATVEC")
        finally:
            p.close()
        e_sym, e_one = _rel(auto[:, rows], ref), _rel(one[:, rows], ref)
        _log(f"  symmetric (automatic) {e_sym:.2e}, one-sided {e_one:.2e} on 192 rows")
        assert np.array_equal(auto, sym) and not np.array_equal(auto, one)
        assert e_sym <= 1e-5 and e_one <= 1e-5


def test_config3_gradient_trace_sampled_rows(monkeypatch):
    """Config 3's gradient trace at size (N = 250 000, d = 16, Matern-5/2 ARD,
    16 weight columns): the BBMM gradient step's trace
    g_p = sum_ab dK_p[a, b] sum_c Lf[c, a] Rf[c, b], with Lf nonzero on 96
    sampled rows only, equals sum over those rows of Lf . (dK_p Rf), which the
    float64 oracle evaluates at full size.  Checked for the matrix-core trace
    (k_grad_sym, the route taken at this size) and the pair loop."""
    rng = np.random.default_rng(0)
    n, d, t = 250_000, 16, 16
    X = rng.normal(size=(n, d)).astype(np.float32)
    params = np.concatenate([np.full(d, 1.0), [1.0]]).astype(np.float32)
    rows = np.sort(rng.choice(n, size=96, replace=False))
    L = np.zeros((t, n), np.float32)
    L[:, rows] = rng.normal(size=(t, rows.size))
    R = rng.normal(size=(t, n)).astype(np.float32)
    _log("config 3 gradient trace: N=250000 d=16 Matern-5/2 ARD, 16 columns")
    p = NativeProvider(ok.MATERN52, True, X, params, 0.1)
    try:
        monkeypatch.delenv("MGP_GRAD_MFMA", raising=False)
        g_mfma = p.gradient_trace(L, R)
        monkeypatch.setenv("MGP_GRAD_MFMA", "0")
        g_loop = p.gradient_trace(L, R)
        monkeypatch.delenv("MGP_GRAD_MFMA")
    finally:
        p.close()
    G = ok.gradient_matvec(ok.MATERN52, X, R, params, True, rows=rows, block=8)
    ref = np.einsum("pcr,cr->p", G, L[:, rows].astype(np.float64))
    e_m, e_l = _rel(g_mfma, ref), _rel(g_loop, ref)
    _log(f"  matrix-core trace {e_m:.2e}, pair loop {e_l:.2e} against float64 "
         f"(per-parameter max {np.max(np.abs(g_mfma - ref) / np.abs(ref)):.2e})")
    assert e_m <= 2e-5 and e_l <= 5e-6    # measured 3.8e-6 and 5.4e-7


def test_config2_fit_and_predict_at_size():
    rng = np.random.default_rng(0)
    n, d = 50_000, 8
    X = rng.uniform(size=(n, d)).astype(np.float32)
    y = (np.sin(3 * X).sum(1) + 0.1 * rng.normal(size=n)).astype(np.float32)
    Xs = rng.uniform(size=(2000, d)).astype(np.float32)
    _log("config 2: RBF ARD N=50000 d=8, 30 iterations, 15 probes, rank 100 greedy")
    gp = SingleOutputGP(RBF(ard=True))
    t0 = time.perf_counter()
    tr = gp.fit(X, y, max_iterations=30, method="matrix_free", num_probes=15,
                preconditioner_rank=100, preconditioner="greedy", progress=_progress("c2"))
    info = gp.backend_train_info
    h, cg = _fit_checks(tr, info, 30, 100)
    _log(f"  fit {time.perf_counter() - t0:.1f}s, NLL {h[0]:.5f} -> {h[-1]:.5f}, "
         f"CG total {cg.sum()}")
    assert info["precond_rank"] == 100

    mean, var = gp.predict(Xs, return_var=True)
    pinfo = gp.backend_predict_info
    params = np.asarray(gp.kernel.to_engine_params(np.asarray(tr.params, np.float32)),
                        np.float64)
    mu = float(gp._engine_predict_mean if gp._engine_predict_mean is not None else tr.mean)
    assert np.all(var > 0) and np.all(var <= params[-1] * (1 + 1e-6))
    alpha = np.asarray(gp._cached_alpha, np.float64)
    r2 = np.random.default_rng(12)
    sub = np.sort(r2.choice(Xs.shape[0], size=256, replace=False))
    _mean_check(ok.RBF, True, Xs[sub], X, alpha, params, mu, mean[sub], "config 2")
    rows = np.sort(r2.choice(n, size=192, replace=False))
    res = _alpha_residual(ok.RBF, True, X, y, mu, params, tr.noise, alpha, rows)
    _log(f"  alpha residual on 192 rows: {res:.2e} after {pinfo['alpha_cg_iterations']} "
         f"iterations (tolerance {pinfo['cg_tolerance']})")
    if pinfo["alpha_cg_iterations"] < pinfo["max_cg_iterations"]:
        assert res <= 2.0 * pinfo["cg_tolerance"]
    # the model explains the signal: test RMSE far below the signal's spread
    ftrue = np.sin(3 * Xs).sum(1)
    rmse = float(np.sqrt(np.mean((mean - ftrue) ** 2)))
    _log(f"  test RMSE {rmse:.4f} (signal std {np.std(ftrue):.4f})")
    assert rmse < 0.2 * np.std(ftrue)


# ----------------------------------------------------------------- config 4
def test_config4_materialized_fit_and_exact_variance_at_size():
    rng = np.random.default_rng(0)
    n, d, m = 40_000, 4, 4096
    X = rng.uniform(-2, 2, size=(n, d)).astype(np.float32)
    y = (np.prod(np.cos(X), axis=1) + 0.05 * rng.normal(size=n)).astype(np.float32)
    Xs = rng.uniform(-2, 2, size=(m, d)).astype(np.float32)
    _log("config 4: RBF N=40000 d=4, materialized (dense K 6.4 GB), defaults")
    gp = SingleOutputGP(RBF())
    t0 = time.perf_counter()
    tr = gp.fit(X, y, method="materialized", progress=_progress("c4"))
    info = gp.backend_train_info
    assert info["training_route"] == "materialized"
    iters = len(tr.nll_history)
    h, cg = _fit_checks(tr, info, iters, info["max_cg_iter"])
    _log(f"  fit {time.perf_counter() - t0:.1f}s, {iters} iterations, NLL {h[0]:.5f} -> "
         f"{h[-1]:.5f}, CG total {cg.sum()}")
    params = np.asarray(gp.kernel.to_engine_params(np.asarray(tr.params, np.float32)),
                        np.float64)
    os_ = float(params[-1])

    # the dense product at full size (fill + GEMM) on sampled rows
    r2 = np.random.default_rng(13)
    V = r2.normal(size=(16, n)).astype(np.float32)
    prov = NativeProvider(KIND_RBF, False, X, params.astype(np.float32), float(tr.noise))
    try:
        _lib.call("mgp_materialize", prov.handle)
        got = prov.forward_matvec(V)
    finally:
        prov.close()
    rows = np.sort(r2.choice(n, size=192, replace=False))
    ref = ok.forward_matvec(ok.RBF, X, V, params, float(tr.noise), False, rows=rows, block=64)
    err = max(_rel(got[c, rows], ref[c]) for c in range(16))
    _log(f"  materialized (K + s^2 I) V on 192 rows, 16 columns: max relerr {err:.2e}")
    assert err <= 1e-5

    t0 = time.perf_counter()
    mean, var = gp.predict(Xs, return_var=True, variance_method="exact")
    einfo = gp.backend_predict_info
    _log(f"  exact variance at {m} points {time.perf_counter() - t0:.1f}s: "
         f"{einfo.get('exact_cg_block_count')} blocks, "
         f"{einfo.get('exact_cg_total_iterations')} CG iterations")
    assert np.all(var > 0) and np.all(var <= os_ * (1 + 1e-6))
    mu = float(gp._engine_predict_mean if gp._engine_predict_mean is not None else tr.mean)
    alpha = np.asarray(gp._cached_alpha, np.float64)
    sub = np.sort(r2.choice(m, size=256, replace=False))
    _mean_check(ok.RBF, False, Xs[sub], X, alpha, params, mu, mean[sub], "config 4")

    # exact variance of 64 points through both routes at a tight tolerance:
    # the dense K with its GEMM, and the matrix-free fused tile products.  At
    # this noise level var = k** - k*^T A^-1 k* cancels to ~1e-3 of k**, so
    # the prediction default (tolerance 1e-3) leaves a large relative error in
    # var; the gap to the tight solve is reported.
    s64 = sub[:64]
    _, var_d = gp.predict(Xs[s64], return_var=True, variance_method="exact",
                          cg_tolerance=1e-6, max_cg_iterations=2000)
    it_d = gp.backend_predict_info.get("exact_cg_total_iterations")
    km = _engine.load_kernel_module("rbf", False, d)
    eng = _engine.load_engine()
    pinfo = km.init_provider(X, params.astype(np.float32), float(tr.noise))
    try:
        r = eng.predict(pinfo, y, Xs[s64], params.astype(np.float32), float(tr.noise), mu,
                        2, 2000, 1e-6, int(info["precond_rank"]), 0, True, 0)
    finally:
        km.destroy_provider(pinfo)
    _log(f"  exact variance at tolerance 1e-6 on 64 points ({it_d} / "
         f"{r.get('exact_cg_total_iterations')} CG iterations): dense vs matrix-free route "
         f"{_rel(var_d, r['variance']):.2e}; default tolerance vs 1e-6: "
         f"{_rel(var[s64], var_d):.2e}; var / k** median {np.median(var_d) / os_:.2e}")
    # the solves agree on k*^T A^-1 k* (of size ~k**) to fp32 accuracy
    assert np.max(np.abs(var_d - r["variance"])) <= 1e-5 * os_


# ----------------------------------------------------------------- config 5
def _c5_data():
    """Config 5: X ~ U[0,1]^{20000 x 6}; latents RBF (l = 0.2) and Matern-5/2
    (l = 0.7) random-Fourier-feature draws; W ~ N(0,1)^{4x2}; Y = F W^T + 0.05 N."""
    rng = np.random.default_rng(0)
    n, d, T = 20_000, 6, 4
    X = rng.uniform(0, 1, size=(n, d)).astype(np.float32)

    def rff(ls, matern):
        Wf = rng.standard_normal((1024, d))
        if matern:
            Wf = Wf / np.sqrt(rng.chisquare(5, size=(1024, 1)) / 5.0)
        b = rng.uniform(0, 2 * np.pi, size=1024)
        w = rng.standard_normal(1024)
        return lambda Z: np.sqrt(2.0 / 1024) * np.cos(Z / ls @ Wf.T + b) @ w

    f1, f2 = rff(0.2, False), rff(0.7, True)
    Wm = rng.standard_normal((T, 2))
    Y = (np.stack([f1(X), f2(X)], 1) @ Wm.T
         + 0.05 * rng.standard_normal((n, T))).astype(np.float32)
    Xs = rng.uniform(0, 1, size=(1000, d)).astype(np.float32)
    return X, Y, Xs


def test_config5_lmc_product_fit_and_pathwise_at_size():
    X, Y, Xs = _c5_data()
    n, T = Y.shape
    C = 16
    kinds, ards = [ok.RBF, ok.MATERN52], [False, False]
    params = [np.array([0.2, 1.0], np.float32), np.array([0.7, 1.0], np.float32)]
    rng = np.random.default_rng(14)
    A = np.stack([np.outer(w, w) + 0.1 * np.eye(T) for w in rng.normal(size=(2, T))])
    A = A.astype(np.float32)
    noise = np.full(T, 0.0025, np.float32)
    V = rng.standard_normal((C, T * n)).astype(np.float32)
    _log("config 5: LMC structured product N=20000 T=4 Q=2, 16 task-blocked columns")
    provs = [NativeProvider(k, a, X, p, 0.0) for k, a, p in zip(kinds, ards, params)]
    out = np.zeros_like(V)
    try:
        _lib.call("mgp_lmc_forward_matvec", _lib.handles(provs), 2, T, _lib.fptr(A),
                  _lib.fptr(noise), None, _lib.fptr(V), C, _lib.fptr(out))
    finally:
        for p in provs:
            p.close()
    rows = np.sort(rng.choice(n, size=128, replace=False))
    Vb = V.reshape(C, T, n).astype(np.float64)
    ref = np.zeros((C, T, rows.size))
    for s in range(2):
        Ks = ok.kernel_matrix(kinds[s], X[rows], X, params[s].astype(np.float64), ards[s])
        KV = np.einsum("rj,ctj->ctr", Ks, Vb)            # [C][T'][rows]
        ref += np.einsum("tu,cur->ctr", A[s].astype(np.float64), KV)
    ref += noise[None, :, None] * Vb[:, :, rows]
    got = out.reshape(C, T, n)[:, :, rows]
    err = max(_rel(got[c], ref[c]) for c in range(C))
    _log(f"  structured product on 128 rows x 4 tasks: max column relerr {err:.2e}")
    assert err <= 1e-5

    _log("config 5: MultiOutputLMCGP fit (matrix-free, 15 probes) + 64 pathwise samples")
    gp = MultiOutputLMCGP(kernels=["rbf", "matern52"], num_probes=15)
    t0 = time.perf_counter()
    res = gp.fit(X, Y, method="matrix_free")
    h = np.asarray(res.nll_history, np.float64)
    _log(f"  fit {time.perf_counter() - t0:.1f}s, {res.iterations} iterations, "
         f"NLL {h[0]:.5f} -> {h[-1]:.5f}")
    assert np.all(np.isfinite(h)) and h[-1] < h[0]
    r = gp._result
    lat = [np.asarray(p, np.float64) for p in r.params_per_latent]
    Ar = np.asarray(r.A_matrices, np.float64)
    mu_t = np.asarray(gp._fitted_mean, np.float64)
    mean, var = gp.predict(Xs, return_var=True)
    assert np.all(np.isfinite(mean)) and np.all(var > 0)
    # predict()'s mean is the structured cross product of the training alpha
    # (multi_output_gp.py:5635-5726 reuses it): float64 on 64 test points,
    # bounded by the magnitudes of the summed products
    al = np.asarray(r.alpha, np.float64)
    ref_m = ol.predict_mean(kinds, ards, X, Xs[:64], lat, Ar, al, mu_t)
    mag = ol.predict_mean(kinds, ards, X, Xs[:64], lat, np.abs(Ar), np.abs(al), np.zeros(T))
    scaled = float(np.linalg.norm(mean[:64] - ref_m) / np.linalg.norm(mag))
    _log(f"  predict mean vs float64 from the training alpha: {_rel(mean[:64], ref_m):.2e} "
         f"relative, {scaled:.2e} of the product magnitudes")
    assert scaled <= 1e-5

    # Pathwise samples.  The reference's defaults (training tolerance 1.0,
    # 200 CG iterations) leave both the training alpha and the correction
    # solve unconverged on this system (~4000 iterations reach 1e-2), so the
    # samples are checked at a converging budget: their mean must be the
    # posterior mean re-solved through the same correction entry point with
    # y - mu as the one residual.
    gp.max_cg_iter, gp.cg_tol = 8000, 1e-3
    y_c = (Y - mu_t[None, :]).astype(np.float32)
    acc = gp._engine.sample_lmc_pathwise(gp._ensure_providers(), y_c, r.A_matrices, Xs,
                                         [np.asarray(p, np.float32) for p in r.params_per_latent],
                                         np.asarray(r.noise_per_task, np.float32), 8000, 1e-3)
    post_mean = mu_t[None, :] + np.asarray(acc["correction"], np.float64).reshape(-1, T)
    _log(f"  posterior mean re-solved in {acc['cg_iterations']} CG iterations; predict() mean "
         f"(training alpha) vs re-solved: {_rel(mean, post_mean):.2e}")
    t0 = time.perf_counter()
    S = gp.sample_posterior(Xs, n_samples=64, method="pathwise", rng=np.random.default_rng(1))
    S = np.asarray(S, np.float64)
    _log(f"  64 pathwise samples {time.perf_counter() - t0:.1f}s, shape {S.shape}")
    assert S.shape == (64, Xs.shape[0], T) and np.all(np.isfinite(S))
    svar = S.var(0, ddof=1)
    z = (S.mean(0) - post_mean) / np.sqrt(svar / 64)
    _log(f"  z = (sample mean - posterior mean) / (sample sd / 8): mean square "
         f"{np.mean(z ** 2):.3f}, max |z| {np.max(np.abs(z)):.2f}; sample variance / "
         f"predict() variance median {np.median(svar / var):.2e} (the LMC LOVE recipe adds "
         f"the task noise and uses the average noise per latent)")
    assert np.mean(z ** 2) < 4.0
    assert np.mean(np.abs(z) < 4.0) > 0.97
