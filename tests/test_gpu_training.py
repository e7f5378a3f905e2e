"""GPU parity of the training loop and the prediction cache against the CPU
restatement (oracle/engine.py, whose loop is pinned in test_oracle_training.py
by torch.optim.Adam and known answers).

* Config 1 exactly as stated (N = 2000, 1-D RBF, 50 Adam iterations, LOVE at
  128 test points): NLL history, parameters, noise and mean within 1e-4.
* NaN recovery (jit_training.mojo:605-685) forced from the host with the
  engine's nan_inject_mask: halved rate, best-snapshot restore of parameters,
  moments and mean, preconditioner rebuild — on the restatement's trajectory.
* Cosine annealing (training_utils.mojo:23-40) and early stopping
  (jit_training.mojo:884-905).
* prepare_prediction_cache / predict_with_cache / destroy_prediction_cache
  (jit_engine_bindings.mojo:636-942) for a single kernel and a kernel tree.
"""

import sys

import numpy as np
import pytest

from mojogp_amd import RBF, RQ, Matern52, SingleOutputGP
from mojogp_amd import _engine
from mojogp_amd._lib import NativeCallError
from oracle import engine as oe
from oracle import kernels as ok

pytestmark = pytest.mark.gpu


def _rel(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def _log(msg):
    print(msg, flush=True)
    sys.__stderr__.write(msg + "\n")
    sys.__stderr__.flush()


def _c1_data(n=2000):
    """Config 1 (README.md:94-104): X = linspace(-3, 3, 2000), y = sin(2x) +
    0.05 N(0, 1) with seed 0; test points linspace(-4, 4, 128)."""
    rng = np.random.default_rng(0)
    X = np.linspace(-3, 3, n, dtype=np.float32)[:, None]
    y = (np.sin(2 * X[:, 0]) + 0.05 * rng.normal(size=n)).astype(np.float32)
    Xs = np.linspace(-4, 4, 128, dtype=np.float32)[:, None]
    return X, y, Xs


def test_config1_fit_and_love_predict_at_size():
    X, y, Xs = _c1_data()
    _log("config 1: N=2000 RBF, 50 iterations, matrix-free fit")
    gp = SingleOutputGP(RBF())
    tr = gp.fit(X, y, max_iterations=50, method="matrix_free")
    info = gp.backend_train_info
    assert info["use_preconditioner"] is False and info["precond_rank"] == 0
    ref = oe.train(ok.RBF, False, X, y, [1.0, 1.0], 0.1, max_iterations=50, num_probes=10,
                   max_cg=100, cg_tol=1e-2, precond_rank=0, max_tridiag=30)
    h, rh = np.asarray(tr.nll_history, np.float64), ref["nll_history"]
    _log(f"  params {tr.params} vs {ref['params']}; noise {tr.noise:.7g} vs "
         f"{ref['noise']:.7g}; mean {tr.mean:.7g} vs {ref['mean']:.7g}; max NLL history "
         f"relerr {np.max(np.abs(h - rh) / np.abs(rh)):.2e}")
    assert len(h) == 50
    np.testing.assert_array_equal(tr.cg_iterations_history, ref["cg_iterations_history"])
    np.testing.assert_allclose(h, rh, rtol=1e-4)
    assert tr.nll == pytest.approx(ref["final_nll"], rel=1e-4)
    # Parameters after 50 Adam steps carry the fp32 rounding of the CG solves
    # (measured 2.0e-4; the restatement itself moves by 2.0e-4 when its CG
    # runs in fp32, test_oracle_training.py::test_c1_fp32_rounding_floor)
    np.testing.assert_allclose(tr.params, ref["params"], rtol=5e-4)
    assert tr.noise == pytest.approx(ref["noise"], rel=1e-4)
    # the mean sits near 0 (y is centred): compare on the scale of y
    assert abs(tr.mean - ref["mean"]) <= 1e-4 * float(np.std(y))

    mean, std = gp.predict(Xs, return_std=True, variance_method="love")
    params = np.asarray(tr.params, np.float64)
    mu, var, _ = oe.predict(ok.RBF, False, X, y, Xs, params, tr.noise, tr.mean, max_cg=300,
                            tol=1e-3, lanczos_rank=100)
    kss = float(tr.params[-1])
    var_err = float(np.max(np.abs(std.astype(np.float64) ** 2 - var))) / kss
    _log(f"  LOVE std relerr {_rel(std, np.sqrt(var)):.2e}, variance error {var_err:.2e} of "
         f"k**, mean relerr {_rel(mean, mu):.2e}")
    # var = k** - ||K* S||^2 cancels ~5000-fold inside the data (var ~2e-4
    # k**), so the float64 std is out of fp32's reach at 1e-4 there: LOVE in
    # the reference's own fp32 arithmetic and order lands ~1.2e-4 from it
    # (oracle.engine.love_variance_fp32; pinned on the CPU by
    # test_oracle_engine.py::test_love_fp32_floor_on_config1).  The device
    # must be at least as close to float64 as that restatement, and within
    # 1e-5 k** on the variance itself.
    var32 = oe.love_variance_fp32(ok.RBF, False, X, Xs, params, tr.noise, lanczos_rank=100)
    floor = _rel(np.sqrt(var32.astype(np.float64)), np.sqrt(var))
    std_err = _rel(std, np.sqrt(var))
    _log(f"  LOVE std relerr {std_err:.2e} (fp32 reference-order restatement: {floor:.2e})")
    assert var_err <= 1e-5
    assert std_err <= max(1e-4, floor)
    # predictions of the two fits (GPU hyperparameters vs the restatement's),
    # both evaluated in float64
    mu_r, var_r, _ = oe.predict(ok.RBF, False, X, y, Xs, np.asarray(ref["params"], np.float64),
                                ref["noise"], ref["mean"], max_cg=300, tol=1e-8,
                                lanczos_rank=100)
    mu_g, var_g, _ = oe.predict(ok.RBF, False, X, y, Xs, params, tr.noise, tr.mean,
                                max_cg=300, tol=1e-8, lanczos_rank=100)
    _log(f"  fitted-model predictions: mean {_rel(mu_g, mu_r):.2e}, "
         f"std {_rel(np.sqrt(var_g), np.sqrt(var_r)):.2e}")
    assert _rel(mu_g, mu_r) <= 1e-4
    assert _rel(np.sqrt(var_g), np.sqrt(var_r)) <= 1e-4
    # alpha CG stops at relative residual 1e-3: two correct solves (fp32 /
    # fp64) agree on the mean only to about that; at 1e-6 the bar is 1e-4
    assert _rel(mean, mu) <= 5e-3
    mean_t, _ = gp.predict(Xs, return_std=True, cg_tolerance=1e-6)
    mu_t, _, _ = oe.predict(ok.RBF, False, X, y, Xs, params, tr.noise, tr.mean, max_cg=300,
                            tol=1e-6, lanczos_rank=100)
    _log(f"  tight-tolerance mean relerr {_rel(mean_t, mu_t):.2e}")
    assert _rel(mean_t, mu_t) <= 1e-4


def _hello(n=400):
    rng = np.random.default_rng(0)
    X = np.linspace(-3, 3, n, dtype=np.float32)[:, None]
    y = (np.sin(2 * X[:, 0]) + 0.05 * rng.normal(size=n)).astype(np.float32)
    return X, y


def _engine_train(X, y, init, noise, iters, lr, rank, *, cosine=False, es=False,
                  patience=10, es_tol=1e-4, nan_mask=0):
    km = _engine.load_kernel_module("rbf", False, X.shape[1])
    eng = _engine.load_engine()
    info = km.init_provider(X, np.asarray(init, np.float32), noise)
    try:
        return eng.train(info, y, np.asarray(init, np.float32), noise, iters, lr, 10, 100, 1e-2,
                         rank, False, cosine, rank > 0, 30, 0.5, 0,
                         float(np.mean(y)), es, patience, es_tol,
                         nan_inject_mask=nan_mask)
    finally:
        km.destroy_provider(info)


def _check_trajectory(got, ref, tag, lr):
    h, rh = np.asarray(got["nll_history"], np.float64), ref["nll_history"]
    _log(f"  {tag}: {len(h)} NLLs, max relerr "
         f"{np.max(np.abs(h - rh) / np.abs(rh)) if len(h) == len(rh) else float('nan'):.2e}; "
         f"params {got['params']} vs {ref['params']}")
    assert len(h) == len(rh)
    np.testing.assert_array_equal(got["cg_iterations_history"], ref["cg_iterations_history"])
    np.testing.assert_allclose(h, rh, rtol=1e-4)
    np.testing.assert_allclose(got["params"], ref["params"], rtol=1e-4)
    assert got["noise"] == pytest.approx(ref["noise"], rel=1e-4)
    # the constant mean's gradient -sum(alpha)/n is ~0 on centred y, so its
    # Adam steps are sign-normalised noise: compare on the scale of one step
    assert abs(got["mean"] - ref["mean"]) <= 1e-2 * lr
    assert got["final_nll"] == pytest.approx(ref["final_nll"], rel=1e-4)


def test_nan_recovery_matches_oracle():
    """Forced NaN NLLs at iterations 3, 4 and 9 with a rank-15 preconditioner:
    the GPU loop restores the best snapshot, halves the rate and rebuilds the
    preconditioner exactly where the restatement does."""
    X, y = _hello()
    nan_at = (3, 4, 9)
    _log("NaN recovery: n=400, rank 15, NaN at iterations 3, 4, 9")
    got = _engine_train(X, y, [0.5, 1.0], 0.1, 14, 0.05, 15,
                        nan_mask=sum(1 << i for i in nan_at))
    ref = oe.train(ok.RBF, False, X, y, [0.5, 1.0], 0.1, max_iterations=14, learning_rate=0.05,
                   num_probes=10, max_cg=100, cg_tol=1e-2, precond_rank=15, max_tridiag=30,
                   nan_iterations=nan_at)
    _check_trajectory(got, ref, "nan recovery", 0.05)
    assert len(got["nll_history"]) == 14 - len(nan_at)
    assert len(got["cg_iterations_history"]) == 14
    for i in nan_at:
        assert i in got["precond_rebuild_steps"]
    assert got["precond_rebuild_steps"] == ref["precond_rebuild_steps"]


def test_cosine_lr_matches_oracle():
    X, y = _hello()
    _log("cosine LR: n=400, 16 iterations, NaN at iteration 5")
    got = _engine_train(X, y, [0.5, 1.0], 0.1, 16, 0.08, 0, cosine=True, nan_mask=1 << 5)
    ref = oe.train(ok.RBF, False, X, y, [0.5, 1.0], 0.1, max_iterations=16, learning_rate=0.08,
                   num_probes=10, max_cg=100, cg_tol=1e-2, precond_rank=0, max_tridiag=30,
                   use_cosine_lr=True, nan_iterations=(5,))
    _check_trajectory(got, ref, "cosine", 0.08)


def test_early_stopping_matches_oracle():
    """Patience 2, tolerance 0.02: the restatement stops after 7 iterations,
    every decision at least 4e-3 from the threshold (GPU and restatement NLLs
    agree to ~1e-5)."""
    X, y = _hello()
    _log("early stopping: n=400, patience 2, tol 0.02")
    got = _engine_train(X, y, [0.5, 1.0], 0.1, 40, 0.05, 0, es=True, patience=2, es_tol=0.02)
    ref = oe.train(ok.RBF, False, X, y, [0.5, 1.0], 0.1, max_iterations=40, learning_rate=0.05,
                   num_probes=10, max_cg=100, cg_tol=1e-2, precond_rank=0, max_tridiag=30,
                   enable_early_stopping=True, early_stop_patience=2, early_stop_tol=0.02)
    assert ref["converged"] and ref["iterations"] == 7
    assert got["converged"] and got["iterations"] == ref["iterations"]
    _check_trajectory(got, ref, "early stop", 0.05)


# ------------------------------------------------------------------ cache
def _cache_case(kernel, X, y, Xs, iters):
    gp = SingleOutputGP(kernel)
    gp.fit(X, y, max_iterations=iters, method="matrix_free", learning_rate=0.05)
    mean0, var0 = gp.predict(Xs, return_var=True)           # alpha + LOVE root, no cache
    cinfo = gp.prepare_prediction_cache(variance_method="love")
    assert cinfo["prediction_cache_has_love_root"] and cinfo["prediction_cache_rank"] > 0
    handle = cinfo["prediction_cache_handle"]
    mean1, var1 = gp.predict(Xs, return_var=True)           # through predict_with_cache
    assert gp.backend_predict_info["alpha_cache_used"]
    assert gp.backend_predict_info["love_root_cache_used"]
    return gp, handle, (mean0, var0), (mean1, var1)


@pytest.mark.parametrize("case", ["rbf_ard", "tree"])
def test_prediction_cache_matches_predict(case):
    rng = np.random.default_rng(4)
    n, d, m = 900, 2, 70
    X = rng.uniform(-2, 2, size=(n, d)).astype(np.float32)
    y = (np.sin(2 * X[:, 0]) * np.cos(X[:, 1]) + 0.05 * rng.normal(size=n)).astype(np.float32)
    Xs = rng.uniform(-2.2, 2.2, size=(m, d)).astype(np.float32)
    if case == "rbf_ard":
        kernel, kind = RBF(ard=True), ok.RBF
    else:
        kernel, kind = RBF(active_dims=[0]) * Matern52(active_dims=[1]) + RQ(), None
    _log(f"prediction cache: {case}")
    gp, handle, (mean0, var0), (mean1, var1) = _cache_case(kernel, X, y, Xs, 6)
    # the cache holds the same alpha and a deterministic Lanczos root: the
    # cached prediction is the uncached one, bit for bit
    np.testing.assert_array_equal(mean1, mean0)
    np.testing.assert_array_equal(var1, var0)
    tr = gp.training_result
    if kind is not None:
        params = np.asarray(tr.params, np.float64)
        mu, var, _ = oe.predict(kind, True, X, y, Xs, params, tr.noise, gp._engine_predict_mean,
                                max_cg=300, tol=1e-3, lanczos_rank=200)
        _log(f"  vs oracle: mean {_rel(mean1, mu):.2e}, std {_rel(np.sqrt(var1), np.sqrt(var)):.2e}")
        assert _rel(np.sqrt(var1), np.sqrt(var)) <= 1e-4
        assert _rel(mean1, mu) <= 5e-3
    # a cached mean-only prediction equals the mean of the LOVE one
    res = gp._engine.predict_with_cache(gp._provider_info, handle, Xs, None, tr.noise,
                                        gp._engine_predict_mean, 0)
    np.testing.assert_array_equal(res["mean"], mean0)
    # destroy: the handle is then rejected cleanly, and predict recomputes
    gp._destroy_prediction_cache()
    with pytest.raises(NativeCallError, match="unknown or destroyed"):
        gp._engine.predict_with_cache(gp._provider_info, handle, Xs, None, tr.noise,
                                      gp._engine_predict_mean, 1)
    with pytest.raises(NativeCallError, match="unknown or destroyed"):
        _lib_destroy(handle)
    mean2, var2 = gp.predict(Xs, return_var=True)
    np.testing.assert_allclose(mean2, mean0, rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(var2, var0, rtol=1e-6, atol=1e-7)


def _lib_destroy(handle):
    from mojogp_amd import _lib
    import ctypes as C
    _lib.call("mgp_destroy_prediction_cache", C.c_void_p(int(handle)))
