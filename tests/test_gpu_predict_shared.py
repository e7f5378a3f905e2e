"""Alpha CG and Lanczos root side by side (one two-column product per
iteration while both run) on the symmetric product route.

The route gives every column the same bits alone or beside another, so the
side-by-side solves must reproduce the sequential ones exactly: alpha from a
mean-only prediction, and the Lanczos root from a LOVE prediction handed that
alpha (which then runs the Lanczos alone).  MGP_SYM_MATVEC=1 puts small n on
the symmetric route; the larger case takes it by default."""

import numpy as np
import pytest

from mojogp_amd._engine import KernelModule, load_engine
from oracle import engine as oe
from oracle import kernels as ok

pytestmark = pytest.mark.gpu


def _rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def _predicts(kind, ard, X, y, Xs, params, noise, mean, tol, rank):
    km = KernelModule(kind, ard, X.shape[1])
    info = km.init_provider(X, params, noise)
    eng = load_engine()
    try:
        both = eng.predict(info, y, Xs, params, noise, mean, 1, 300, tol, 0, rank, False, 0)
        mean_only = eng.predict(info, y, Xs, params, noise, mean, 0, 300, tol, 0, rank, False, 0)
        root_alone = eng.predict(info, y, Xs, params, noise, mean, 1, 300, tol, 0, rank, False,
                                 0, mean_only["cached_alpha"])
    finally:
        km.destroy_provider(info)
    return both, mean_only, root_alone


@pytest.mark.parametrize("n,rank,force", [(800, 100, True), (26_000, 60, False)])
def test_side_by_side_equals_sequential(monkeypatch, n, rank, force):
    rng = np.random.default_rng(n)
    d, m = 3, 200
    X = rng.uniform(-2, 2, size=(n, d)).astype(np.float32)
    Xs = rng.uniform(-2.5, 2.5, size=(m, d)).astype(np.float32)
    y = (np.cos(X).prod(1) + 0.05 * rng.normal(size=n)).astype(np.float32)
    params = np.array([0.7, 0.9, 1.2, 1.1], np.float32)
    if force:
        monkeypatch.setenv("MGP_SYM_MATVEC", "1")
    else:
        monkeypatch.delenv("MGP_SYM_MATVEC", raising=False)
    print(f"side-by-side case n={n} rank={rank} force={force}", flush=True)
    both, mean_only, root_alone = _predicts(ok.MATERN52, True, X, y, Xs, params, 0.05, 0.1,
                                            1e-3, rank)
    print(f"  alpha iterations {both['alpha_cg_iterations']} / {mean_only['alpha_cg_iterations']}",
          flush=True)
    assert both["alpha_cg_iterations"] == mean_only["alpha_cg_iterations"]
    assert np.array_equal(both["cached_alpha"], mean_only["cached_alpha"])
    assert np.array_equal(both["mean"], mean_only["mean"])
    assert root_alone["alpha_cache_used"]
    assert np.array_equal(both["cached_lanczos_root"], root_alone["cached_lanczos_root"])
    assert np.array_equal(both["variance"], root_alone["variance"])


def test_side_by_side_matches_oracle(monkeypatch):
    """The side-by-side path against the CPU restatement (LOVE std 1e-4)."""
    rng = np.random.default_rng(21)
    n, d, m = 800, 2, 64
    X = rng.uniform(-2, 2, size=(n, d)).astype(np.float32)
    Xs = rng.uniform(-2.5, 2.5, size=(m, d)).astype(np.float32)
    y = (np.cos(X).prod(1) + 0.05 * rng.normal(size=n)).astype(np.float32)
    params = np.array([0.8, 1.3], np.float32)
    noise, mean = 0.02, 0.1
    monkeypatch.setenv("MGP_SYM_MATVEC", "1")
    both, _, _ = _predicts(ok.RBF, False, X, y, Xs, params, noise, mean, 1e-6, 100)
    mu, var, _ = oe.predict(ok.RBF, False, X, y, Xs, params.astype(np.float64), noise, mean,
                            max_cg=300, tol=1e-6, lanczos_rank=100)
    e_m, e_s = _rel(both["mean"], mu), _rel(both["std"], np.sqrt(var))
    print(f"  mean relerr {e_m:.2e}, std relerr {e_s:.2e}", flush=True)
    assert e_m <= 1e-4
    assert e_s <= 1e-4
