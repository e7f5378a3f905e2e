"""SingleOutputGP's scoring and sampling surface (gp.py:759-779, 3059-3196,
3266-3433, 3642): score, get_learned_params, log_marginal_likelihood,
nll_history, backend_sample_info, and sample_posterior (diagonal and pathwise).

Pathwise samples are checked three ways: a seeded call repeats bit for bit;
the samples' mean and variance match the exact posterior (z-test over 256
draws); and each sample equals a float64 restatement of Matheron's rule that
draws from the same Generator in the reference's order -- features W, phases,
then per sample the weights and the noise vector (pathwise_prior.py:37-97,
gp.py:3352-3364) -- with the exact solve in place of the engine's CG, to the
correction solve's tolerance: the engine stops the unpreconditioned alpha CG
at ||A alpha - r|| <= 1e-2 ||r|| (the tolerance the reference passes), so a
sample may differ from the exact one by at most ||K* A^-1||_2 1e-2 ||r||.
(That error is mostly common to all samples -- every residual shares its
y - mu part -- so the sample mean's z-test is loose by design.)"""

import numpy as np
import pytest

from mojogp_amd import RBF, Matern52, SingleOutputGP
from oracle import kernels as ok

pytestmark = pytest.mark.gpu


def _data(n=400, seed=0):
    rng = np.random.default_rng(seed)
    X = np.sort(rng.uniform(-3, 3, size=n)).astype(np.float32)[:, None]
    y = (np.sin(2 * X[:, 0]) + 0.1 * rng.normal(size=n)).astype(np.float32)
    Xs = np.linspace(-3.5, 3.5, 60, dtype=np.float32)[:, None]
    return X, y, Xs


def _exact_posterior(kind, ard, X, y, Xs, params, noise, mean):
    X64, Xs64 = X.astype(np.float64), Xs.astype(np.float64)
    A = ok.kernel_matrix(kind, X64, X64, params, ard) + noise * np.eye(X.shape[0])
    Ks = ok.kernel_matrix(kind, Xs64, X64, params, ard)
    mu = Ks @ np.linalg.solve(A, y.astype(np.float64) - mean) + mean
    var = params[-1] - np.sum(Ks * np.linalg.solve(A, Ks.T).T, axis=1)
    return mu, var, A, Ks


def test_score_params_lml_and_history():
    X, y, Xs = _data()
    gp = SingleOutputGP(RBF())
    tr = gp.fit(X, y, max_iterations=20, method="matrix_free")
    print(f"surface fit: params {tr.params} noise {tr.noise:.4g}", flush=True)
    np.testing.assert_array_equal(gp.nll_history, tr.nll_history)
    assert gp.log_marginal_likelihood() == -float(tr.nll)
    p = gp.get_learned_params()
    assert list(p) == gp.kernel.get_param_names() + ["noise", "mean"]
    assert p["noise"] == float(tr.noise) and p["mean"] == float(tr.mean)
    yt = np.sin(2 * Xs[:, 0]).astype(np.float32)
    mean, _ = gp.predict(Xs, return_std=True)
    r2 = 1.0 - np.sum((yt - mean) ** 2) / np.sum((yt - yt.mean()) ** 2)
    assert gp.score(Xs, yt) == pytest.approx(float(r2), rel=1e-6)
    assert gp.score(Xs, yt) > 0.9
    assert gp.backend_sample_info is None


def test_diagonal_samples_are_mean_plus_std_noise():
    X, y, Xs = _data()
    gp = SingleOutputGP(Matern52())
    gp.fit(X, y, max_iterations=10, method="matrix_free")
    s = gp.sample_posterior(Xs, n_samples=5, rng=np.random.default_rng(3))
    pred = gp.predict(Xs)
    z = np.random.default_rng(3).standard_normal((5, Xs.shape[0]))
    np.testing.assert_allclose(s, pred.mean + pred.std * z, rtol=1e-6, atol=1e-6)
    assert s.dtype == np.float32
    info = gp.backend_sample_info
    assert info["actual_sampling_method"] == "diagonal"
    assert info["actual_sampling_route"] == "diagonal_from_predictive_std"
    with pytest.raises(ValueError, match="method must be"):
        gp.sample_posterior(Xs, method="cholesky")


@pytest.mark.parametrize("kernel,kind,ard", [(lambda: RBF(), ok.RBF, False),
                                             (lambda: Matern52(ard=True), ok.MATERN52, True)])
def test_pathwise_samples(kernel, kind, ard):
    X, y, Xs = _data()
    gp = SingleOutputGP(kernel())
    tr = gp.fit(X, y, max_iterations=20, method="matrix_free")
    params = np.asarray(gp.kernel.to_engine_params(np.asarray(tr.params, np.float32)),
                        np.float64)
    noise, mean = float(tr.noise), float(tr.mean)
    F, S = 1024, 256
    print(f"pathwise kind={kind} ard={ard}: params {params} noise {noise:.4g}", flush=True)
    s1 = gp.sample_posterior(Xs, n_samples=S, method="pathwise", n_rff_features=F,
                             rng=np.random.default_rng(11))
    s2 = gp.sample_posterior(Xs, n_samples=S, method="pathwise", n_rff_features=F,
                             rng=np.random.default_rng(11))
    assert s1.shape == (S, Xs.shape[0]) and s1.dtype == np.float32
    np.testing.assert_array_equal(s1, s2)
    info = gp.backend_sample_info
    assert info["actual_sampling_method"] == "pathwise" and info["n_rff_features"] == F
    mu, var, A, Ks = _exact_posterior(kind, ard, X, y, Xs, params, noise, mean)
    # sample mean and variance against the exact posterior
    z = (s1.mean(axis=0) - mu) / np.sqrt(var / S)
    ratio = s1.var(axis=0, ddof=1) / var
    print(f"  mean z^2 {np.mean(z ** 2):.2f}, variance ratio median {np.median(ratio):.2f}",
          flush=True)
    assert np.mean(z ** 2) < 4.0
    assert 0.7 < np.median(ratio) < 1.4
    # float64 restatement with the same draws (RFF prior, exact solve)
    rng = np.random.default_rng(11)
    d = X.shape[1]
    W = rng.standard_normal((F, d)) if kind == ok.RBF else rng.standard_t(df=5, size=(F, d))
    phase = rng.uniform(0.0, 2.0 * np.pi, size=F)
    ls = params[:d] if ard else np.full(d, params[0])

    def phi(Z):
        return np.sqrt(params[-1]) * np.sqrt(2.0 / F) * np.cos((Z / ls) @ W.T + phase)

    PX, PXs = phi(X.astype(np.float64)), phi(Xs.astype(np.float64))
    gain = np.linalg.norm(Ks @ np.linalg.inv(A), 2)   # ||K* A^-1||_2
    errs, bounds = [], []
    for k in range(S):
        w = rng.standard_normal((1, F)).astype(np.float32).astype(np.float64)[0]
        eps = rng.standard_normal(X.shape[0]).astype(np.float32)
        obs = PX @ w + np.sqrt(noise) * eps
        r = (y.astype(np.float64) - mean) - obs
        ref = mean + PXs @ w + Ks @ np.linalg.solve(A, r)
        errs.append(np.linalg.norm(s1[k] - ref))
        bounds.append(1.1 * 1e-2 * gain * np.linalg.norm(r) + 1e-5 * np.linalg.norm(ref))
    errs, bounds = np.array(errs), np.array(bounds)
    print(f"  samples vs float64 restatement: error / solve-tolerance bound median "
          f"{np.median(errs / bounds):.2f}, max {np.max(errs / bounds):.2f}", flush=True)
    assert np.all(errs <= bounds)


def test_pathwise_rejects_trees():
    X, y, Xs = _data(200)
    gp = SingleOutputGP(RBF() + Matern52())
    gp.fit(X, y, max_iterations=3, method="matrix_free")
    with pytest.raises(NotImplementedError, match="single RBF / Matern"):
        gp.sample_posterior(Xs, method="pathwise")
