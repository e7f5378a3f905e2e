"""GPU parity of learned per-sample noise (the reference's noise modes 2-4:
one variance per point, one per group, softplus of a linear function of the
inputs) against the float64 restatement: the fit's kernel parameters and
learned variances on the restatement's trajectory, prediction with the
learned training vector, observed prediction with learned test noise, and
persistence."""

import numpy as np
import pytest

from mojogp_amd import RBF, SingleOutputGP
from oracle import engine as oe
from oracle import kernels as ok

pytestmark = pytest.mark.gpu


def _rel(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def _data(n=300, seed=7):
    rng = np.random.default_rng(seed)
    X = np.stack([np.linspace(-3, 3, n), rng.uniform(-1, 1, n)], 1).astype(np.float32)
    sd = 0.05 + 0.25 * (X[:, 0] > 0)
    y = (np.sin(2 * X[:, 0]) + sd * rng.normal(size=n)).astype(np.float32)
    groups = (X[:, 0] > 0).astype(np.int32) + 2 * (X[:, 1] > 0.5).astype(np.int32)
    return X, y, groups


@pytest.mark.parametrize("mode,name", [(2, "learned_vector"), (3, "learned_grouped"),
                                       (4, "learned_input_dependent")])
def test_learned_noise_fit_matches_oracle(mode, name, tmp_path):
    X, y, groups = _data()
    gp = SingleOutputGP(RBF())
    # The learned variances fall to ~0.003; without a preconditioner fp32 and
    # fp64 SLQ then part by ~1e-3 in the per-sample NLL, so the fit runs with
    # the rank-15 diagonal-noise Woodbury preconditioner, rebuilt every step.
    kw = dict(max_iterations=10, method="matrix_free", initial_params=[0.6, 1.0],
              initial_noise=0.1, learning_rate=0.05, preconditioner_rank=15)
    if mode == 2:
        tr = gp.fit(X, y, noise_model="learned_vector", **kw)
    elif mode == 3:
        tr = gp.fit(X, y, noise_model="grouped", noise_group_train=groups, learn_noise=True, **kw)
    else:
        tr = gp.fit(X, y, noise_model="learned_input_dependent", noise_function="linear", **kw)
    info = gp.backend_train_info
    print(f"{name}: noise_mode {info['noise_mode']}, params {tr.params}", flush=True)
    assert info["noise_mode"] == name
    ref = oe.train(ok.RBF, False, X, y, [0.6, 1.0], 0.1, max_iterations=10, learning_rate=0.05,
                   num_probes=10, max_cg=100, cg_tol=1e-2, precond_rank=15, max_tridiag=30,
                   learned=dict(mode=mode, floor=1e-6, reg=0.01, groups=groups, X=X))
    learned = gp._observation_noise_train
    print(f"  params {tr.params} vs {ref['params']}; noise vector relerr "
          f"{_rel(learned, ref['learned_noise']):.2e}; nll {tr.nll} vs {ref['final_nll']}",
          flush=True)
    assert _rel(tr.params, ref["params"]) <= 1e-3
    assert _rel(learned, ref["learned_noise"]) <= 2e-3
    assert tr.nll == pytest.approx(ref["final_nll"], rel=1e-3, abs=1e-4)
    if mode == 3:
        gv = gp._noise_group_values
        for g in range(4):
            assert gv[g] == pytest.approx(float(np.mean(learned[groups == g])), rel=1e-6)
    if mode == 4:
        print(f"  noise fn {gp._noise_function_params} vs {ref['noise_raw']}", flush=True)
        assert _rel(gp._noise_function_params, ref["noise_raw"]) <= 1e-3
    # prediction treats the learned training variances as a fixed vector
    Xs = np.stack([np.linspace(-3.5, 3.5, 40), np.linspace(-1, 1, 40)], 1).astype(np.float32)
    mean_t, std_t = gp.predict(Xs, return_std=True, cg_tolerance=1e-6)
    pr = tr.params.astype(np.float64)
    mu, var, _ = oe.predict(ok.RBF, False, X, y, Xs, pr, 0.0, tr.mean, max_cg=300, tol=1e-6,
                            lanczos_rank=100, noise_vec=learned.astype(np.float64))
    print(f"  predict mean {_rel(mean_t, mu):.2e} std {_rel(std_t, np.sqrt(var)):.2e}",
          flush=True)
    assert _rel(mean_t, mu) <= 1e-4
    assert _rel(std_t, np.sqrt(var)) <= 1e-4
    _, v_l = gp.predict(Xs, return_var=True, cg_tolerance=1e-6)
    if mode == 4:
        _, v_o = gp.predict_observed(Xs, return_var=True, cg_tolerance=1e-6)
        w = gp._noise_function_params
        ref_noise = np.logaddexp(0.0, w[0] + Xs @ w[1:]) + 1e-6
        np.testing.assert_allclose(v_o, v_l + ref_noise, rtol=1e-5)
    if mode == 3:
        gt = (Xs[:, 0] > 0).astype(np.int32)
        _, v_o = gp.predict_observed(Xs, noise_group_test=gt, return_var=True, cg_tolerance=1e-6)
        np.testing.assert_allclose(v_o, v_l + gp._noise_group_values[gt], rtol=1e-5)
    gp.save(tmp_path / "ln")
    gp2 = SingleOutputGP.load(str(tmp_path / "ln"))
    np.testing.assert_array_equal(gp2._observation_noise_train, learned)
    m2, s2 = gp2.predict(Xs, return_std=True, cg_tolerance=1e-6)
    np.testing.assert_allclose(m2, mean_t, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(s2, std_t, rtol=1e-5, atol=1e-6)
