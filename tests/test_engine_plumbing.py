"""Default-resolution contract of SingleOutputGP.fit against a fake engine (CPU).

Restates the expectations of the reference's
``tests/unit/test_exactgp_engine_plumbing.py:66-189``: the positional engine
arguments ``fit`` resolves (preconditioner rank / method / use flag, tridiagonal
length, rebuild threshold) and the exact ``backend_train_info`` dict, plus the
other defaults of ``gp.py:1306-1480`` (auto route, initial-lengthscale caps,
periodic noise floor, init mean).  No native library is loaded: the fakes
stand in for the kernel module and the engine, as in the reference's test.
"""

import numpy as np
import pytest

from mojogp_amd import RBF, Matern32, Matern52, Periodic, SingleOutputGP


class _FakeKernelModule:
    def __init__(self):
        self.materialize_calls = 0
        self.init_calls = []

    def init_provider(self, X, params, noise):
        self.init_calls.append((X, np.array(params), float(noise)))
        return {"provider_ptr": 1, "n": int(X.shape[0]),
                "num_gradient_params": int(len(params)), "materialization_mode": 0,
                "is_ard": False}

    def materialize(self, provider_info):
        self.materialize_calls += 1
        provider_info["materialization_mode"] = 1


class _FakeEngine:
    def __init__(self):
        self.train_calls = []

    def train(self, *args):
        self.train_calls.append(args)
        info = args[0]
        return {"params": np.array(args[2], dtype=np.float32), "noise": float(args[3]),
                "mean": 0.0, "final_nll": 1.23, "iterations": 1, "converged": False,
                "nll_history": [1.23],
                "materialization_mode": int(info.get("materialization_mode", 0)),
                "precond_method": int(args[15]), "precond_rank": int(args[9])}


def _make_data(n=2000, d=5):
    rng = np.random.RandomState(0)
    X = rng.randn(n, d).astype(np.float32)
    y = (np.sin(X[:, 0]) + 0.1 * rng.randn(n)).astype(np.float32)
    return X, y


def _fake_gp(kernel):
    gp = SingleOutputGP(kernel)
    gp._kernel_module = _FakeKernelModule()
    gp._engine = _FakeEngine()
    gp._ensure_compiled = lambda: None
    return gp


def test_fit_passes_resolved_preconditioner_controls_to_engine():
    gp = _fake_gp(RBF())
    X, y = _make_data()
    result = gp.fit(X, y, max_iterations=1, method="materialized", max_tridiag_iterations=17,
                    precond_rebuild_threshold=0.125, preconditioner="greedy", verbose=False)
    args = gp._engine.train_calls[-1]
    assert gp._kernel_module.materialize_calls == 1
    assert len(args) == 23
    assert args[13] == 17
    assert np.isclose(float(args[14]), 0.125)
    assert args[15] == 0
    assert result.lanczos_rank == 17
    assert gp.backend_train_info == {
        "training_route": "materialized", "materialization_mode": 1, "is_ard": False,
        "precond_method": 0, "precond_rank": 100, "max_cg_iter": 100,
        "max_cg_iterations": 100, "cg_tol": 0.01, "cg_tolerance": 0.01,
        "max_tridiag_iter": 17, "precond_rebuild_threshold": 0.125,
        "enable_early_stopping": False, "early_stop_patience": 10, "early_stop_tol": 1e-4,
        "use_preconditioner": True, "noise_mode": "scalar", "learn_noise": True,
        "has_observation_noise_vector": False, "noise_regularization": 0.01,
    }


def test_matrix_free_default_preconditioner_policy_enables_low_dim_rbf():
    gp = _fake_gp(RBF())
    X, y = _make_data(n=5000, d=5)
    gp.fit(X, y, max_iterations=1, method="matrix_free", verbose=False)
    args = gp._engine.train_calls[-1]
    assert args[9] == 256
    assert args[12] is True
    assert args[15] == 0
    assert gp.backend_train_info["precond_rank"] == 256
    assert gp.backend_train_info["use_preconditioner"] is True


def test_fit_method_aliases_resolve_to_canonical_routes():
    X, y = _make_data(n=5000, d=5)
    gp_mat = _fake_gp(RBF())
    gp_mat.fit(X, y, max_iterations=1, method="mat", verbose=False)
    assert gp_mat._training_method == "materialized"
    assert gp_mat._kernel_module.materialize_calls == 1
    gp_mf = _fake_gp(RBF())
    gp_mf.fit(X, y, max_iterations=1, method="mf", verbose=False)
    assert gp_mf._training_method == "matrix_free"
    assert gp_mf._kernel_module.materialize_calls == 0


def test_matrix_free_default_preconditioner_policy_disables_unsupported_route():
    gp = _fake_gp(RBF())
    X, y = _make_data(n=5000, d=17)
    gp.fit(X, y, max_iterations=1, method="matrix_free", verbose=False)
    args = gp._engine.train_calls[-1]
    assert args[9] == 0
    assert args[12] is False
    assert gp.backend_train_info["precond_rank"] == 0
    assert gp.backend_train_info["use_preconditioner"] is False


def test_matrix_free_explicit_preconditioner_overrides_route_policy():
    gp = _fake_gp(RBF())
    X, y = _make_data(n=5000, d=17)
    gp.fit(X, y, max_iterations=1, method="matrix_free", preconditioner="nystrom",
           preconditioner_rank=128, verbose=False)
    args = gp._engine.train_calls[-1]
    assert args[9] == 128
    assert args[12] is True
    assert args[15] == 2
    assert gp.backend_train_info["precond_rank"] == 128
    assert gp.backend_train_info["use_preconditioner"] is True


# ---- further defaults of gp.py:1306-1480 -----------------------------------

def test_positional_engine_arguments_balanced_preset():
    """Order and values of the 23 positional train() arguments (gp.py:1665-1691)
    under the balanced preset (gp.py:800-808) for the config-3 kernel."""
    gp = _fake_gp(Matern52(ard=True))
    X, y = _make_data(n=3000, d=4)
    gp.fit(X, y, max_iterations=7, learning_rate=0.02, method="matrix_free", verbose=False,
           num_probes=15, preconditioner_rank=200)
    a = gp._engine.train_calls[-1]
    assert len(a) == 23
    np.testing.assert_array_equal(a[1], y)
    np.testing.assert_array_equal(a[2], np.ones(5, np.float32))  # 4 lengthscales + os
    assert a[3] == pytest.approx(0.1)          # initial noise
    assert a[4] == 7 and a[5] == pytest.approx(0.02)
    assert a[6] == 15                          # probes
    assert a[7] == 100                         # max_cg
    assert a[8] == pytest.approx(0.01)         # cg tolerance
    assert a[9] == 200 and a[12] is True       # explicit rank enables the preconditioner
    assert a[10] is False and a[11] is False   # verbose, cosine LR
    assert a[13] == 30                         # max tridiagonal iterations
    assert a[14] == pytest.approx(0.5)         # rebuild threshold
    assert a[15] == 0                          # balanced preset: greedy pivots
    assert a[16] == pytest.approx(float(np.mean(y)))  # init mean
    assert a[17] is False and a[18] == 10 and a[19] == pytest.approx(1e-4)
    assert a[20] is True                       # learn noise
    assert a[21] == pytest.approx(1e-6) and a[22] == pytest.approx(0.01)


def test_matrix_free_ard_matern_defaults_to_no_preconditioner():
    gp = _fake_gp(Matern52(ard=True))
    X, y = _make_data(n=6000, d=6)
    gp.fit(X, y, max_iterations=1, method="matrix_free", verbose=False)
    a = gp._engine.train_calls[-1]
    assert a[9] == 0 and a[12] is False


def test_auto_route_threshold():
    X, y = _make_data(n=2000, d=2)
    gp = _fake_gp(RBF())
    gp.fit(X, y, max_iterations=1, verbose=False)
    assert gp._training_method == "materialized"
    X2, y2 = _make_data(n=2001, d=2)
    gp2 = _fake_gp(RBF())
    gp2.fit(X2, y2, max_iterations=1, verbose=False)
    assert gp2._training_method == "matrix_free"


def test_initial_lengthscale_caps():
    # materialized, 1-D RBF, lr <= 0.05: lengthscale capped at 0.5
    X, y = _make_data(n=500, d=1)
    gp = _fake_gp(RBF())
    gp.fit(X, y, max_iterations=1, method="materialized", verbose=False)
    assert gp._engine.train_calls[-1][2][0] == pytest.approx(0.5)
    # not capped with a larger learning rate
    gp = _fake_gp(RBF())
    gp.fit(X, y, max_iterations=1, method="materialized", learning_rate=0.1, verbose=False)
    assert gp._engine.train_calls[-1][2][0] == pytest.approx(1.0)
    # matrix-free isotropic RBF, 1 < d <= 8, n >= 10000: capped at 0.6
    X, y = _make_data(n=10000, d=3)
    gp = _fake_gp(RBF())
    gp.fit(X, y, max_iterations=1, method="matrix_free", verbose=False)
    assert gp._engine.train_calls[-1][2][0] == pytest.approx(0.6)
    X, y = _make_data(n=9999, d=3)
    gp = _fake_gp(RBF())
    gp.fit(X, y, max_iterations=1, method="matrix_free", verbose=False)
    assert gp._engine.train_calls[-1][2][0] == pytest.approx(1.0)
    # explicit initial parameters are never capped
    X, y = _make_data(n=500, d=1)
    gp = _fake_gp(RBF())
    gp.fit(X, y, max_iterations=1, method="materialized", initial_params=[2.0, 1.0],
           verbose=False)
    assert gp._engine.train_calls[-1][2][0] == pytest.approx(2.0)


def test_materialized_matern32_defaults_to_greedy_and_ard_threshold():
    X, y = _make_data(n=800, d=3)
    gp = _fake_gp(Matern32())
    gp.fit(X, y, max_iterations=1, method="materialized", verbose=False)
    a = gp._engine.train_calls[-1]
    assert a[15] == 0 and a[14] == pytest.approx(0.5)
    gp = _fake_gp(RBF(ard=True))
    gp.fit(X, y, max_iterations=1, method="materialized", verbose=False)
    a = gp._engine.train_calls[-1]
    assert a[14] == pytest.approx(0.1) and a[15] == 0


def test_periodic_noise_floor():
    X, y = _make_data(n=300, d=1)
    gp = _fake_gp(Periodic())
    gp.fit(X, y, max_iterations=1, method="materialized", initial_noise=0.01, verbose=False)
    assert gp._engine.train_calls[-1][3] == pytest.approx(0.05)
    gp = _fake_gp(RBF())
    gp.fit(X, y, max_iterations=1, method="materialized", initial_noise=0.01, verbose=False)
    assert gp._engine.train_calls[-1][3] == pytest.approx(0.01)


def test_fixed_init_mean_and_result_packaging():
    X, y = _make_data(n=300, d=2)
    gp = SingleOutputGP(RBF(), init_mean=0.25)
    gp._kernel_module = _FakeKernelModule()
    gp._engine = _FakeEngine()
    gp._ensure_compiled = lambda: None
    res = gp.fit(X, y, max_iterations=1, method="materialized", verbose=False)
    assert gp._engine.train_calls[-1][16] == pytest.approx(0.25)
    assert res.nll == pytest.approx(1.23) and res.iterations == 1
    assert gp.is_trained
    # the provider was created from (X, engine params, noise) positionally
    Xp, pp, nz = gp._kernel_module.init_calls[-1]
    np.testing.assert_array_equal(Xp, X)
    np.testing.assert_array_equal(pp, np.array([1.0, 1.0], np.float32))
    assert nz == pytest.approx(0.1)
