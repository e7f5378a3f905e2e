"""Pins of the mixed continuous x categorical LMC restatement
(oracle.lmc.cat_gradients, oracle.lmc.train_mixed; jit_lmc_mixed.mojo:684-1557).

* cat_gradients: with probes chosen as N times the unit basis (P = N), the
  reference's estimator (-0.5 alpha^T dK alpha + (0.5/P) sum_j u_j^T dK zn_j) / N
  with u_j = K^-1 z_j and unit zn_j equals the exact gradient of the NLL
  (0.5 y^T K^-1 y + 0.5 log|K|) / N in the raw categorical parameters; it is
  compared with central differences of the exact NLL for GD, CR and EHH
  leaves, which pins the leaf derivative, dR/dtheta, the Kronecker mixing
  with A_s and the transform chain.
* train_mixed through its evaluate hook: the categorical raw parameters
  follow torch.optim.Adam on the scripted gradients (their own moments, the
  shared step count); NaN ends the run; after iteration 20 the patience
  counts every evaluation not below the best NLL, the improving one included
  (the counter is reset and then incremented in the same iteration, so a
  stall right after an improvement stops one evaluation early), as the
  reference's loop does.
"""

import numpy as np
import pytest
import torch

from mojogp_amd import CR, EHH, GD, RBF
from oracle import categorical as oc
from oracle import kernels as ok
from oracle import lmc as ol

F32 = np.float32


def _data(n=40, T=2, seed=0, L=3):
    rng = np.random.default_rng(seed)
    X = np.c_[rng.uniform(0, 1, n), rng.integers(0, L, n)].astype(np.float32)
    Y = np.stack([np.sin(4 * X[:, 0]) + 0.3 * X[:, 1], np.cos(3 * X[:, 0]) - 0.2 * X[:, 1]])
    Y = (Y[:T] + 0.05 * rng.normal(size=(T, n))).astype(np.float32)
    return X, Y


@pytest.mark.parametrize("leaf,kind", [(GD, oc.GD), (CR, oc.CR), (EHH, oc.EHH)])
def test_cat_gradient_is_the_exact_nll_gradient_with_basis_probes(leaf, kind):
    X, Y = _data()
    n, T, L = X.shape[0], Y.shape[0], 3
    node = (RBF(active_dims=[0]) * leaf(L, active_dims=[1])).to_dict()
    params = np.array([0.4, 1.3], np.float64)
    A = np.array([[1.0, 0.3], [0.3, 0.7]])
    noise = np.array([0.05, 0.08])
    rng = np.random.default_rng(3)
    raw = (oc.default_raw(kind, L) + 0.3 * rng.normal(size=oc.num_params(kind, L))).astype(F32)
    y = Y.reshape(-1).astype(np.float64)
    N = n * T

    def full(rc):
        tab = oc.correlation(kind, L, oc.constrain(kind, L, rc))
        tr = ok.TreeKernel(node, 2, [tab])
        return tr, ol.dense_operator([tr.matrix(X, X, params)], A[None], noise)

    def nll(rc):
        _, Kf = full(np.asarray(rc, np.float64))
        s, ld = np.linalg.slogdet(Kf)
        return (0.5 * y @ np.linalg.solve(Kf, y) + 0.5 * ld) / N

    tr, Kf = full(raw)
    Kinv = np.linalg.inv(Kf)
    ev = {"alpha": Kinv @ y, "U": N * Kinv, "Zn": np.eye(N)}
    got = ol.cat_gradients(tr, X, params, A, [(kind, L)], raw, ev)
    h = 1e-3
    want = []
    for k in range(raw.size):
        e = np.zeros(raw.size)
        e[k] = h
        want.append((nll(raw + e) - nll(raw - e)) / (2 * h))
    np.testing.assert_allclose(got, np.array(want), rtol=2e-4, atol=1e-8)


class _Scripted:
    """Scripted evaluation: continuous gradients zero, categorical raw
    gradients w (raw - c) of latent 1, the NLL from a sequence (or NaN)."""

    def __init__(self, n, T, nll_seq, nan_at=()):
        self.n, self.T = n, T
        self.c = np.array([0.2, -0.4, 0.6])
        self.w = np.array([1.0, 0.5, 2.0])
        self.nll_seq = nll_seq
        self.nan_at = set(nan_at)
        self.raw_seen = []

    def __call__(self, it, trees, params, A, noise, yc, cat_raw):
        raw = np.asarray(cat_raw[1], np.float64)
        self.raw_seen.append(raw.copy())
        nll = float("nan") if it in self.nan_at else float(self.nll_seq[it])
        R = len(params)
        return {"nll": F32(nll), "kernel_grads": np.zeros(sum(len(p) for p in params), F32),
                "noise_grads": np.zeros(self.T, F32), "G_A": np.zeros((R, self.T, self.T), F32),
                "alpha": np.zeros(self.n * self.T),
                "cat_grads": [np.zeros(0, F32), (self.w * (raw - self.c)).astype(F32)]}


def _train(obj, X, Y, iters, **kw):
    init = oc.default_raw(oc.EHH, 3).astype(F32)
    node = (RBF(active_dims=[0]) * EHH(3, active_dims=[1])).to_dict()
    return ol.train_mixed([ok.RBF, node], X, Y.reshape(-1), [[0.5, 1.0], [0.5, 1.0]],
                          [0.1, 0.1], [0.0, 0.0], [[], [(oc.EHH, 3)]],
                          [np.zeros(0, F32), init], max_iterations=iters, precond_rank=0,
                          evaluate=obj, **kw), init


def test_train_mixed_categorical_adam_matches_torch():
    X, Y = _data()
    iters = 30
    obj = _Scripted(X.shape[0], Y.shape[0], nll_seq=np.linspace(2.0, 1.0, iters))
    res, init = _train(obj, X, Y, iters, learning_rate=0.05, early_stop_tol=0.0)
    raw = torch.tensor(init, dtype=torch.float32, requires_grad=True)
    opt = torch.optim.Adam([raw], lr=0.05, betas=(0.9, 0.999), eps=1e-8)
    c, w = torch.tensor(obj.c, dtype=torch.float32), torch.tensor(obj.w, dtype=torch.float32)
    for it in range(iters):
        np.testing.assert_allclose(obj.raw_seen[it], raw.detach().numpy(), rtol=2e-5, atol=1e-6,
                                   err_msg=f"it {it}")
        opt.zero_grad()
        raw.grad = (w * (raw.detach() - c)).clamp(-1e30, 1e30)
        opt.step()
    # best snapshot = the last (strictly decreasing NLL): the raw values it saw
    np.testing.assert_allclose(res["cat_raw"][1], obj.raw_seen[-1], rtol=0, atol=0)
    assert res["iterations"] == iters and not res["converged"]


def test_train_mixed_nan_ends_the_run():
    X, Y = _data()
    obj = _Scripted(X.shape[0], Y.shape[0], nll_seq=np.linspace(2.0, 1.0, 10), nan_at={4})
    res, _ = _train(obj, X, Y, 10)
    assert res["iterations"] == 5 and len(res["nll_history"]) == 5
    assert np.isnan(res["nll_history"][-1])
    assert res["final_nll"] == pytest.approx(float(np.linspace(2.0, 1.0, 10)[3]), rel=1e-6)


def test_train_mixed_patience_counts_improving_steps_after_20():
    """After iteration 20 an improving evaluation resets the counter and then
    counts itself (it is not above the new best): a stall right after an
    improvement stops one evaluation early (patience 3: the improvement at
    25 and the stalls at 26, 27), and steady improvement never stops."""
    X, Y = _data()
    seq = np.r_[np.linspace(5.0, 1.0, 26), np.full(34, 1.0)]
    obj = _Scripted(X.shape[0], Y.shape[0], nll_seq=seq)
    res, _ = _train(obj, X, Y, 60, early_stop_tol=1e-4, early_stop_patience=3)
    assert res["converged"] and res["iterations"] == 28
    obj = _Scripted(X.shape[0], Y.shape[0], nll_seq=np.linspace(5.0, 1.0, 60))
    res, _ = _train(obj, X, Y, 60, early_stop_tol=1e-4, early_stop_patience=3)
    assert not res["converged"] and res["iterations"] == 60
    # a flat NLL after 20: the counter is never reset
    seq = np.r_[np.linspace(5.0, 1.0, 21), np.full(39, 1.0)]
    obj = _Scripted(X.shape[0], Y.shape[0], nll_seq=seq)
    res, _ = _train(obj, X, Y, 60, early_stop_tol=1e-4, early_stop_patience=5)
    assert res["converged"] and res["iterations"] == 26
    # early_stop_tol 0 disables the stop
    obj = _Scripted(X.shape[0], Y.shape[0], nll_seq=np.linspace(5.0, 1.0, 30))
    res, _ = _train(obj, X, Y, 30, early_stop_tol=0.0, early_stop_patience=3)
    assert not res["converged"] and res["iterations"] == 30


@pytest.mark.parametrize("kind", [oc.GD, oc.CR, oc.EHH, oc.HH, oc.FE])
def test_cat_raw_from_constrained_inverts_the_transform(kind):
    """Models store constrained categorical parameters (the reference's
    cat_params_latent_s); loading recovers the raw values through
    kernel.cat_raw_from_constrained, the inverse of the oracle's constrain."""
    from mojogp_amd.kernel import KernelType, cat_raw_from_constrained
    kt = {oc.GD: KernelType.GD, oc.CR: KernelType.CR, oc.EHH: KernelType.EHH,
          oc.HH: KernelType.HH, oc.FE: KernelType.FE}[kind]
    L = 4
    rng = np.random.default_rng(kind)
    raw = (oc.default_raw(kind, L) + rng.uniform(-1.5, 1.5, oc.num_params(kind, L))).astype(F32)
    theta = oc.constrain(kind, L, raw)
    back = cat_raw_from_constrained(kt, L, theta.astype(F32))
    np.testing.assert_allclose(back, raw, rtol=1e-5, atol=2e-6)
    # the tables from the recovered values match the stored state
    np.testing.assert_allclose(oc.correlation(kind, L, oc.constrain(kind, L, back)),
                               oc.correlation(kind, L, theta), rtol=0, atol=2e-6)
