"""Pins of the mixed continuous x categorical ICM restatement
(oracle.icm.kron_pivot_precond, mixed_gradients, train_mixed;
jit_multi_output_mixed.mojo:477-1148).

* mixed_gradients and the categorical gradient: with probes chosen as N
  times the unit basis the estimators are exact, so G_B equals the
  derivative of the per-entry NLL in the entries of B (central differences),
  the noise gradients the derivative in the task noises, and the categorical
  gradient (neither divided by nT nor clipped in this loop) the derivative of
  N times the per-entry NLL in the raw categorical parameters.
* kron_pivot_precond: at full rank with a unit-diagonal base kernel and
  equal task noises the factor rebuilds the operator exactly
  (L L^T + noise I = os B (x) K + D); the Woodbury noise is the smallest task
  noise; the first pivot is the first entry of the task with the largest os B_ss and
  its column is scaled by 1 / sqrt(os B_ss) whatever the base diagonal (the
  provider reports a base diagonal of 1).
* train_mixed through its evaluate hook: categorical raw parameters and
  kernel parameters follow torch.optim.Adam on scripted gradients (their own
  moments, one step count, softplus chain on the kernel side); W and raw_v
  see G_B clipped at +-10; early stopping counts evaluations not below the
  best by early_stop_tol; the cosine rate applies to every group.
"""

import numpy as np
import pytest
import torch

from mojogp_amd import EHH, GD, RBF
from oracle import categorical as oc
from oracle import engine as oe
from oracle import icm as oi
from oracle import kernels as ok
from oracle import lmc as ol

F32 = np.float32


def _data(n=30, T=2, seed=0, L=3):
    rng = np.random.default_rng(seed)
    X = np.c_[rng.uniform(0, 1, n), rng.integers(0, L, n)].astype(np.float32)
    Y = np.stack([np.sin(4 * X[:, 0]) + 0.3 * X[:, 1], np.cos(3 * X[:, 0]) - 0.2 * X[:, 1]])
    return X, (Y[:T] + 0.05 * rng.normal(size=(T, n))).astype(np.float32)


def _exact_ev(A, y):
    """Basis probes z_j = sqrt(N) e_j: U = A^-1 Z, W = Z (no preconditioner)
    and the unit probes Zn = I, with which (1/P) sum_j u_j^T dA w_j and
    (1/P) sum_j (N A^-1 e_j)^T dA zn_j are both tr(A^-1 dA)."""
    N = A.shape[0]
    Ainv = np.linalg.inv(A)
    s = np.sqrt(N)
    return {"alpha": Ainv @ y, "U": s * Ainv, "W": s * np.eye(N), "Zn": np.eye(N)}


def _nll(A, y):
    N = A.shape[0]
    return (0.5 * y @ np.linalg.solve(A, y) + 0.5 * np.linalg.slogdet(A)[1]) / N


def test_task_and_noise_gradients_are_exact_with_basis_probes():
    X, Y = _data()
    n, T = X.shape[0], Y.shape[0]
    K = ok.kernel_matrix(ok.RBF, X, X, np.array([0.4, 1.2]), False)
    os_, B = 0.8, np.array([[1.0, 0.35], [0.35, 0.6]])
    noise = np.array([0.07, 0.11])
    y = Y.reshape(-1).astype(np.float64)

    def A_of(Bm, nz):
        return os_ * np.kron(Bm, K) + np.diag(np.repeat(nz, n))

    GB, gn = oi.mixed_gradients(K, os_, _exact_ev(A_of(B, noise), y), n, T)
    h = 1e-5
    for s in range(T):
        for t in range(T):
            E = np.zeros((T, T))
            E[s, t] = h
            fd = (_nll(A_of(B + E, noise), y) - _nll(A_of(B - E, noise), y)) / (2 * h)
            assert GB[s, t] == pytest.approx(fd, rel=1e-5, abs=1e-9)
    for t in range(T):
        e = np.zeros(T)
        e[t] = h
        fd = (_nll(A_of(B, noise + e), y) - _nll(A_of(B, noise - e), y)) / (2 * h)
        assert gn[t] == pytest.approx(fd, rel=1e-5, abs=1e-9)


def test_cat_gradient_unnormalised_and_unclipped():
    X, Y = _data()
    n, T, L = X.shape[0], Y.shape[0], 3
    node = (RBF(active_dims=[0]) * EHH(L, active_dims=[1])).to_dict()
    params = np.array([0.4, 1.3])
    os_, B = 0.9, np.array([[1.0, 0.3], [0.3, 0.7]])
    noise = np.array([0.05, 0.08])
    raw = (oc.default_raw(oc.EHH, L) + np.array([0.3, -0.2, 0.1])).astype(F32)
    y = Y.reshape(-1).astype(np.float64)
    N = n * T

    def full(rc):
        tab = oc.correlation(oc.EHH, L, oc.constrain(oc.EHH, L, rc))
        tr = ok.TreeKernel(node, 2, [tab])
        K = tr.matrix(X, X, params)
        return tr, os_ * np.kron(B, K) + np.diag(np.repeat(noise, n))

    tr, A = full(raw)
    ev = _exact_ev(A, y)
    ev["U"] = ev["U"] * np.sqrt(N)  # the categorical form pairs U with the unit probes
    got = ol.cat_gradients(tr, X, params, os_ * B, [(oc.EHH, L)], raw, ev,
                           clip=None, per_entry=False)
    h = 1e-3
    for k in range(raw.size):
        e = np.zeros(raw.size)
        e[k] = h
        fd = N * (_nll(full(raw + e)[1], y) - _nll(full(raw - e)[1], y)) / (2 * h)
        assert got[k] == pytest.approx(fd, rel=2e-4, abs=1e-7)


def test_kron_pivot_precond_full_rank_and_diagonal_quirk():
    X, _ = _data(n=12)
    n, T = X.shape[0], 2
    # unit diagonal, well conditioned, so that full rank is reached in fp32
    K = ok.kernel_matrix(ok.RBF, X, X, np.array([0.04, 1.0]), False)
    os_, B = 0.7, np.array([[0.5, 0.2], [0.2, 1.1]], np.float32)
    # equal task noises: the diagonal the provider reports is the residual's own
    eq = np.array([0.05, 0.05], np.float32)
    P = oi.kron_pivot_precond(K, os_, B, eq, n * T, method=0)
    A = float(F32(os_)) * np.kron(B.astype(np.float64), K) + np.diag(np.repeat(eq, n))
    np.testing.assert_allclose(P.L @ P.L.T + P.noise * np.eye(n * T), A, atol=2e-5)
    # unequal noises: the Woodbury noise is the smallest one
    noise = np.array([0.09, 0.05], np.float32)
    assert oi.kron_pivot_precond(K, os_, B, noise, 4).noise == pytest.approx(0.05)
    # base outputscale 2: the residual diagonal still starts at os B_ss
    K2 = 2.0 * K
    P2 = oi.kron_pivot_precond(K2, os_, B, noise, 3, method=0)
    p = n  # first entry of task 1 (os B_11 = 0.77 > os B_00 = 0.35)
    col = float(F32(os_)) * np.kron(B[:, 1].astype(np.float64), K2[:, 0])
    col[p] += float(noise[1] - noise.min())
    np.testing.assert_allclose(P2.L[:, 0], col / np.sqrt(float(F32(os_) * B[1, 1])),
                               rtol=2e-6, atol=1e-7)


class _Scripted:
    def __init__(self, n, T, nll_seq, GB):
        self.n, self.T, self.nll_seq, self.GB = n, T, nll_seq, np.asarray(GB, F32)
        self.c = np.array([0.2, -0.4, 0.6])
        self.w = np.array([1.0, 0.5, 2.0])
        self.raw_seen, self.params_seen, self.B_seen = [], [], []

    def __call__(self, it, tr, params, os_, B, noise, yc, cat_raw):
        self.raw_seen.append(np.asarray(cat_raw, np.float64).copy())
        self.params_seen.append(np.asarray(params, np.float64).copy())
        self.B_seen.append(np.asarray(B, np.float64).copy())
        raw = np.asarray(cat_raw, np.float64)
        return {"nll": F32(self.nll_seq[it]), "grads": np.array([0.3, -0.2, 0.1], F32),
                "alpha": np.zeros(self.n * self.T), "G_B": self.GB,
                "noise_grads": np.zeros(self.T, F32), "cg_iterations": 5,
                "cat_grads": (self.w * (raw - self.c)).astype(F32)}


def _train(obj, X, Y, iters, **kw):
    init = oc.default_raw(oc.EHH, 3).astype(F32)
    node = (RBF(active_dims=[0]) * EHH(3, active_dims=[1])).to_dict()
    return oi.train_mixed(node, X, Y.reshape(-1), [0.5, 1.0], [0.1, 0.1], 1.0, [0.0, 0.0],
                          [(oc.EHH, 3)], init, max_iterations=iters, precond_rank=0,
                          evaluate=obj, **kw), init


def test_train_mixed_adam_groups_match_torch():
    X, Y = _data()
    iters = 12
    GB = [[30.0, -0.5], [0.25, -40.0]]  # the diagonal entries clip at +-10
    obj = _Scripted(X.shape[0], Y.shape[0], np.linspace(2.0, 1.0, iters), GB)
    res, init = _train(obj, X, Y, iters, learning_rate=0.05, early_stop_tol=0.0)
    raw = torch.tensor(init, dtype=torch.float32, requires_grad=True)
    kp = torch.tensor([oe._inv_softplus(F32(0.5)), oe._inv_softplus(F32(1.0))],
                      dtype=torch.float32, requires_grad=True)
    opt = torch.optim.Adam([raw, kp], lr=0.05, betas=(0.9, 0.999), eps=1e-8)
    c, w = torch.tensor(obj.c, dtype=torch.float32), torch.tensor(obj.w, dtype=torch.float32)
    g_kp = torch.tensor([0.3, -0.2], dtype=torch.float32)
    for it in range(iters):
        np.testing.assert_allclose(obj.raw_seen[it], raw.detach().numpy(), rtol=2e-5, atol=1e-6)
        np.testing.assert_allclose(obj.params_seen[it],
                                   torch.nn.functional.softplus(kp).detach().numpy(),
                                   rtol=2e-5, atol=1e-6)
        opt.zero_grad()
        raw.grad = w * (raw.detach() - c)
        kp.grad = g_kp * torch.sigmoid(kp.detach())
        opt.step()
    # W and raw_v: G_B clipped at +-10, W rows updated in place in order
    # one optimiser per W row: row 1's gradient reads row 0 already updated
    # this step (the rows are swept in place, in order)
    W0 = oi.init_w(2, 2)
    rows = [torch.tensor(W0[s], dtype=torch.float32, requires_grad=True) for s in range(2)]
    v = torch.zeros(2, dtype=torch.float32, requires_grad=True)
    opts = [torch.optim.Adam([r], lr=0.05, betas=(0.9, 0.999), eps=1e-8) for r in rows]
    optv = torch.optim.Adam([v], lr=0.05, betas=(0.9, 0.999), eps=1e-8)
    Gc = torch.tensor(np.clip(np.asarray(GB, F32), -10, 10))
    for it in range(iters):
        Wt = torch.stack([r.detach() for r in rows])
        Bt = (Wt.double() @ Wt.double().T).numpy() + np.diag(
            torch.nn.functional.softplus(v).detach().double().numpy())
        np.testing.assert_allclose(obj.B_seen[it], Bt, rtol=2e-5, atol=1e-6)
        for s_, (r, o) in enumerate(zip(rows, opts)):
            Wt = torch.stack([q.detach() for q in rows])
            o.zero_grad()
            r.grad = 2.0 * (Gc[s_] @ Wt)
            o.step()
        optv.zero_grad()
        v.grad = torch.diagonal(Gc) * torch.sigmoid(v.detach())
        optv.step()
    assert res["iterations"] == iters and not res["converged"]


def test_train_mixed_early_stop_and_cosine_rate():
    X, Y = _data()
    seq = np.r_[np.linspace(3.0, 1.0, 5), np.full(20, 1.0)]
    obj = _Scripted(X.shape[0], Y.shape[0], seq, np.zeros((2, 2)))
    res, _ = _train(obj, X, Y, 25, early_stop_tol=1e-4, early_stop_patience=4)
    assert res["converged"] and res["iterations"] == 9  # improvements end at 4
    assert res["final_nll"] == pytest.approx(1.0)
    # cosine: the first step is lr, later steps smaller than a constant-rate run
    obj_c = _Scripted(X.shape[0], Y.shape[0], np.linspace(2, 1, 10), np.zeros((2, 2)))
    _train(obj_c, X, Y, 10, early_stop_tol=0.0, use_cosine_lr=True)
    obj_k = _Scripted(X.shape[0], Y.shape[0], np.linspace(2, 1, 10), np.zeros((2, 2)))
    _train(obj_k, X, Y, 10, early_stop_tol=0.0)
    d_c = np.abs(np.diff(np.array(obj_c.raw_seen), axis=0))
    d_k = np.abs(np.diff(np.array(obj_k.raw_seen), axis=0))
    np.testing.assert_allclose(d_c[0], d_k[0], rtol=1e-5)
    lr8 = oe.cosine_lr(0.05, 8, 10)
    assert np.all(d_c[8] < d_k[8]) and lr8 < 0.05
