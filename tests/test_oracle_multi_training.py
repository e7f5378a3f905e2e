"""Pins of the multi-output training-loop restatements (oracle.lmc.train and
oracle.icm.train) from independent implementations, on the CPU.

Both loops run on scripted objectives through their ``evaluate`` hook, and
their parameter trajectories are compared with torch.optim.Adam (Kingma & Ba
2015, beta = (0.9, 0.999), eps = 1e-8) driven by torch autograd through the
reference's parametrisation:

* LMC (jit_lmc.mojo:699-1529): raw kernel parameters and noise through
  softplus, A_s = L_s L_s^T + diag(softplus(raw_vd_s)) with L_s lower
  triangular, its diagonal through softplus, constant learning rate;
* ICM (jit_multi_output.mojo:130-817): raw kernel parameters, outputscale and
  noise through softplus, A = os B with B = W W^T + diag(softplus(raw_v)),
  optional cosine learning rate (training_utils.mojo:23-40).

The chain rule of A (dNLL/dL = 2 G L, dNLL/dvar_diag = G_ii, dNLL/dW =
2 G_B W, dNLL/dos = sum B o G) is autograd's here.  Both references sweep the
factor in place (jit_lmc.mojo:1277-1295, jit_multi_output.mojo:651-663): the
entries of L (row by row, j <= i) and of W (row-major) take their Adam steps
one at a time, each gradient formed from the current factor (entries already
stepped in this sweep included; the diagonal of L stays at the iteration's
value) and the evaluation's G.  The torch references sweep in the same order,
one torch Adam per swept entry, the gradient from autograd of the first-order
term sum(G o (F F^T)) at the current factor F.  The mean step is the
reference's scaled rule -sum(alpha_t)/(n T): the scripted evaluation returns
alpha with that sum equal to n T dNLL/dmu_t, so autograd's dNLL/dmu_t is the
step's gradient.  The gradient clips (LMC: every gradient at +-10 before the
softplus chain; ICM: G_B = os G_A at +-10) are pinned as known answers of
two Adam steps.
"""

import math

import numpy as np
import pytest
import torch

from oracle import engine as oe
from oracle import icm as oi
from oracle import lmc as ol

F32 = np.float32
LR = 0.05


def _sp(x):
    return torch.nn.functional.softplus(x, beta=1.0, threshold=20.0)


def _isp(v):
    return float(oe._inv_softplus(F32(v)))


# ------------------------------------------------------------------ LMC
class _LmcObjective:
    """f = sum w (theta - c)^2 + wn sum (nu - cn)^2 + wa sum_s |A_s - A*_s|_F^2
    + wm sum (mu - cm)^2, float64."""

    def __init__(self, n, T):
        self.n, self.T = n, T
        self.c = [np.array([0.5, 1.5]), np.array([1.0, 0.8])]
        self.w = [np.array([1.0, 0.5]), np.array([0.8, 0.3])]
        self.cn, self.wn = np.array([0.05, 0.3, 0.2]), 2.0
        self.As = np.array([[[1.0, 0.3, 0.1], [0.3, 0.8, -0.2], [0.1, -0.2, 0.6]],
                            [[0.5, -0.2, 0.3], [-0.2, 1.1, 0.2], [0.3, 0.2, 0.9]]])
        self.wa = 0.5
        self.cm, self.wm = np.array([0.3, -0.4, 0.1]), 1.0
        self.calls = []

    def __call__(self, it, params, A, noise, yc):
        n, T = self.n, self.T
        mu = -np.asarray(yc, np.float64).reshape(T, n)[:, 0]  # Y = 0
        th = [np.asarray(p, np.float64) for p in params]
        nu = np.asarray(noise, np.float64)
        A = np.asarray(A, np.float64)
        self.calls.append(([t.copy() for t in th], nu.copy(), A.copy(), mu.copy()))
        f = (sum(float(np.sum(w * (t - c) ** 2)) for t, c, w in zip(th, self.c, self.w))
             + self.wn * float(np.sum((nu - self.cn) ** 2))
             + self.wa * float(np.sum((A - self.As) ** 2))
             + self.wm * float(np.sum((mu - self.cm) ** 2)))
        kg = np.concatenate([2 * w * (t - c) for t, c, w in zip(th, self.c, self.w)])
        gmu = 2 * self.wm * (mu - self.cm)
        alpha = np.zeros((T, n))
        alpha[:, 0] = -gmu * n * T
        return {"nll": F32(f), "kernel_grads": kg.astype(F32),
                "noise_grads": (2 * self.wn * (nu - self.cn)).astype(F32),
                "G_A": (2 * self.wa * (A - self.As)).astype(F32), "alpha": alpha.reshape(-1)}


def _adam1(value):
    """A scalar parameter with its own torch Adam."""
    p = torch.tensor(float(value), dtype=torch.float32, requires_grad=True)
    return p, torch.optim.Adam([p], lr=LR, betas=(0.9, 0.999), eps=1e-8)


def _sweep_grad(F, G, i, j):
    """d/dF[i, j] of sum(G o (F F^T)) at F (float64 autograd)."""
    Ft = F.detach().double().clone().requires_grad_(True)
    torch.sum(G * (Ft @ Ft.T)).backward()
    return float(Ft.grad[i, j])


def _lmc_torch(obj, init_params, init_noise, R, T, iters):
    raw_k = [torch.tensor([_isp(v) for v in p], dtype=torch.float32, requires_grad=True)
             for p in init_params]
    raw_noise = torch.tensor([_isp(v) for v in init_noise], dtype=torch.float32,
                             requires_grad=True)
    raw_vd = torch.full((R, T), _isp(0.1), dtype=torch.float32, requires_grad=True)
    mu = torch.zeros(T, dtype=torch.float32, requires_grad=True)
    opt = torch.optim.Adam([*raw_k, raw_noise, raw_vd, mu], lr=LR, betas=(0.9, 0.999),
                           eps=1e-8)
    # reference initial state: diag(L_s) = sqrt(1/R), strictly lower
    # L_s[i][j] = 0.01 (s + 1) / R, var_diag = 0.1, mean 0
    Lp = {}
    for s in range(R):
        for i in range(T):
            for j in range(i + 1):
                Lp[s, i, j] = _adam1(_isp(math.sqrt(1.0 / R)) if i == j
                                     else 0.01 * (s + 1) / R)
    c = [torch.tensor(v) for v in obj.c]
    w = [torch.tensor(v) for v in obj.w]
    As = torch.tensor(obj.As)

    def factor(s):
        L = torch.zeros((T, T), dtype=torch.float64)
        for i in range(T):
            for j in range(i + 1):
                v = Lp[s, i, j][0]
                L[i, j] = (_sp(v) if i == j else v).double()
        return L

    out = []
    for _ in range(iters):
        th = [_sp(r).double() for r in raw_k]
        nu = _sp(raw_noise).double()
        Ls = [factor(s) for s in range(R)]
        A = torch.stack([L @ L.T for L in Ls]) + torch.diag_embed(_sp(raw_vd).double())
        A.retain_grad()
        m = mu.double()
        out.append(([t.detach().numpy().copy() for t in th], nu.detach().numpy().copy(),
                     A.detach().numpy().copy(), m.detach().numpy().copy()))
        f = (sum(torch.sum(wi * (t - ci) ** 2) for t, ci, wi in zip(th, c, w))
             + obj.wn * torch.sum((nu - torch.tensor(obj.cn)) ** 2)
             + obj.wa * torch.sum((A - As) ** 2)
             + obj.wm * torch.sum((m - torch.tensor(obj.cm)) ** 2))
        opt.zero_grad()
        for p, _ in Lp.values():
            p.grad = None
        f.backward()
        G = A.grad.detach()
        opt.step()
        for s in range(R):  # in-place sweep of L_s
            F = Ls[s].detach().clone()
            for i in range(T):
                for j in range(i + 1):
                    g = _sweep_grad(F, G[s], i, j)
                    p, o = Lp[s, i, j]
                    if i == j:
                        (gr,) = torch.autograd.grad(_sp(p), p)
                        p.grad = (g * gr).float()
                    else:
                        p.grad = torch.tensor(g, dtype=torch.float32)
                    o.step()
                    if i != j:
                        F[i, j] = float(p.detach())
    return out


def test_lmc_loop_matches_torch_adam():
    R, T, n, iters = 2, 3, 8, 40
    X = np.random.default_rng(0).normal(size=(n, 2))
    init_params = [[1.0, 1.0], [0.7, 1.2]]
    init_noise = [0.1, 0.2, 0.15]
    obj = _LmcObjective(n, T)
    res = ol.train([0, 1], [False, False], X, np.zeros(T * n, F32), init_params, init_noise,
                   [0.0] * T, max_iterations=iters, learning_rate=LR, precond_rank=0,
                   early_stop_tol=0.0, evaluate=obj)
    ref = _lmc_torch(obj, init_params, init_noise, R, T, iters)
    assert len(obj.calls) == iters and len(res["nll_history"]) == iters
    for it, ((th, nu, A, mu), (rth, rnu, rA, rmu)) in enumerate(zip(obj.calls, ref)):
        for t, rt in zip(th, rth):
            np.testing.assert_allclose(t, rt, rtol=5e-5, err_msg=f"params it {it}")
        np.testing.assert_allclose(nu, rnu, rtol=5e-5, err_msg=f"noise it {it}")
        np.testing.assert_allclose(A, rA, rtol=5e-5, atol=1e-6, err_msg=f"A it {it}")
        np.testing.assert_allclose(mu, rmu, rtol=5e-5, atol=1e-6, err_msg=f"mean it {it}")
    # the objective decreased and the result is the best evaluation's state
    k = int(np.argmin(res["nll_history"]))
    assert res["nll_history"][-1] < 0.5 * res["nll_history"][0]
    for p, t in zip(res["params"], obj.calls[k][0]):
        np.testing.assert_allclose(p, t, rtol=1e-6)
    np.testing.assert_allclose(res["A"], obj.calls[k][2], rtol=1e-5, atol=1e-7)


def _adam2(g1, g2, raw0, dchain):
    """Two Adam steps (float64) of a raw parameter whose gradient is
    g_k * dchain(raw) at the current raw value."""
    b1, b2, eps = 0.9, 0.999, 1e-8
    m = v = 0.0
    raw = raw0
    for t, g in ((1, g1), (2, g2)):
        gr = g * dchain(raw)
        m = b1 * m + (1 - b1) * gr
        v = b2 * v + (1 - b2) * gr * gr
        raw = raw - LR * (m / (1 - b1 ** t)) / (math.sqrt(v / (1 - b2 ** t)) + eps)
    return raw


def _sig(x):
    return 1.0 / (1.0 + math.exp(-x))


def test_lmc_gradients_clip_at_10_before_the_softplus_chain():
    """Kernel gradient 100 then 1: the reference clips it to 10 first (its
    second Adam step is then lr m/sqrt(v) of the clipped pair; unclipped it
    would be 4.8x larger)."""
    R, T, n = 1, 1, 4
    X = np.zeros((n, 1))
    seq = {0: 100.0, 1: 1.0}

    def ev(it, params, A, noise, yc):
        return {"nll": F32(1.0 - 0.1 * it), "kernel_grads": np.array([seq.get(it, 0.0), 0.0], F32),
                "noise_grads": np.zeros(T, F32), "G_A": np.zeros((R, T, T), F32),
                "alpha": np.zeros(T * n)}

    calls = []

    def rec(it, params, A, noise, yc):
        calls.append(np.asarray(params[0], np.float64).copy())
        return ev(it, params, A, noise, yc)

    ol.train([0], [False], X, np.zeros(n, F32), [[1.0, 1.0]], [0.1], [0.0], max_iterations=3,
             learning_rate=LR, precond_rank=0, early_stop_tol=0.0, evaluate=rec)
    raw0 = _isp(1.0)
    want = _adam2(10.0, 1.0, raw0, _sig)
    got = float(oe._inv_softplus(F32(calls[2][0])))
    assert got == pytest.approx(want, abs=2e-6)
    assert abs(_adam2(100.0, 1.0, raw0, _sig) - want) > 100 * 2e-6  # the clip matters


# ------------------------------------------------------------------ ICM
class _IcmObjective:
    """f = sum w (theta - c)^2 + wn sum (nu - cn)^2 + wa |os B - A*|_F^2
    + wm sum (mu - cm)^2, float64; dNLL/dos = sum B o G_A."""

    def __init__(self, n, T):
        self.n, self.T = n, T
        self.c, self.w = np.array([0.6, 1.4]), np.array([1.0, 0.4])
        self.cn, self.wn = np.array([0.05, 0.2, 0.15]), 2.0
        self.As = np.array([[1.2, 0.4, 0.1], [0.4, 0.9, -0.2], [0.1, -0.2, 0.7]])
        self.wa = 0.3
        self.cm, self.wm = np.array([0.2, -0.3, 0.5]), 1.0
        self.calls = []

    def __call__(self, it, params, os_, B, noise, yc):
        n, T = self.n, self.T
        mu = -np.asarray(yc, np.float64).reshape(T, n)[:, 0]
        th, nu = np.asarray(params, np.float64), np.asarray(noise, np.float64)
        B = np.asarray(B, np.float64)
        os_ = float(os_)
        self.calls.append((th.copy(), os_, B.copy(), nu.copy(), mu.copy()))
        A = os_ * B
        G = 2 * self.wa * (A - self.As)
        f = (float(np.sum(self.w * (th - self.c) ** 2))
             + self.wn * float(np.sum((nu - self.cn) ** 2))
             + self.wa * float(np.sum((A - self.As) ** 2))
             + self.wm * float(np.sum((mu - self.cm) ** 2)))
        alpha = np.zeros((T, n))
        alpha[:, 0] = -2 * self.wm * (mu - self.cm) * n * T
        return {"nll": F32(f), "kernel_grads": (2 * self.w * (th - self.c)).astype(F32),
                "noise_grads": (2 * self.wn * (nu - self.cn)).astype(F32),
                "G_A": G[None].astype(F32), "grad_outputscale": float(np.sum(B * G)),
                "alpha": alpha.reshape(-1), "cg_iterations": 5}


def _icm_torch(obj, init_params, init_os, init_noise, T, iters, cosine):
    raw_p = torch.tensor([_isp(v) for v in init_params], dtype=torch.float32,
                         requires_grad=True)
    raw_os = torch.tensor(_isp(init_os), dtype=torch.float32, requires_grad=True)
    raw_noise = torch.tensor([_isp(v) for v in init_noise], dtype=torch.float32,
                             requires_grad=True)
    raw_v = torch.zeros(T, dtype=torch.float32, requires_grad=True)
    mu = torch.zeros(T, dtype=torch.float32, requires_grad=True)
    opt = torch.optim.Adam([raw_p, raw_os, raw_noise, raw_v, mu], lr=LR, betas=(0.9, 0.999),
                           eps=1e-8)
    # W starts at the reference's hash initialisation (task_covariance.mojo:
    # 196-203), raw_v at 0 (B's diagonal term softplus(0) = ln 2)
    W0 = oi.init_w(T, T)
    Wp = {(s, r): _adam1(W0[s, r]) for s in range(T) for r in range(T)}
    opts = [opt] + [o for _, o in Wp.values()]
    As = torch.tensor(obj.As)
    out = []
    for it in range(iters):
        if cosine:
            lr_min = LR / 20.0
            for o in opts:
                for gr in o.param_groups:
                    gr["lr"] = lr_min + 0.5 * (LR - lr_min) * (1 + math.cos(math.pi * it / iters))
        th, os_, nu = _sp(raw_p).double(), _sp(raw_os).double(), _sp(raw_noise).double()
        W = torch.stack([torch.stack([Wp[s, r][0] for r in range(T)]) for s in range(T)])
        W = W.detach().double()
        B = (W @ W.T + torch.diag(_sp(raw_v).double()))
        B.retain_grad()
        m = mu.double()
        out.append((th.detach().numpy().copy(), float(os_.detach()), B.detach().numpy().copy(),
                    nu.detach().numpy().copy(), m.detach().numpy().copy()))
        A = os_ * B
        f = (torch.sum(torch.tensor(obj.w) * (th - torch.tensor(obj.c)) ** 2)
             + obj.wn * torch.sum((nu - torch.tensor(obj.cn)) ** 2)
             + obj.wa * torch.sum((A - As) ** 2)
             + obj.wm * torch.sum((m - torch.tensor(obj.cm)) ** 2))
        opt.zero_grad()
        f.backward()
        GB = B.grad.detach()
        opt.step()
        F = W.clone()  # in-place sweep of W, row-major
        for s_ in range(T):
            for r in range(T):
                p, o = Wp[s_, r]
                p.grad = torch.tensor(_sweep_grad(F, GB, s_, r), dtype=torch.float32)
                o.step()
                F[s_, r] = float(p.detach())
    return out


@pytest.mark.parametrize("cosine", [False, True])
def test_icm_loop_matches_torch_adam(cosine):
    T, n, iters = 3, 6, 40
    X = np.random.default_rng(1).normal(size=(n, 2))
    init_params, init_os, init_noise = [1.0, 1.0], 1.0, [0.1, 0.1, 0.1]
    obj = _IcmObjective(n, T)
    res = oi.train(0, False, X, np.zeros(T * n, F32), init_params, init_noise, init_os,
                   [0.0] * T, max_iterations=iters, learning_rate=LR, precond_rank=0,
                   early_stop_tol=0.0, use_cosine_lr=cosine, evaluate=obj)
    ref = _icm_torch(obj, init_params, init_os, init_noise, T, iters, cosine)
    assert len(obj.calls) == iters
    for it, (got, want) in enumerate(zip(obj.calls, ref)):
        th, os_, B, nu, mu = got
        rth, ros, rB, rnu, rmu = want
        np.testing.assert_allclose(th, rth, rtol=5e-5, err_msg=f"params it {it}")
        assert os_ == pytest.approx(ros, rel=5e-5), f"outputscale it {it}"
        np.testing.assert_allclose(B, rB, rtol=5e-5, atol=1e-6, err_msg=f"B it {it}")
        np.testing.assert_allclose(nu, rnu, rtol=5e-5, err_msg=f"noise it {it}")
        np.testing.assert_allclose(mu, rmu, rtol=5e-5, atol=1e-6, err_msg=f"mean it {it}")
    assert res["nll_history"][-1] < 0.5 * res["nll_history"][0]
    k = int(np.argmin(res["nll_history"]))
    np.testing.assert_allclose(res["params"], obj.calls[k][0], rtol=1e-6)
    np.testing.assert_allclose(res["B"], obj.calls[k][2], rtol=1e-6)


def test_icm_task_gradient_clips_at_10():
    """G_B = os G_A of 100 on the first step, then 1: raw_v's step uses the
    gradient clipped to 10 (kernel gradients are not clipped on this path)."""
    T, n = 1, 4
    X = np.zeros((n, 1))
    seq = {0: 100.0, 1: 1.0}
    calls = []

    def ev(it, params, os_, B, noise, yc):
        calls.append(np.asarray(B, np.float64).copy())
        G = np.full((1, T, T), seq.get(it, 0.0) / float(os_), F32)
        return {"nll": F32(1.0 - 0.1 * it), "kernel_grads": np.zeros(2, F32),
                "noise_grads": np.zeros(T, F32), "G_A": G, "grad_outputscale": 0.0,
                "alpha": np.zeros(T * n), "cg_iterations": 5}

    oi.train(0, False, X, np.zeros(n, F32), [1.0, 1.0], [0.1], 1.0, [0.0], max_iterations=3,
             learning_rate=LR, precond_rank=0, early_stop_tol=0.0, evaluate=ev)
    W0 = float(oi.init_w(1, 1)[0, 0])
    # B = W^2 + softplus(raw_v): W moves by -lr sign(2 G_B W) steps as well;
    # recover raw_v from the third evaluation's B and W's own Adam pair
    w2 = _adam2(10.0, 1.0, W0, lambda w: 2.0 * w)
    rv = float(oe._inv_softplus(F32(calls[2][0, 0] - w2 * w2)))
    want = _adam2(10.0, 1.0, 0.0, _sig)
    assert rv == pytest.approx(want, abs=5e-5)
    assert abs(_adam2(100.0, 1.0, 0.0, _sig) - want) > 20 * 5e-5  # the clip matters
