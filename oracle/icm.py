"""CPU restatement of the reference's ICM (Kronecker) multi-output engine — TEST INFRASTRUCTURE ONLY.

Dense NumPy statement of caspbian/mojogp's Intrinsic Coregionalization Model
path, used only to check the gfx950 product (never imported by it):

  init_w / task_b   TaskCovariance (kernels/task_covariance.mojo:168-307):
                    W = 0.1 + 0.4 u from a 31-bit LCG, B = W W^T +
                    diag(softplus(raw_v)) accumulated in fp64
  jacobi_eigen      _symmetric_eigen_cpu (kernels/kronecker_preconditioner.mojo:736-822)
  KronPrecond       KroneckerPreconditioner (:140-730): P = os (B (x) L L^T) +
                    D (x) I with B~ = D^-1/2 B D^-1/2 + 1e-6 I; apply by the
                    eigenbasis Woodbury, log|P| from the eigenvalues, probes
                    D^1/2 z_noise + (C_B (x) L) z_rank
  bbmm              oracle.lmc.bbmm with one latent and A = os B; the ICM
                    gradients follow train_multi_output_jit
                    (kernels/jit/jit_multi_output.mojo:498-598):
                    dNLL/d(os) = sum B o G_A, G_B = os G_A
  train             train_multi_output_jit (:130-817)
  predict           predict_multi_output_python
                    (kernels/jit/jit_engine_multi_output_bindings.mojo:329-549)
  pathwise          sample_multi_output_pathwise_python (:552-712) is the LMC
                    correction with one latent and A = B: oracle.lmc.pathwise_correction
  kron_pivot_precond / mixed_gradients / train_mixed
                    the mixed continuous x categorical ICM
                    (kernels/jit/jit_multi_output_mixed.mojo:477-1148): the
                    single-output BBMM of the full operator under a pivoted
                    Cholesky of that operator, categorical raw parameters
                    trained beside the ICM ones

What pins each piece (tests/test_oracle_icm.py): jacobi_eigen against
numpy.linalg.eigh and the reconstruction V diag(e) V^T; the preconditioner's
apply against a dense solve with the assembled P, its log-determinant against
slogdet(P), the probe factor by C_B C_B^T = os (B + 1e-6 D) and the probes by
their explicit assembly from the two Gaussian streams; the ICM gradients by
finite differences of the exact NLL (many probes); the rotated prediction
against the dense joint posterior (equal task noise makes the eigen-task
decomposition exact); init_w by its range and the LCG's first values worked
out by hand in the test.
"""

from __future__ import annotations

import numpy as np

from . import engine as oe
from . import kernels as ok
from . import lmc as ol

F32 = np.float32


# ---------------------------------------------------------------- task covariance
def init_w(T: int, R: int, seed: int = 42) -> np.ndarray:
    """W [T, R] (task_covariance.mojo:196-203)."""
    out = np.empty(T * R, F32)
    for i in range(T * R):
        state = (seed ^ (i * 2654435761)) & 0xFFFFFFFFFFFFFFFF
        state = (state * 1103515245 + 12345) & 0x7FFFFFFF
        out[i] = F32(0.1) + F32(F32(state) / F32(0x7FFFFFFF)) * F32(0.4)
    return out.reshape(T, R)


def task_b(W: np.ndarray, raw_v: np.ndarray) -> np.ndarray:
    """B = W W^T + diag(softplus(raw_v)) in fp64, stored fp32 (:274-307)."""
    W = np.asarray(W, F32).astype(np.float64)
    v = np.array([oe._softplus(F32(x)) for x in np.asarray(raw_v, F32)], F32).astype(np.float64)
    return (W @ W.T + np.diag(v)).astype(F32)


def jacobi_eigen(A: np.ndarray):
    """Classical Jacobi (largest off-diagonal pivot, tol 1e-12, at most
    100 k^2 rotations) in fp64; eigenvalues ascending, V columns the
    eigenvectors; returned as fp32 like the reference."""
    a = np.asarray(A, F32).astype(np.float64).copy()
    k = a.shape[0]
    v = np.eye(k)
    for _ in range(100 * k * k):
        if k < 2:
            break
        off = np.abs(np.triu(a, 1))
        p, q = np.unravel_index(int(np.argmax(off)), off.shape)
        if off[p, q] < 1e-12:
            break
        app, aqq, apq = a[p, p], a[q, q], a[p, q]
        tau = (aqq - app) / (2.0 * apq)
        t = 1.0 / (tau + np.sqrt(1.0 + tau * tau)) if tau >= 0 else \
            -1.0 / (-tau + np.sqrt(1.0 + tau * tau))
        c = 1.0 / np.sqrt(1.0 + t * t)
        s = t * c
        cp, cq = a[:, p].copy(), a[:, q].copy()
        a[:, p], a[:, q] = c * cp - s * cq, s * cp + c * cq
        rp, rq = a[p, :].copy(), a[q, :].copy()
        a[p, :], a[q, :] = c * rp - s * rq, s * rp + c * rq
        a[p, p], a[q, q] = app - t * apq, aqq + t * apq
        a[p, q] = a[q, p] = 0.0
        vp, vq = v[:, p].copy(), v[:, q].copy()
        v[:, p], v[:, q] = c * vp - s * vq, s * vp + c * vq
    e = np.diag(a).copy()
    for i in range(k):                      # selection sort, first minimum
        mi = i + int(np.argmin(e[i:]))
        if mi != i:
            e[[i, mi]] = e[[mi, i]]
            v[:, [i, mi]] = v[:, [mi, i]]
    return e.astype(F32), v.astype(F32)


# ---------------------------------------------------------------- preconditioner
class KronPrecond:
    """P = os (B (x) L L^T) + D (x) I_n, task-blocked (index t*n + i)."""

    def __init__(self, K_base, os: float, B, noise, rank: int, method: int = 0):
        B = np.asarray(B, F32)
        noise = np.asarray(noise, F32)
        self.T = T = B.shape[0]
        self.n = n = K_base.shape[0]
        self.os = F32(os)
        err = 0.0 if method == 0 else 1e-3
        self.L = oe.pivoted_cholesky(K_base, rank, method=method, error_tol=err)[0]
        self.r = r = self.L.shape[1]
        self.sigma, self.V = jacobi_eigen((self.L.T @ self.L).astype(F32))
        self.dis = (F32(1.0) / np.sqrt(noise)).astype(F32)
        self.ds = np.sqrt(noise).astype(F32)
        Bt = (self.dis[:, None] * B * self.dis[None, :]).astype(F32) + F32(1e-6) * np.eye(T, dtype=F32)
        self.lam, self.Qt = jacobi_eigen(Bt)
        lc = np.maximum(self.lam, F32(1e-8))
        sc = np.maximum(self.sigma, F32(1e-8))
        self.cinv = (F32(1.0) / (F32(1.0) / (self.os * lc[:, None]) + sc[None, :])).astype(F32)
        ld = F32(0.0)
        for t in range(T):
            ld = F32(ld + F32(n) * F32(np.log(noise[t])))
        for j in range(T):
            for i in range(r):
                arg = F32(1.0) + self.os * lc[j] * sc[i]
                ld = F32(ld + F32(np.log(arg if arg > 0 else F32(1e-10))))
        self.logdet = float(ld)
        self.Cb = (np.sqrt(self.os) * self.ds[:, None] * self.Qt
                   * np.sqrt(np.maximum(self.lam, F32(1e-8)))[None, :]).astype(F32)
        self.noise = noise
        self.D = np.repeat(noise.astype(np.float64), n)
        LLt = self.L @ self.L.T
        Beff = B.astype(np.float64) + 1e-6 * np.diag(noise.astype(np.float64))
        self.P = float(self.os) * np.kron(Beff, LLt) + np.diag(self.D)

    def apply(self, Rm: np.ndarray) -> np.ndarray:
        """P^-1 R for R [N, C] by the eigenbasis Woodbury steps 1-7 (:388-520)."""
        T, n = self.T, self.n
        Rm = np.asarray(Rm, np.float64)
        C = Rm.shape[1]
        w = Rm.reshape(T, n, C) * self.dis.astype(np.float64)[:, None, None]
        Y = np.einsum("nk,tnc->ctk", self.L, w)                       # L^T w_t
        Qt, V = self.Qt.astype(np.float64), self.V.astype(np.float64)
        rot = np.einsum("tj,ki,ctk->cji", Qt, V, Y) * self.cinv.astype(np.float64)[None]
        back = np.einsum("tj,ki,cji->ctk", Qt, V, rot)
        Lb = np.einsum("nk,ctk->tnc", self.L, back)
        out = (w - Lb) * self.dis.astype(np.float64)[:, None, None]
        return out.reshape(T * n, C)

    def sample(self, C: int, seed: int) -> np.ndarray:
        """N(0, P) probes [N, C] from the device streams (:629-730)."""
        T, n, r = self.T, self.n, self.r
        N = n * T
        zn = oe.gaussian(N * C, seed + 12345).astype(np.float64).reshape(C, T, n)
        zr = oe.gaussian(r * T * C, seed).astype(np.float64).reshape(T, C, r)
        Lz = np.einsum("nk,tck->ctn", self.L, zr)                     # L z_rank[t, c]
        out = self.ds.astype(np.float64)[None, :, None] * zn + np.einsum(
            "st,ctn->csn", self.Cb.astype(np.float64), Lz)
        return out.reshape(C, N).T


# ---------------------------------------------------------------- BBMM
def bbmm(kind: int, ard: bool, X, params, os: float, B, noise, y_c, *, fixed=None,
         num_probes=10, max_cg=200, max_tridiag=30, tol=1.0, iteration=0, precond_rank=0,
         precond_method=0, P: KronPrecond | None = None):
    """One ICM evaluation: the LMC evaluation with A = os B plus dNLL/d(os)
    and G_B = os G_A (before the reference's +-10 clip)."""
    B = np.asarray(B, np.float64)
    A = (F32(os) * np.asarray(B, F32)).astype(np.float64)[None]
    X = np.asarray(X, np.float64)
    if P is None and precond_rank > 0:
        Kb = ok.kernel_matrix(kind, X, X, params, ard)
        P = KronPrecond(Kb, os, B, noise, precond_rank, precond_method)
    ev = ol.bbmm([kind], [ard], X, [params], A, noise, y_c, fixed=fixed, num_probes=num_probes,
                 max_cg=max_cg, max_tridiag=max_tridiag, tol=tol, iteration=iteration, P=P)
    G = ev["G_A"][0]
    ev["grad_outputscale"] = float(np.sum(B * G))
    ev["grad_B"] = float(os) * G
    return ev


# ---------------------------------------------------------------- training
def train(kind: int, ard: bool, X, Y_blocked, init_params, init_noise, init_os, init_mean, *,
          trainable=None, fixed=None, max_iterations=100, learning_rate=0.05, task_rank=-1,
          num_probes=10, max_cg=200, max_tridiag=30, cg_tol=1e-2, precond_rank=15,
          precond_method=0, rebuild_threshold=0.5, early_stop_patience=15,
          early_stop_tol=1e-4, use_cosine_lr=False, evaluate=None):
    """train_multi_output_jit restated (jit_multi_output.mojo:130-817), fp32
    host scalars; the preconditioner keeps the parameters of its last build.

    Test hook: ``evaluate(it, params, os, B, noise, y_c)`` replaces the BBMM
    evaluation and returns a dict with ``nll``, ``kernel_grads``,
    ``noise_grads``, ``G_A`` ([1][T][T], dNLL/dA for A = os B),
    ``grad_outputscale``, ``alpha`` (T*n) and ``cg_iterations``."""
    sp, isp = oe._softplus, oe._inv_softplus
    X = np.asarray(X, np.float64)
    n = X.shape[0]
    T = len(init_noise)
    R = T if task_rank < 0 else task_rank
    P_ = len(init_params)
    Y = np.asarray(Y_blocked, F32).reshape(T, n)
    trainable = np.ones(P_, bool) if trainable is None else np.asarray(trainable, bool)
    fixed_vec = fixed is not None
    raw_p = np.array([isp(F32(v)) for v in init_params], F32)
    raw_os = isp(F32(init_os))
    raw_noise = np.array([isp(F32(v)) for v in init_noise], F32)
    raw_mean = np.asarray(init_mean, F32).copy()
    W = init_w(T, R)
    raw_v = np.zeros(T, F32)
    total = P_ + 1 + T + T * R + T + T
    madam = np.zeros(total, F32)
    vadam = np.zeros(total, F32)
    b1, b2, eps = F32(0.9), F32(0.999), F32(1e-8)
    use_pre = precond_rank > 0 and not fixed_vec and evaluate is None
    sig = lambda x: F32(1.0) / (F32(1.0) + F32(np.exp(-F32(x))))  # noqa: E731

    def constrained(raw):
        return np.array([sp(F32(v)) for v in raw], F32)

    def build(p, os_, B_, noise_):
        Kb = ok.kernel_matrix(kind, X, X, p, ard)
        return KronPrecond(Kb, os_, B_, noise_, precond_rank, precond_method)

    cur_p, os_ = constrained(raw_p), sp(raw_os)
    noise = constrained(raw_noise)
    B = task_b(W, raw_v)
    P = build(cur_p, os_, B, noise) if use_pre else None
    last = (cur_p.copy(), os_, noise.copy(), B.copy())
    rebuilds = 0
    best_nll, best_seen, has_best, patience = F32(1e30), F32(1e30), False, 0
    best = (raw_p.copy(), raw_os, raw_noise.copy(), raw_mean.copy(), B.copy(), np.zeros(n * T))
    hist, cg_hist = [], []
    converged, iterations, t_step = False, 0, 1

    def adam(idx, g, lr):
        madam[idx] = b1 * madam[idx] + (F32(1) - b1) * F32(g)
        vadam[idx] = b2 * vadam[idx] + (F32(1) - b2) * F32(g) * F32(g)
        mh = madam[idx] / (F32(1) - F32(b1 ** t_step))
        vh = vadam[idx] / (F32(1) - F32(b2 ** t_step))
        return F32(-F32(lr) * mh / (np.sqrt(vh) + eps))

    for it in range(max_iterations):
        iterations = it + 1
        cur_p, os_ = constrained(raw_p), sp(raw_os)
        noise = constrained(raw_noise)
        B = task_b(W, raw_v)
        rebuild = False
        if it > 0:
            rel = lambda a, b: float(np.max(np.abs(np.asarray(b, F32) - np.asarray(a, F32))  # noqa: E731
                                            / (np.abs(np.asarray(a, F32)) + F32(1e-8))))
            mr = max(rel(last[0], cur_p), rel([last[1]], [os_]), rel(last[2], noise),
                     rel(last[3], B))
            rebuild = mr > rebuild_threshold
        if rebuild and use_pre:
            P = build(cur_p, os_, B, noise)
            last = (cur_p.copy(), os_, noise.copy(), B.copy())
            rebuilds += 1
        elif rebuild:
            last = (cur_p.copy(), os_, noise.copy(), B.copy())
            rebuilds += 1
        yc = (Y - raw_mean[:, None]).reshape(-1)
        op_noise = np.zeros(T) if fixed_vec else noise
        if evaluate is not None:
            ev = evaluate(it, cur_p, os_, B, op_noise, yc)
        else:
            ev = bbmm(kind, ard, X, cur_p, os_, B, op_noise, yc, fixed=fixed,
                      num_probes=num_probes, max_cg=max_cg, max_tridiag=max_tridiag, tol=cg_tol,
                      iteration=it, P=P)
        ok_cg = ev["cg_iterations"] < max_cg
        if not ok_cg and use_pre:
            P = build(cur_p, os_, B, noise)
            last = (cur_p.copy(), os_, noise.copy(), B.copy())
            rebuilds += 1
            ev = bbmm(kind, ard, X, cur_p, os_, B, op_noise, yc, fixed=fixed,
                      num_probes=num_probes, max_cg=max_cg, max_tridiag=max_tridiag, tol=cg_tol,
                      iteration=it, P=P)
            ok_cg = ev["cg_iterations"] < max_cg
        nll = F32(ev["nll"])
        hist.append(float(nll))
        cg_hist.append(int(ev["cg_iterations"]))
        if not ok_cg:
            if not has_best:
                best_seen = nll
                best = (raw_p.copy(), raw_os, raw_noise.copy(), raw_mean.copy(), B.copy(),
                        ev["alpha"].copy())
            break
        if nll < best_seen:
            best_seen = nll
            best = (raw_p.copy(), raw_os, raw_noise.copy(), raw_mean.copy(), B.copy(),
                    ev["alpha"].copy())
            has_best = True
        GB = np.clip(F32(os_) * ev["G_A"][0].astype(F32), -10, 10).astype(F32)
        lr = learning_rate
        if use_cosine_lr:
            lr_min = learning_rate / 20.0
            lr = F32(lr_min + 0.5 * (learning_rate - lr_min)
                     * (1.0 + np.cos(np.pi * it / max(max_iterations, 1))))
        ai = 0
        for p in range(P_):
            if trainable[p]:
                g = F32(ev["kernel_grads"][p])
                g = F32(0.0) if not np.isfinite(g) else g
                raw_p[p] += adam(ai, g * sig(raw_p[p]), lr)
            ai += 1
        g_os = F32(ev["grad_outputscale"])
        raw_os = F32(raw_os + adam(ai, g_os * sig(raw_os), lr))
        ai += 1
        for t in range(T):
            if not fixed_vec:
                raw_noise[t] += adam(ai, F32(ev["noise_grads"][t]) * sig(raw_noise[t]), lr)
            ai += 1
        for s in range(T):
            for r in range(R):
                gw = F32(0.0)
                for t in range(T):
                    gw = F32(gw + GB[s, t] * W[t, r])
                W[s, r] += adam(ai, F32(2.0) * gw, lr)
                ai += 1
        for t in range(T):
            raw_v[t] += adam(ai, GB[t, t] * sig(raw_v[t]), lr)
            ai += 1
        al = ev["alpha"].reshape(T, n)
        for t in range(T):
            g = oe._clip(F32(-np.sum(al[t])) / F32(n * T))
            raw_mean[t] += adam(ai, g, lr)
            ai += 1
        t_step += 1
        if early_stop_tol > 0:
            if nll < best_nll - F32(early_stop_tol):
                best_nll, patience = nll, 0
            else:
                patience += 1
                if patience >= early_stop_patience:
                    converged = True
                    break
    bp, bos, bn, bm, bB, balpha = best
    return {"params": constrained(bp), "outputscale": sp(bos), "noise": constrained(bn),
            "mean": bm, "B": bB, "alpha": balpha, "nll_history": np.array(hist),
            "cg_iterations_history": np.array(cg_hist), "final_nll": float(best_seen),
            "iterations": iterations, "converged": converged, "precond_rebuild_count": rebuilds,
            "W": W, "raw_v": raw_v}


# ---------------------------------------------------------------- mixed categorical
def kron_pivot_precond(K, os: float, B, noise, rank: int, method: int = 0) -> oe.Precond:
    """The mixed ICM's preconditioner (jit_multi_output_mixed.mojo:594-611,
    741-755): build_pivoted_cholesky_precond_unified over the full Kronecker
    operator (KroneckerDirectProvider, kronecker_direct_provider.mojo:182-209,
    338-386, 511-553).  Its columns are forward products of unit vectors
    minus the provider noise at the pivot, i.e. columns of
    os (B (x) K) + diag(noise_s - min_t noise_t); the provider noise is the
    smallest task noise; the residual diagonal starts at os B_ss (the provider
    reports a base-kernel diagonal of 1) and the error normaliser is
    max_s os B_ss.  P = L L^T + min noise I."""
    K = np.asarray(K, np.float64)
    n = K.shape[0]
    B = np.asarray(B, F32).astype(np.float64)
    noise = np.asarray(noise, F32)
    T = noise.size
    nmin = F32(noise.min())
    os32 = F32(os)
    Kf = float(os32) * np.kron(B, K) + np.diag(np.repeat((noise - nmin).astype(np.float64), n))
    dB = (os32 * np.diag(np.asarray(B, F32))).astype(F32)
    L, _ = oe.pivoted_cholesky(Kf, rank, method=method,
                               error_tol=0.0 if method == 0 else 1e-3, noise=float(nmin),
                               diag_value=float(dB.max()), diag_init=np.repeat(dB, n))
    return oe.Precond(L, float(nmin))


def mixed_gradients(K, os: float, ev, n: int, T: int):
    """Task-covariance and per-task noise gradients of the mixed ICM
    (jit_multi_output_mixed.mojo:815-885) from one evaluation of the full
    operator: G_B[s][t] = 0.5 os (-a_s^T K a_t + (1/P) sum_j u_js^T K w_jt) / nT
    (before the +-10 clip; u: probe solutions, w: P^-1 probes) and
    g_noise[t] = 0.5 (-a_t^T a_t + (1/P) sum_j u_jt^T w_jt) / nT."""
    K = np.asarray(K, np.float64)
    a = np.asarray(ev["alpha"], np.float64).reshape(T, n)
    U = np.asarray(ev["U"], np.float64)
    W = np.asarray(ev["W"], np.float64)
    P = U.shape[1]
    GB = -(a @ K @ a.T)
    gn = -np.sum(a * a, axis=1)
    for j in range(P):
        u = U[:, j].reshape(T, n)
        w = W[:, j].reshape(T, n)
        GB += (u @ K @ w.T) / P
        gn += np.sum(u * w, axis=1) / P
    return 0.5 * float(os) * GB / (n * T), 0.5 * gn / (n * T)


def train_mixed(node: dict, X, Y_blocked, init_params, init_noise, init_os, init_mean,
                cat_specs, init_cat_raw, *, task_rank=-1, max_iterations=100,
                learning_rate=0.05, num_probes=10, max_cg=200, max_tridiag=30, cg_tol=1e-2,
                precond_rank=15, precond_method=0, rebuild_threshold=0.5,
                use_cosine_lr=False, early_stop_patience=15, early_stop_tol=1e-4,
                evaluate=None):
    """train_multi_output_mixed_jit restated (jit_multi_output_mixed.mojo:477-1148):
    the ICM parametrisation (kernel parameters, outputscale, per-task noise,
    W, raw_v, means; one Adam moment array in that order) plus the raw
    categorical parameters of the kernel tree's categorical leaves (their own
    moments, the same step count), on the single-output BBMM of the full
    operator os (B (x) K) + D (oracle.engine.bbmm_dense) under
    kron_pivot_precond.  This loop's rules: kernel, outputscale, noise and W
    gradients are not clipped (G_B is, at +-10; the mean gradient at +-100);
    categorical gradients are (-0.5 a^T dK a + (0.5/P) sum_j u_j^T dK zn_j)
    times the transform's chain derivative, dK = os (B (x) dK_X), neither
    divided by nT nor clipped; rebuild after iteration 0 when a kernel
    parameter, a constrained categorical parameter, the outputscale, a task
    noise or an entry of B moved by more than the threshold; no NaN handling;
    best-NLL snapshot; early stop after early_stop_patience evaluations not
    below the best by early_stop_tol; cosine rate optional.  Float32 host
    scalars as the reference.

    Test hook: ``evaluate(it, tree, params, os, B, noise, y_c, cat_raw)``
    replaces the evaluation; it returns ``nll``, ``grads`` (kernel params then
    outputscale), ``alpha``, ``G_B`` (before the clip), ``noise_grads``,
    ``cat_grads`` and ``cg_iterations``."""
    from . import categorical as oc
    sp, isp = oe._softplus, oe._inv_softplus
    X = np.asarray(X, np.float64)
    n, d = X.shape
    T = len(init_noise)
    R = T if task_rank < 0 else task_rank
    P_ = len(init_params)
    Y = np.asarray(Y_blocked, F32).reshape(T, n)
    raw_p = np.array([isp(F32(v)) for v in init_params], F32)
    raw_os = isp(F32(init_os))
    raw_noise = np.array([isp(F32(v)) for v in init_noise], F32)
    raw_mean = np.asarray(init_mean, F32).copy()
    rcat = np.asarray(init_cat_raw, F32).copy()
    W = init_w(T, R)
    raw_v = np.zeros(T, F32)
    total = P_ + 1 + T + T * R + T + T
    madam, vadam = np.zeros(total, F32), np.zeros(total, F32)
    mcat, vcat = np.zeros(rcat.size, F32), np.zeros(rcat.size, F32)
    b1, b2, eps = F32(0.9), F32(0.999), F32(1e-8)
    sig = lambda x: F32(1.0) / (F32(1.0) + F32(np.exp(-F32(x))))  # noqa: E731

    def constrained(raw):
        return np.array([sp(F32(v)) for v in raw], F32)

    def constrained_cat(rc):
        out, off = [], 0
        for kind, L in cat_specs:
            k = oc.num_params(kind, L)
            out.append(oc.constrain(kind, L, rc[off:off + k]))
            off += k
        return np.concatenate(out).astype(F32) if out else np.zeros(0, F32)

    def tree(rc):
        tabs, off = [], 0
        for kind, L in cat_specs:
            k = oc.num_params(kind, L)
            tabs.append(oc.correlation(kind, L, oc.constrain(kind, L, rc[off:off + k])))
            off += k
        return ok.TreeKernel(node, d, tabs or None)

    def build(params, rc, os_, B_, noise_):
        if precond_rank <= 0 or evaluate is not None:
            return None
        K = tree(rc).matrix(X, X, np.asarray(params, np.float64))
        return kron_pivot_precond(K, os_, B_, noise_, precond_rank, precond_method)

    # initial preconditioner: the given kernel parameters, round-tripped
    # outputscale and noise (:566-611)
    os0 = sp(raw_os)
    noise0 = constrained(raw_noise)
    B = task_b(W, raw_v)
    P = build(np.asarray(init_params, F32), rcat, os0, B, noise0)
    last = (np.asarray(init_params, F32).copy(), constrained_cat(rcat), os0, noise0.copy(),
            B.copy())
    rebuilds = 0
    best_nll, best_seen, patience = F32(1e30), F32(1e30), 0
    best = (raw_p.copy(), raw_os, raw_noise.copy(), raw_mean.copy(), rcat.copy(), B.copy(),
            np.zeros(n * T))
    hist, cg_hist = [], []
    converged, iterations, t_step = False, 0, 1
    x_prev = None

    def adam(mm, vv, idx, g, lr):
        mm[idx] = b1 * mm[idx] + (F32(1) - b1) * F32(g)
        vv[idx] = b2 * vv[idx] + (F32(1) - b2) * F32(g) * F32(g)
        mh = mm[idx] / (F32(1) - F32(b1 ** t_step))
        vh = vv[idx] / (F32(1) - F32(b2 ** t_step))
        return F32(-F32(lr) * mh / (np.sqrt(vh) + eps))

    rel = lambda a, b: (float(np.max(np.abs(np.asarray(b, F32) - np.asarray(a, F32))  # noqa: E731
                                      / (np.abs(np.asarray(a, F32)) + F32(1e-8))))
                        if np.size(a) else 0.0)
    for it in range(max_iterations):
        iterations = it + 1
        params = constrained(raw_p)
        cc = constrained_cat(rcat)
        os_ = sp(raw_os)
        noise = constrained(raw_noise)
        B = task_b(W, raw_v)
        tr = tree(rcat)
        rebuild = False
        if it > 0:
            mr = max(rel(last[0], params), rel(last[1], cc), rel([last[2]], [os_]),
                     rel(last[3], noise), rel(last[4], B))
            rebuild = mr > rebuild_threshold
        if rebuild:
            P = build(params, rcat, os_, B, noise)
            last = (params.copy(), cc.copy(), os_, noise.copy(), B.copy())
            rebuilds += 1
        yc = (Y - raw_mean[:, None]).reshape(-1)
        if evaluate is not None:
            ev = evaluate(it, tr, params, os_, B, noise, yc, rcat.copy())
        else:
            K = tr.matrix(X, X, params.astype(np.float64))
            Bd = np.asarray(B, F32).astype(np.float64)
            os32 = float(F32(os_))
            A = os32 * np.kron(Bd, K) + np.diag(np.repeat(noise.astype(np.float64), n))
            dAs = [os32 * np.kron(Bd, g) for g in tr.gradients(X, X, params.astype(np.float64))]
            dAs.append(np.kron(Bd, K))
            warm = None
            if it > 0 and not rebuild and x_prev is not None:
                warm = x_prev.copy()
                warm[:, 1:] = 0.0
            ev = oe.bbmm_dense(A, dAs, yc.astype(np.float64), P, num_probes, max_cg,
                               max_tridiag, cg_tol, it, warm)
            ev["grads"] = ev["grads"][:-1]  # kernel params then outputscale
            ev["G_B"], ev["noise_grads"] = mixed_gradients(K, os_, ev, n, T)
            if rcat.size:
                ev["cat_grads"] = ol.cat_gradients(tr, X, params, os32 * Bd, cat_specs, rcat,
                                                   ev, clip=None, per_entry=False)
            x_prev = ev["x"]
        nll = F32(ev["nll"])
        hist.append(float(nll))
        cg_hist.append(int(ev["cg_iterations"]))
        if nll < best_seen:
            best_seen = nll
            best = (raw_p.copy(), raw_os, raw_noise.copy(), raw_mean.copy(), rcat.copy(),
                    B.copy(), np.asarray(ev["alpha"]).copy())
        GB = np.clip(np.asarray(ev["G_B"], F32), -10, 10).astype(F32)
        lr = learning_rate
        if use_cosine_lr:
            lr = oe.cosine_lr(learning_rate, it, max_iterations)
        if rcat.size:
            g = np.asarray(ev["cat_grads"], F32)
            for k in range(rcat.size):
                rcat[k] += adam(mcat, vcat, k, g[k], lr)
        ai = 0
        for p in range(P_):
            raw_p[p] += adam(madam, vadam, ai, F32(ev["grads"][p]) * sig(raw_p[p]), lr)
            ai += 1
        raw_os = F32(raw_os + adam(madam, vadam, ai, F32(ev["grads"][P_]) * sig(raw_os), lr))
        ai += 1
        for t in range(T):
            raw_noise[t] += adam(madam, vadam, ai, F32(ev["noise_grads"][t]) * sig(raw_noise[t]),
                                 lr)
            ai += 1
        for s_ in range(T):
            for r in range(R):
                gw = F32(0.0)
                for t in range(T):
                    gw = F32(gw + GB[s_, t] * W[t, r])
                W[s_, r] += adam(madam, vadam, ai, F32(2.0) * gw, lr)
                ai += 1
        for t in range(T):
            raw_v[t] += adam(madam, vadam, ai, GB[t, t] * sig(raw_v[t]), lr)
            ai += 1
        al = np.asarray(ev["alpha"]).reshape(T, n)
        for t in range(T):
            g = oe._clip(F32(-np.sum(al[t].astype(F32), dtype=F32)) / F32(n * T))
            raw_mean[t] += adam(madam, vadam, ai, g, lr)
            ai += 1
        t_step += 1
        if early_stop_tol > 0:
            if nll < best_nll - F32(early_stop_tol):
                best_nll, patience = nll, 0
            else:
                patience += 1
                if patience >= early_stop_patience:
                    converged = True
                    break
    bp, bos, bn, bm, bc, bB, balpha = best
    return {"params": constrained(bp), "outputscale": sp(bos), "noise": constrained(bn),
            "mean": bm, "cat_raw": bc, "B": bB, "alpha": balpha, "nll_history": np.array(hist),
            "cg_iterations_history": np.array(cg_hist), "final_nll": float(best_seen),
            "iterations": iterations, "converged": converged, "precond_rebuild_count": rebuilds,
            "task_rank": R}


# ---------------------------------------------------------------- prediction
def rotate(os: float, B, alpha_blocked, n: int):
    """The wrapper's eigen-task state (multi_output_gp.py:1956-1975): Q,
    Lambda = max(eig(os B), 1e-6) and alpha_rot = alpha [n, T] @ Q."""
    Bs = float(os) * np.asarray(B, np.float64)
    lam, Q = np.linalg.eigh(Bs)
    T = Bs.shape[0]
    al = np.asarray(alpha_blocked, np.float64).reshape(T, n).T
    return Q, np.maximum(lam, 1e-6), al @ Q


def predict(kind: int, ard: bool, X, Xs, params, alpha_rot, Q, scales, noise: float,
            variance: bool = True):
    """mean [m, T] and exact per-eigen-task variance [m, T] (dense)."""
    X = np.asarray(X, np.float64)
    Xs = np.asarray(Xs, np.float64)
    n = X.shape[0]
    K = ok.kernel_matrix(kind, X, X, params, ard)
    Kx = ok.kernel_matrix(kind, Xs, X, params, ard)
    kss = float(np.asarray(params)[-1])
    cross = Kx @ np.asarray(alpha_rot, np.float64)                     # [m, T]
    mean = cross @ (np.asarray(Q, np.float64) * np.asarray(scales, np.float64)[None, :]).T
    if not variance:
        return mean, None
    T = len(scales)
    var = np.zeros_like(mean)
    for s in range(T):
        if not scales[s] > 1e-8:
            continue
        A = K + (noise / scales[s]) * np.eye(n)
        v = np.maximum(kss - np.sum(Kx * np.linalg.solve(A, Kx.T).T, axis=1), 1e-10)
        var += (np.asarray(Q, np.float64)[:, s] ** 2 * scales[s])[None, :] * v[:, None]
    return mean, var
