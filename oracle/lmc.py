"""CPU restatement of the reference's LMC multi-output engine — TEST INFRASTRUCTURE ONLY.

Dense NumPy float64 (small n) statement of caspbian/mojogp's Linear Model of
Coregionalization path, used only to check the gfx950 product:

  operator          K_full = sum_s A_s (x) K_s + diag(noise_t) + diag(fixed):
                    JITLMCGradientAdapter.forward_matvec
                    (kernels/jit/jit_lmc.mojo:275-330), task-blocked index
                    t*n + i (kernels/lmc_provider.mojo:113-170)
  Precond           LMCPreconditioner (kernels/lmc_preconditioner.mojo:143-589):
                    P = sum_s A_s (x) L_s L_s^T + D, L_s the greedy pivoted
                    Cholesky of K_s (noise 0), D = noise_t + mean fixed noise
                    (jit_lmc.mojo:856-900); probes z = D^1/2 eps + U w
                    (:590-700) with U = [C_s (x) L_s], C_s = chol(A_s)
  bbmm              bbmm_with_precond on the LMC operator (jit_lmc.mojo:1132)
                    plus _compute_A_and_noise_gradients_jit (:582-696)
  train             train_lmc_jit (jit_lmc.mojo:699-1529)
  predict_mean      predict_lmc_python (jit_engine_lmc_bindings.mojo:1102-1394)
  pathwise          sample_lmc_pathwise_python (:599-797) and the RFF prior
                    of mojogp/pathwise_prior.py:37-160

The probe draws are the counter-hash Gaussians of oracle.engine.gaussian laid
out as the device draws them: without a preconditioner, probe j is
gaussian(N*P, seed)[j*N:(j+1)*N]; with one, eps = gaussian(C*N, seed+1000000)
([C][T][n]) and w = gaussian(C*K, seed) ([C][K], K index off_s + j*r_s + k).
The reference draws these two from Mojo's host randn, which is not
reproducible here; this is a deliberate deviation of the product as well.

What pins each piece (tests/test_oracle_lmc.py): the operator against an
explicit Kronecker assembly and, for T = R = 1, the single-output operator;
the preconditioner's log-determinant against slogdet and its Woodbury apply
against a dense solve; the probe covariance against P by sample moments;
the BBMM gradients by finite differences of the exact NLL and by
convergence to the exact trace with many probes; the pathwise RFF prior by
its covariance converging to the kernel.
"""

from __future__ import annotations

import numpy as np

from . import engine as oe
from . import kernels as ok

F32 = np.float32


# ---------------------------------------------------------------- operator
def latent_kernels(kinds, ards, X, params_list):
    """Dense K_s (noise 0) for every latent."""
    X = np.asarray(X, np.float64)
    return [ok.kernel_matrix(k, X, X, p, a) for k, a, p in zip(kinds, ards, params_list)]


def dense_operator(Ks, A, noise, fixed=None) -> np.ndarray:
    """sum_s kron(A_s, K_s) + diag(noise_t) + diag(fixed[t][i]) (task-blocked)."""
    A = np.asarray(A, np.float64)
    n = Ks[0].shape[0]
    T = A.shape[1]
    out = np.zeros((n * T, n * T))
    for s, K in enumerate(Ks):
        out += np.kron(A[s], K)
    d = np.repeat(np.asarray(noise, np.float64), n)
    if fixed is not None:
        d = d + np.asarray(fixed, np.float64).reshape(-1)
    out[np.diag_indices_from(out)] += d
    return out


def forward_matvec(kinds, ards, X, params_list, A, noise, V, fixed=None) -> np.ndarray:
    """K_full V for task-blocked columns V [C][T*n] (float64)."""
    Kf = dense_operator(latent_kernels(kinds, ards, X, params_list), A, noise, fixed)
    return (Kf @ np.asarray(V, np.float64).T).T


def chol_mixing(A_s: np.ndarray) -> np.ndarray:
    """C_s = chol(A_s), retried with +1e-4 on the diagonal (jit_lmc.mojo:780-788)."""
    try:
        return np.linalg.cholesky(A_s)
    except np.linalg.LinAlgError:
        return np.linalg.cholesky(A_s + 1e-4 * np.eye(A_s.shape[0]))


def precond_noise(noise, fixed, n: int) -> np.ndarray:
    """noise_t + mean_i fixed[t][i] (jit_lmc.mojo:882-888)."""
    d = np.asarray(noise, np.float64).copy()
    if fixed is not None:
        d += np.asarray(fixed, np.float64).reshape(len(d), n).mean(axis=1)
    return d


class Precond:
    """Sum-of-Kronecker preconditioner P = U U^T + D."""

    def __init__(self, Ks, A, noise_t, rank: int, method: int = 0):
        A = np.asarray(A, np.float64)
        self.T = A.shape[1]
        self.n = Ks[0].shape[0]
        self.noise = np.asarray(noise_t, np.float64)
        err = 0.0 if method == 0 else 1e-3
        self.L = [oe.pivoted_cholesky(K, rank, method=method, error_tol=err)[0] for K in Ks]
        self.ranks = [L.shape[1] for L in self.L]
        self.C = [chol_mixing(A[s]) for s in range(A.shape[0])]
        blocks = [np.kron(self.C[s], self.L[s]) for s in range(len(self.L))]
        self.U = np.concatenate(blocks, axis=1)
        self.K = self.U.shape[1]
        self.D = np.repeat(self.noise, self.n)
        self.P = self.U @ self.U.T + np.diag(self.D)
        self.logdet = float(np.linalg.slogdet(self.P)[1])

    def apply(self, R: np.ndarray) -> np.ndarray:
        """P^-1 R for R [N, C]."""
        return np.linalg.solve(self.P, R)

    def sample(self, C: int, seed: int) -> np.ndarray:
        """N(0, P) probes [N, C] in the device's draw layout."""
        N = self.n * self.T
        eps = oe.gaussian(C * N, seed + 1000000).astype(np.float64).reshape(C, N)
        w = oe.gaussian(C * self.K, seed).astype(np.float64).reshape(C, self.K)
        return (np.sqrt(np.float32(1.0) * self.D.astype(F32)).astype(np.float64) * eps
                + w @ self.U.T).T


# ---------------------------------------------------------------- BBMM
def bbmm(kinds, ards, X, params_list, A, noise, y_c, *, fixed=None, num_probes=10,
         max_cg=200, max_tridiag=30, tol=1.0, iteration=0, precond_rank=0, precond_method=0,
         P: Precond | None = None):
    """One LMC BBMM evaluation: NLL per joint entry, inv_quad, logdet, kernel
    gradients (per latent, concatenated), dNLL/dA [R][T][T], dNLL/dnoise [T],
    alpha [T*n] and the CG iteration count.  P: a prebuilt preconditioner
    (else one of precond_rank is built at these parameters, 0: none)."""
    X = np.asarray(X, np.float64)
    A = np.asarray(A, np.float64)
    n = X.shape[0]
    R, T = A.shape[0], A.shape[1]
    N = n * T
    Ks = latent_kernels(kinds, ards, X, params_list)
    Kf = dense_operator(Ks, A, noise, fixed)
    if P is None and precond_rank > 0:
        P = Precond(Ks, A, precond_noise(noise, fixed, n), precond_rank, precond_method)
    Pn = num_probes
    seed = iteration * 104729 + 42
    if P is not None:
        Z = P.sample(Pn, seed)
    else:
        Z = oe.gaussian(N * Pn, seed).astype(np.float64).reshape(Pn, N).T
    pnorm = np.linalg.norm(Z, axis=0)
    Zn = Z / pnorm
    rhs = np.concatenate([np.asarray(y_c, np.float64)[:, None], Zn], axis=1)
    rnorm = np.linalg.norm(rhs, axis=0)
    x, iters, conv, diags, offs = oe.batched_cg(Kf, rhs / rnorm, P, max_cg, max_tridiag, tol)
    sol = x * rnorm
    alpha = sol[:, 0]
    inv_quad = float(np.dot(y_c, alpha))
    logdet = 0.0
    if max_tridiag > 0 and Pn > 0:
        logdet = oe.slq_logdet(diags[1:], offs[1:], N)
        if P is not None:
            logdet += P.logdet
    nll = (0.5 * inv_quad + 0.5 * logdet + 0.5 * N * np.log(2 * np.pi)) / N
    U = sol[:, 1:] * pnorm            # probe solutions
    W = Zn * pnorm                    # right factors
    if P is not None:
        W = P.apply(W)
    kgrads = []
    G_A = np.zeros((R, T, T))
    al = alpha.reshape(T, n)
    Ub = U.T.reshape(Pn, T, n)
    Wb = W.T.reshape(Pn, T, n)
    for s in range(R):
        for g in ok.kernel_gradients(kinds[s], X, X, params_list[s], ards[s]):
            dK = np.kron(A[s], g)
            data = alpha @ dK @ alpha
            trace = np.sum(U * (dK @ W)) if Pn > 0 else 0.0
            kgrads.append((-0.5 * data + 0.5 * trace / max(Pn, 1)) / N)
        K = Ks[s]
        for i in range(T):
            for j in range(T):
                v = -al[i] @ K @ al[j]
                if Pn > 0:
                    v += sum(Ub[k, i] @ K @ Wb[k, j] for k in range(Pn)) / Pn
                G_A[s, i, j] = 0.5 * v / N
    ng = np.zeros(T)
    for t in range(T):
        v = -al[t] @ al[t]
        if Pn > 0:
            v += sum(Ub[k, t] @ Wb[k, t] for k in range(Pn)) / Pn
        ng[t] = 0.5 * v / N
    return {"nll": nll, "inv_quad": inv_quad, "logdet": logdet, "kernel_grads": np.array(kgrads),
            "G_A": G_A, "noise_grads": ng, "alpha": alpha, "cg_iterations": iters,
            "precond_logdet": P.logdet if P is not None else 0.0, "x": x,
            "U": U, "Zn": Zn}


# ---------------------------------------------------------------- training
def _a_from_l(L, vd):
    return L @ L.T + np.diag(vd)


def train(kinds, ards, X, Y_blocked, init_params, init_noise, init_mean, *, trainable=None,
          fixed=None, max_iterations=100, learning_rate=0.05, num_probes=10, max_cg=200,
          max_tridiag=30, cg_tol=1.0, precond_rank=15, precond_method=0,
          rebuild_threshold=0.5, early_stop_tol=1e-4, early_stop_patience=15, evaluate=None):
    """train_lmc_jit restated (jit_lmc.mojo:699-1529): Adam over raw (inverse
    softplus) kernel parameters and noise, L_s (diagonal through softplus,
    strictly lower part unconstrained), var_diag (softplus) and the per-task
    mean, gradient clip 10, NaN recovery, best-NLL tracking and smoothed-NLL
    early stopping.  Float32 host scalars as the reference.

    Test hook: ``evaluate(it, params, A, noise, y_c)`` replaces the BBMM
    evaluation and returns a dict with ``nll``, ``kernel_grads`` (latents'
    parameters concatenated), ``noise_grads``, ``G_A`` ([R][T][T], dNLL/dA_s)
    and ``alpha`` (T*n; the mean step is -sum(alpha_t)/(n T))."""
    sp, isp, dsp = oe._softplus, oe._inv_softplus, oe._softplus_deriv
    X = np.asarray(X, np.float64)
    n = X.shape[0]
    T = len(init_noise)
    R = len(kinds)
    TT = T * T
    Y = np.asarray(Y_blocked, F32).reshape(T, n)
    if trainable is None:
        trainable = [np.ones(len(p), bool) for p in init_params]
    raw = [np.array([isp(v) for v in p], F32) for p in init_params]
    raw_noise = np.array([isp(v) for v in init_noise], F32)
    raw_mean = np.asarray(init_mean, F32).copy()
    init_diag = F32(np.sqrt(F32(1.0) / F32(R)))
    Lall = np.zeros((R, T, T), F32)
    raw_Ld = np.zeros((R, T), F32)
    for s in range(R):
        for i in range(T):
            for j in range(T):
                if i == j:
                    Lall[s, i, j] = init_diag
                elif j < i:
                    Lall[s, i, j] = F32(0.01) * F32(s + 1) / F32(R)
            raw_Ld[s, i] = isp(init_diag)
    raw_vd = np.full((R, T), isp(F32(0.1)), F32)
    nkp = sum(len(p) for p in init_params)
    total = nkp + T + R * TT + R * T + T
    madam = np.zeros(total, F32)
    vadam = np.zeros(total, F32)
    b1, b2, eps, lr = F32(0.9), F32(0.999), F32(1e-8), F32(learning_rate)

    def clip(g):
        g = F32(g)
        return F32(10.0) if g > 10 else (F32(-10.0) if g < -10 else g)

    def adam(idx, g, t):
        m = b1 * madam[idx] + (F32(1) - b1) * F32(g)
        v = b2 * vadam[idx] + (F32(1) - b2) * F32(g) * F32(g)
        madam[idx], vadam[idx] = m, v
        mh = m / (F32(1) - F32(b1 ** t))
        vh = v / (F32(1) - F32(b2 ** t))
        return F32(-lr * mh / (np.sqrt(vh) + eps))

    last_rb = np.concatenate([np.asarray(p, F32) for p in init_params])
    last_rb_noise = np.asarray(init_noise, F32).copy()
    snap = lambda: ([r.copy() for r in raw], raw_noise.copy(), raw_mean.copy(), Lall.copy(),
                    raw_Ld.copy(), raw_vd.copy())
    good = snap()
    best = snap()
    best_alpha = np.zeros(n * T)
    nan_count, last_good, best_nll = 0, F32(1e10), F32(1e30)
    smoothed, patience = F32(1e10), 0
    hist = []
    converged = False
    P_state = None
    iterations = 0
    for it in range(max_iterations):
        iterations = it + 1
        tstep = it + 1
        params = [np.array([sp(v) for v in r], F32) for r in raw]
        noise = np.array([sp(v) for v in raw_noise], F32)
        yc = (Y - raw_mean[:, None]).reshape(-1)
        A = np.zeros((R, T, T), F32)
        for s in range(R):
            vd = np.array([sp(v) for v in raw_vd[s]], F32)
            for i in range(T):
                Lall[s, i, i] = sp(raw_Ld[s, i])
            A[s] = _a_from_l(Lall[s].astype(np.float64), vd).astype(F32)
            try:
                np.linalg.cholesky(A[s].astype(np.float64))
            except np.linalg.LinAlgError:
                A[s] += F32(1e-4) * np.eye(T, dtype=F32)
        rebuild = it == 0
        if not rebuild:
            cur = np.concatenate(params)
            rel = np.abs(cur - last_rb) / (np.abs(last_rb) + F32(1e-8))
            reln = np.abs(noise - last_rb_noise) / (np.abs(last_rb_noise) + F32(1e-8))
            rebuild = max(float(rel.max()), float(reln.max())) > rebuild_threshold
        if rebuild:
            last_rb = np.concatenate(params)
            last_rb_noise = noise.copy()
            P_state = (A.copy(), noise.copy(), [p.copy() for p in params])
        if evaluate is not None:
            ev = evaluate(it, params, A, noise, yc)
        else:
            ev = _bbmm_with_frozen_precond(kinds, ards, X, params, A, noise, yc, fixed,
                                           num_probes, max_cg, max_tridiag, cg_tol, it,
                                           precond_rank, precond_method, P_state)
        nll = F32(ev["nll"])
        hist.append(float(nll))
        if np.isnan(nll):
            nan_count += 1
            last_rb = np.zeros_like(last_rb)  # force a rebuild
            raw = [r.copy() for r in good[0]]
            raw_noise, raw_mean, Lall, raw_Ld = (g.copy() for g in good[1:5])
            raw_vd = good[5] + F32(0.7) * F32(nan_count)
            good = good[:5] + (raw_vd.copy(),)
            continue
        if nll < best_nll:
            best_nll = nll
            best = snap()
            best_alpha = ev["alpha"].copy()
        ai = 0
        off = 0
        for s in range(R):
            for p in range(len(raw[s])):
                if trainable[s][p]:
                    g = clip(ev["kernel_grads"][off + p]) * dsp(raw[s][p])
                    raw[s][p] += adam(ai, g, tstep)
                ai += 1
            off += len(raw[s])
        for t in range(T):
            raw_noise[t] += adam(ai, clip(ev["noise_grads"][t]) * dsp(raw_noise[t]), tstep)
            ai += 1
        G = ev["G_A"].astype(F32)
        for s in range(R):
            for i in range(T):
                for j in range(i + 1):
                    g = F32(0.0)
                    for b in range(T):
                        g += G[s, i, b] * Lall[s, b, j]
                    g = clip(F32(2.0) * g)
                    if i == j:
                        raw_Ld[s, i] += adam(ai, g * dsp(raw_Ld[s, i]), tstep)
                    else:
                        Lall[s, i, j] += adam(ai, g, tstep)
                    ai += 1
                ai += T - 1 - i
        for s in range(R):
            for i in range(T):
                raw_vd[s, i] += adam(ai, clip(G[s, i, i]) * dsp(raw_vd[s, i]), tstep)
                ai += 1
        al = ev["alpha"].reshape(T, n)
        for t in range(T):
            g = clip(F32(-np.sum(al[t].astype(F32), dtype=F32)) / F32(n * T))
            raw_mean[t] += adam(ai, g, tstep)
            ai += 1
        if (last_good - nll) < 2.0 or it < 3:
            nan_count = 0
            last_good = nll
            good = snap()
        prev = smoothed
        smoothed = nll if it == 0 else F32(0.9) * smoothed + F32(0.1) * nll
        if it > 20 and early_stop_tol > 0:
            rel = (prev - smoothed) / (abs(smoothed) + F32(1e-8))
            if early_stop_tol > rel > -0.1:
                patience += 1
                if patience >= early_stop_patience:
                    converged = True
                    break
            else:
                patience = 0
    braw, bnoise, bmean, bL, bLd, bvd = best
    out_params = [np.array([sp(v) for v in r], F32) for r in braw]
    L = bL.copy()
    vdiag = np.zeros((R, T), F32)
    A = np.zeros((R, T, T), F32)
    for s in range(R):
        for i in range(T):
            L[s, i, i] = sp(bLd[s, i])
            vdiag[s, i] = sp(bvd[s, i])
        A[s] = _a_from_l(L[s].astype(np.float64), vdiag[s]).astype(F32)
    return {"params": out_params, "noise": np.array([sp(v) for v in bnoise], F32),
            "mean": bmean, "A": A, "L": L, "var_diag": vdiag, "alpha": best_alpha,
            "nll_history": np.array(hist), "final_nll": float(best_nll) if best_nll < 1e29 else 0.0,
            "iterations": iterations, "converged": converged}


def cat_gradients(tree_s, X, params_s, A_s, cat_specs, raw_cat, ev, clip=10.0,
                  per_entry=True):
    """Categorical raw-parameter gradients of one mixed latent
    (jit_lmc_mixed.mojo:1259-1327): for each constrained parameter theta_k of a
    categorical leaf, dK = A_s (x) (dK_s/dR o dR/dtheta_k) and
        g_k = clip((-0.5 alpha^T dK alpha + (0.5/P) sum_j u_j^T dK zn_j) / N)
    with the probe solutions u_j (scaled by their probe norms) and the
    unit-norm probes zn_j of the evaluation, times the transform's chain
    derivative.  Returns the raw gradients (float32, concatenated over the
    leaves).  per_entry=False, clip=None: the mixed ICM's form (the estimator
    neither divided by N nor clipped, jit_multi_output_mixed.mojo:911-960)."""
    from . import categorical as oc
    D, lv = tree_s.cat_leaf_derivatives(X, X, np.asarray(params_s, np.float64))
    alpha, U, Zn = ev["alpha"], ev["U"], ev["Zn"]
    N = alpha.shape[0]
    Pn = U.shape[1]
    A_s = np.asarray(A_s, np.float64)
    out = []
    off = 0
    for i, (kind, L) in enumerate(cat_specs):
        K = oc.num_params(kind, L)
        rc = np.asarray(raw_cat[off:off + K], F32)
        th = oc.constrain(kind, L, rc)
        dR = oc.correlation_gradients(kind, L, th)
        chain = oc.chain_derivative(kind, L, rc)
        li, lj = lv[i]
        for k in range(K):
            dK = np.kron(A_s, D[i] * dR[k][li[:, None], lj[None, :]])
            val = -0.5 * alpha @ dK @ alpha
            if Pn > 0:
                val += 0.5 / Pn * np.sum(U * (dK @ Zn))
            g = F32(val / N) if per_entry else F32(val)
            if clip is not None:
                g = F32(clip) if g > clip else (F32(-clip) if g < -clip else g)
            out.append(F32(g * F32(chain[k])))
        off += K
    return np.array(out, F32)


def train_mixed(nodes, X, Y_blocked, init_params, init_noise, init_mean, cat_specs,
                init_cat_raw, *, max_iterations=100, learning_rate=0.05, num_probes=10,
                max_cg=200, max_tridiag=30, cg_tol=1.0, precond_rank=15, precond_method=0,
                rebuild_threshold=0.5, early_stop_tol=1e-4, early_stop_patience=15,
                evaluate=None):
    """train_lmc_mixed_jit restated (jit_lmc_mixed.mojo:684-1557): the LMC
    parametrisation and Adam of ``train`` plus per-latent categorical raw
    parameters with their own Adam moments (same step count), and this
    loop's own rules: NaN ends the run, the best-NLL evaluation is the only
    snapshot, after iteration 20 every evaluation not below the best NLL
    (the improving one included, whose counter was just reset) counts toward
    the patience, and the preconditioner rebuild also watches the constrained
    categorical parameters.  nodes: per latent a radial kind code or a kernel
    tree dict; cat_specs[s]: (categorical kind, levels) of latent s's
    categorical leaves in tree order (empty for others); init_cat_raw[s]:
    their raw parameters.  Float32 host scalars as the reference.

    Test hook: ``evaluate(it, trees, params, A, noise, y_c, cat_raw)``
    replaces the BBMM evaluation (dict as ``bbmm`` returns, with ``cat_grads``
    per latent replacing the categorical gradient computation; cat_raw: the
    current raw categorical parameters per latent)."""
    from . import categorical as oc
    sp, isp, dsp = oe._softplus, oe._inv_softplus, oe._softplus_deriv
    X = np.asarray(X, np.float64)
    n, d = X.shape
    T = len(init_noise)
    R = len(nodes)
    Y = np.asarray(Y_blocked, F32).reshape(T, n)
    raw = [np.array([isp(v) for v in p], F32) for p in init_params]
    rcat = [np.asarray(c, F32).copy() for c in init_cat_raw]
    raw_noise = np.array([isp(v) for v in init_noise], F32)
    raw_mean = np.asarray(init_mean, F32).copy()
    init_diag = F32(np.sqrt(F32(1.0) / F32(R)))
    Lall = np.zeros((R, T, T), F32)
    raw_Ld = np.zeros((R, T), F32)
    for s in range(R):
        for i in range(T):
            for j in range(i):
                Lall[s, i, j] = F32(0.01) * F32(s + 1) / F32(R)
            Lall[s, i, i] = init_diag
            raw_Ld[s, i] = isp(init_diag)
    raw_vd = np.full((R, T), isp(F32(0.1)), F32)
    nkp = sum(len(p) for p in init_params)
    total = nkp + T + R * T * T + R * T + T
    madam, vadam = np.zeros(total, F32), np.zeros(total, F32)
    mcat = [np.zeros(len(c), F32) for c in rcat]
    vcat = [np.zeros(len(c), F32) for c in rcat]
    b1, b2, eps, lr = F32(0.9), F32(0.999), F32(1e-8), F32(learning_rate)
    t_step = 0

    def clip(g):
        g = F32(g)
        return F32(10.0) if g > 10 else (F32(-10.0) if g < -10 else g)

    def adam(mm, vv, idx, g):
        m = b1 * mm[idx] + (F32(1) - b1) * F32(g)
        v = b2 * vv[idx] + (F32(1) - b2) * F32(g) * F32(g)
        mm[idx], vv[idx] = m, v
        mh = m / (F32(1) - F32(b1 ** t_step))
        vh = v / (F32(1) - F32(b2 ** t_step))
        return F32(-lr * mh / (np.sqrt(vh) + eps))

    def constrained_cat(s):
        out, off = [], 0
        for kind, L in cat_specs[s]:
            K = oc.num_params(kind, L)
            out.append(oc.constrain(kind, L, rcat[s][off:off + K]))
            off += K
        return np.concatenate(out).astype(F32) if out else np.zeros(0, F32)

    def trees():
        out = []
        for s in range(R):
            if isinstance(nodes[s], dict):
                tabs, off = [], 0
                for kind, L in cat_specs[s]:
                    K = oc.num_params(kind, L)
                    tabs.append(oc.correlation(kind, L, oc.constrain(kind, L,
                                                                  rcat[s][off:off + K])))
                    off += K
                out.append(ok.TreeKernel(nodes[s], d, tabs or None))
            else:
                out.append(nodes[s])
        return out

    def a_all():
        A = np.zeros((R, T, T), F32)
        for s in range(R):
            vd = np.array([sp(v) for v in raw_vd[s]], F32)
            for i in range(T):
                Lall[s, i, i] = sp(raw_Ld[s, i])
            A[s] = _a_from_l(Lall[s].astype(np.float64), vd).astype(F32)
            try:
                np.linalg.cholesky(A[s].astype(np.float64))
            except np.linalg.LinAlgError:
                A[s] += F32(1e-4) * np.eye(T, dtype=F32)
        return A

    ards = [False] * R
    last_p = [np.asarray(p, F32).copy() for p in init_params]
    last_cat = [constrained_cat(s) for s in range(R)]
    last_A = a_all()
    last_noise = np.asarray(init_noise, F32).copy()

    def build(tr, params, A, noise):
        if precond_rank <= 0 or evaluate is not None:
            return None
        return Precond(latent_kernels(tr, ards, X, params), A,
                       precond_noise(noise, None, n), precond_rank, precond_method)

    P = build(trees(), last_p, last_A, last_noise)
    snap = lambda: ([r.copy() for r in raw], [c.copy() for c in rcat], raw_noise.copy(),  # noqa: E731
                    raw_mean.copy(), Lall.copy(), raw_Ld.copy(), raw_vd.copy())
    best = snap()
    best_nll = F32(1e30)
    best_alpha = np.zeros(n * T)
    patience, converged, iterations = 0, False, 0
    hist = []
    for it in range(max_iterations):
        iterations = it + 1
        t_step += 1
        params = [np.array([sp(v) for v in r], F32) for r in raw]
        tr = trees()
        noise = np.array([sp(v) for v in raw_noise], F32)
        yc = (Y - raw_mean[:, None]).reshape(-1)
        A = a_all()
        rel = lambda a, b: float(np.max(np.abs(np.asarray(b, F32) - np.asarray(a, F32))  # noqa: E731
                                        / (np.abs(np.asarray(a, F32)) + F32(1e-8)))) if len(a) else 0.0
        rebuild = (max(rel(last_p[s], params[s]) for s in range(R)) > rebuild_threshold
                   or max(rel(last_cat[s], constrained_cat(s)) for s in range(R)) > rebuild_threshold
                   or rel(last_A.ravel(), A.ravel()) > rebuild_threshold
                   or rel(last_noise, noise) > rebuild_threshold)
        if rebuild:
            P = build(tr, params, A, noise)
            last_p = [p.copy() for p in params]
            last_cat = [constrained_cat(s) for s in range(R)]
            last_A, last_noise = A.copy(), noise.copy()
        if evaluate is not None:
            ev = evaluate(it, tr, params, A, noise, yc, [c.copy() for c in rcat])
        else:
            ev = bbmm(tr, ards, X, params, A, noise, yc, num_probes=num_probes, max_cg=max_cg,
                      max_tridiag=max_tridiag, tol=cg_tol, iteration=it, P=P)
        nll = F32(ev["nll"])
        hist.append(float(nll))
        if np.isnan(nll):
            break
        if nll < best_nll:
            best_nll = nll
            patience = 0
            best = snap()
            best_alpha = np.asarray(ev["alpha"]).copy()
        for s in range(R):  # categorical parameters
            if len(rcat[s]) == 0:
                continue
            g = (ev["cat_grads"][s] if "cat_grads" in ev
                 else cat_gradients(tr[s], X, params[s], A[s], cat_specs[s], rcat[s], ev))
            for k in range(len(rcat[s])):
                rcat[s][k] += adam(mcat[s], vcat[s], k, g[k])
        ai = 0
        off = 0
        for s in range(R):
            for p in range(len(raw[s])):
                g = clip(ev["kernel_grads"][off + p]) * dsp(raw[s][p])
                raw[s][p] += adam(madam, vadam, ai, g)
                ai += 1
            off += len(raw[s])
        for t in range(T):
            raw_noise[t] += adam(madam, vadam, ai, clip(ev["noise_grads"][t]) * dsp(raw_noise[t]))
            ai += 1
        G = np.asarray(ev["G_A"], F32)
        for s in range(R):
            for i in range(T):
                for j in range(i + 1):
                    g = F32(0.0)
                    for b in range(T):
                        g += G[s, i, b] * Lall[s, b, j]
                    g = clip(F32(2.0) * g)
                    if i == j:
                        raw_Ld[s, i] += adam(madam, vadam, ai, g * dsp(raw_Ld[s, i]))
                    else:
                        Lall[s, i, j] += adam(madam, vadam, ai, g)
                    ai += 1
                ai += T - 1 - i
        for s in range(R):
            for i in range(T):
                raw_vd[s, i] += adam(madam, vadam, ai, clip(G[s, i, i]) * dsp(raw_vd[s, i]))
                ai += 1
        al = np.asarray(ev["alpha"]).reshape(T, n)
        for t in range(T):
            g = clip(F32(-np.sum(al[t].astype(F32), dtype=F32)) / F32(n * T))
            raw_mean[t] += adam(madam, vadam, ai, g)
            ai += 1
        if nll >= best_nll and it > 20 and early_stop_tol > 0:
            patience += 1
            if patience >= early_stop_patience:
                converged = True
                break
    braw, bcat, bnoise, bmean, bL, bLd, bvd = best
    L = bL.copy()
    vdiag = np.zeros((R, T), F32)
    A = np.zeros((R, T, T), F32)
    for s in range(R):
        for i in range(T):
            L[s, i, i] = sp(bLd[s, i])
            vdiag[s, i] = sp(bvd[s, i])
        A[s] = _a_from_l(L[s].astype(np.float64), vdiag[s]).astype(F32)
    return {"params": [np.array([sp(v) for v in r], F32) for r in braw], "cat_raw": bcat,
            "noise": np.array([sp(v) for v in bnoise], F32), "mean": bmean, "A": A, "L": L,
            "var_diag": vdiag, "alpha": best_alpha, "nll_history": np.array(hist),
            "final_nll": float(best_nll) if best_nll < 1e29 else 0.0,
            "iterations": iterations, "converged": converged}


def _bbmm_with_frozen_precond(kinds, ards, X, params, A, noise, yc, fixed, num_probes, max_cg,
                              max_tridiag, tol, iteration, precond_rank, precond_method, P_state):
    """bbmm() where the preconditioner keeps the A_s / noise / kernel
    parameters of its last rebuild while the operator uses the current ones."""
    P = None
    if precond_rank > 0 and P_state is not None:
        A_rb, noise_rb, params_rb = P_state
        n = np.asarray(X).shape[0]
        P = Precond(latent_kernels(kinds, ards, X, params_rb), A_rb,
                    precond_noise(noise_rb, fixed, n), precond_rank, precond_method)
    return bbmm(kinds, ards, X, params, A, noise, yc, fixed=fixed, num_probes=num_probes,
                max_cg=max_cg, max_tridiag=max_tridiag, tol=tol, iteration=iteration, P=P)


# ---------------------------------------------------------------- prediction
def predict_mean(kinds, ards, X, Xs, params_list, A, alpha, mean) -> np.ndarray:
    """mean[i][t] = sum_s sum_t' A_s[t][t'] (K_s(X*, X) alpha_t')[i] + mean_t."""
    A = np.asarray(A, np.float64)
    T = A.shape[1]
    n = np.asarray(X).shape[0]
    al = np.asarray(alpha, np.float64).reshape(T, n)
    out = np.zeros((np.asarray(Xs).shape[0], T))
    for s in range(A.shape[0]):
        Kx = ok.kernel_matrix(kinds[s], np.asarray(Xs, np.float64), np.asarray(X, np.float64),
                              params_list[s], ards[s])
        out += (Kx @ al.T) @ A[s].T
    return out + np.asarray(mean, np.float64)[None, :]


def pathwise_correction(kinds, ards, X, Xs, params_list, A, noise, residual, *, fixed=None,
                        max_cg=100, tol=1e-2) -> np.ndarray:
    """correction [m][T] for one residual [T*n]: beta by the per-column CG of
    solve_alpha on K_full, then the LMC cross product."""
    Ks = latent_kernels(kinds, ards, X, params_list)
    Kf = dense_operator(Ks, A, noise, fixed)
    beta = oe.solve_alpha(Kf, np.asarray(residual, np.float64), max_cg, tol)
    return predict_mean(kinds, ards, X, Xs, params_list, A, beta, np.zeros(np.asarray(A).shape[1]))


def rff_prior_values(X, lengthscales, W, phase, outputscale, weights) -> np.ndarray:
    """sample_prior_values over the stationary feature map (float64, cast to
    float32): sqrt(os) * weights @ (sqrt(2/F) cos(X/l @ W^T + phase))^T."""
    Xs = np.asarray(X, np.float64) / np.asarray(lengthscales, np.float64)[None, :]
    F = np.asarray(W).shape[0]
    feats = np.sqrt(max(float(outputscale), 0.0)) * np.sqrt(2.0 / F) * np.cos(
        Xs @ np.asarray(W, np.float64).T + np.asarray(phase, np.float64)[None, :])
    return (np.asarray(weights, np.float64) @ feats.T).astype(F32)
