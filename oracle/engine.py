"""CPU restatement of the reference's exact-GP engine — TEST INFRASTRUCTURE ONLY.

Restates, in NumPy float64 on dense matrices (small n), the algorithm of
caspbian/mojogp's engine so the gfx950 product can be checked against it:

  gaussian              kernels/pivoted_cholesky.mojo:51-86 (counter hash +
                        Box-Muller, bit-identical integer part, float32 math)
  pivoted_cholesky      kernels/pivoted_cholesky.mojo:2104-2444 (greedy,
                        lowest-index ties, early stop at max diag < 1e-10)
  Precond               pivoted_cholesky.mojo:1083-1208 (core inverse with
                        max(noise,1e-6)), 1411-1518 (log|P| via Sylvester),
                        1646-1771 (Woodbury), 1909-2011 (N(0,P) probes)
  batched_cg            kernels/combined_inv_quad_logdet.mojo:81-449 and the
                        safe alpha/beta rules of kernels/cg_solver.mojo:108-255
  slq_logdet            kernels/native_numerics.mojo:403-536
  bbmm_step             kernels/combined_inv_quad_logdet.mojo:452-1140
  train                 kernels/jit/jit_training.mojo:274-1008 with
                        kernels/training_utils.mojo:23-320, kernels/utils.mojo:14-90
  solve_alpha           kernels/jit/jit_prediction.mojo:681-765
  lanczos_inv_root      kernels/jit/jit_prediction.mojo:974-1177 (float64, or
                        fp32 as the reference runs it)
  love_variance_fp32    kernels/jit/jit_prediction.mojo:211-233,1236-1350 in
                        the reference's fp32 arithmetic (a rounding floor)

What pins each piece (tests/test_oracle_engine.py): the RNG by moments and a
Kolmogorov-Smirnov test; pivoted Cholesky by exact reconstruction of low-rank
matrices and a monotone trace error; Woodbury and log|P| by dense inverse and
slogdet; CG by np.linalg.solve; SLQ by closed forms (scaled identity) and by
convergence to slogdet with many probes; BBMM gradients by convergence to the
exact gradient (dense trace) with many probes; alpha by np.linalg.solve;
LOVE by the exact posterior variance at full rank.
"""

from __future__ import annotations

import numpy as np

from . import kernels as ok

F32 = np.float32


# ---------------------------------------------------------------- RNG
def _kdiag(kind, params, Xs=None):
    """k(x, x): the outputscale of a single kernel; for trees k(x*_j, x*_j) per
    test point (linear / polynomial leaves make it vary with x)."""
    if isinstance(kind, ok.TreeKernel):
        if Xs is None:
            return kind.diag(params)
        Xs = np.atleast_2d(np.asarray(Xs, np.float64))
        return np.array([kind.matrix(Xs[j:j + 1], Xs[j:j + 1], params)[0, 0]
                         for j in range(Xs.shape[0])])
    return float(np.asarray(params)[-1])


def gaussian(length: int, seed: int) -> np.ndarray:
    """Counter-hash uniform pair + Box-Muller, float32 (pivoted_cholesky.mojo:51-86)."""
    k = np.arange(1, length + 1, dtype=np.uint64)
    seed = np.uint64(seed % (1 << 64))
    with np.errstate(over="ignore"):
        s1 = k * np.uint64(6364136223846793005) + seed
        s1 ^= s1 >> np.uint64(33)
        s1 *= np.uint64(0xFF51AFD7ED558CCD)
        s1 ^= s1 >> np.uint64(33)
        s2 = k * np.uint64(1442695040888963407) + seed + np.uint64(0xBEEF)
        s2 ^= s2 >> np.uint64(33)
        s2 *= np.uint64(0xC4CEB9FE1A85EC53)
        s2 ^= s2 >> np.uint64(33)
    u1 = ((s1 & np.uint64(0x7FFFFF)).astype(F32) + F32(1.0)) / F32(8388608.0)
    u2 = (s2 & np.uint64(0xFFFFFF)).astype(F32) / F32(16777216.0)
    return (np.sqrt(F32(-2.0) * np.log(u1)) * np.cos(F32(2.0) * F32(3.14159265) * u2)).astype(F32)


# ---------------------------------------------------------------- precond
def _xorshift64(state: int) -> int:
    """One step of the sampler's xorshift64* (pivoted_cholesky.mojo:2308-2312)."""
    m = (1 << 64) - 1
    state ^= state >> 12
    state ^= (state << 25) & m
    state ^= state >> 27
    return (state * 0x2545F4914F6CDD1D) & m


def pivoted_cholesky(K: np.ndarray, rank: int, dtype=np.float32, method: int = 0,
                     error_tol: float = 0.0, adaptive_tol: float = 0.01, seed: int = 42,
                     noise: float = 0.0, diag_value=None, diag_init=None):
    """Pivoted Cholesky of the kernel matrix K (no noise). Returns (L [n,k], k).

    Restates build_pivoted_cholesky_precond_unified
    (pivoted_cholesky.mojo:2104-2444): method 0 greedy (argmax of the residual
    diagonal), 1 rpcholesky and 2 nystrom (pivot drawn proportionally to the
    positive residual diagonal with a host xorshift64 stream, sequential fp32
    sums, :2287-2334).  Stops: residual max < 1e-10; nystrom when
    sum|diag| < adaptive_tol*n*noise after the first pivot; otherwise when
    sum|diag| / diag_value < error_tol.

    Runs at the reference's working precision (fp32 by default): the residual
    diagonal of far-away points rounds to exactly the outputscale, so many
    entries tie and the lowest index wins; a float64 run breaks those ties
    differently and picks other pivots.

    ``diag_init``: the residual diagonal the provider reports, when it is not
    the matrix's own diagonal (the Kronecker operator of the mixed ICM)."""
    n = K.shape[0]
    Kd = np.asarray(K).astype(dtype)
    diag = (np.diag(Kd).copy() if diag_init is None
            else np.asarray(diag_init).astype(dtype).copy())
    dval = dtype(diag_value if diag_value is not None else diag.max())
    mask = np.ones(n, dtype=bool)
    L = np.zeros((n, rank), dtype=dtype)
    actual = rank
    rng = int(seed)
    f32 = np.float32
    for m in range(rank):
        cand = np.where(mask, diag, dtype(-np.inf))
        p = int(np.argmax(cand))           # first maximum = lowest index on ties
        maxval = cand[p]
        if not mask.any() or maxval < 1e-10:
            actual = max(m, 1)
            break
        sumabs = f32(np.abs(diag[mask].astype(np.float64)).sum())
        if method == 2:
            if sumabs < f32(adaptive_tol) * f32(n) * f32(noise) and m > 0:
                actual = m
                break
        elif f32(sumabs / f32(dval)) < f32(error_tol):
            actual = max(m, 1)
            break
        if method != 0:
            d32 = diag.astype(f32)
            w = np.where(mask & (d32 > 0), d32, f32(0.0)).astype(f32)
            csum = np.cumsum(w, dtype=f32)      # sequential fp32 accumulation
            total = csum[-1]
            if total < f32(1e-10):
                actual = max(m, 1)
                break
            rng = _xorshift64(rng)
            u = f32(f32(rng & 0x7FFFFFFF) / f32(2147483648.0))
            u = f32(u * total)
            hit = np.nonzero(mask & (csum >= u))[0]
            if hit.size:
                p = int(hit[0])
                maxval = diag[p]
        mask[p] = False
        col = Kd[:, p] - L[:, :m] @ L[p, :m]
        L[:, m] = col * (dtype(1.0) / np.sqrt(max(maxval, dtype(1e-10))))
        diag[mask] -= L[mask, m] * L[mask, m]
    return L[:, :actual].astype(np.float64), actual


class Precond:
    """P = L L^T + noise I with the reference's cached pieces; with a noise
    vector d [n] (noise mode 1), P = L L^T + diag(d), M = I + L^T D^-1 L
    (pivoted_cholesky.mojo:1209-1240, 1346-1520, 2060-2095)."""

    def __init__(self, L: np.ndarray, noise):
        self.L = L
        self.rank = L.shape[1]
        M = L.T @ L
        self.vec = np.ndim(noise) > 0
        if self.vec:
            self.d = np.asarray(noise, np.float64)
            self.noise = 1e-6
            Mv = np.eye(self.rank) + L.T @ (L / self.d[:, None])
            self.Minv = np.linalg.inv(Mv)
            self.logdet = float(np.sum(np.log(self.d)) + np.linalg.slogdet(Mv)[1])
            return
        self.noise = float(noise)
        eff = max(self.noise, 1e-6)
        self.Minv = np.linalg.inv(M + eff * np.eye(self.rank))
        _, ld = np.linalg.slogdet(np.eye(self.rank) + M / self.noise)
        self.logdet = L.shape[0] * np.log(self.noise) + ld

    def apply(self, V: np.ndarray) -> np.ndarray:
        """(V - L Minv L^T V) / noise for V [n, C] (vector: D^-1 (V - L Minv L^T D^-1 V))."""
        if self.vec:
            W = V / self.d[:, None]
            return (V - self.L @ (self.Minv @ (self.L.T @ W))) / self.d[:, None]
        return (V - self.L @ (self.Minv @ (self.L.T @ V))) / self.noise

    def sample(self, T: int, seed: int) -> np.ndarray:
        """N(0, P) probes [n, T]: L z_rank + sqrt(noise) z_noise."""
        n = self.L.shape[0]
        zr = gaussian(self.rank * T, seed).astype(np.float64).reshape(T, self.rank)
        zn = gaussian(n * T, seed + 1000000).astype(np.float64).reshape(T, n)
        s = (np.sqrt(self.d.astype(np.float32)).astype(np.float64) if self.vec
             else np.sqrt(np.float32(self.noise)))
        return (zr @ self.L.T + s * zn).T


# ---------------------------------------------------------------- CG
def _recip(a):
    return 1.0 if a < 1e-10 else 1.0 / a


def batched_cg(A: np.ndarray, rhs: np.ndarray, P: Precond | None, max_iter: int,
               max_tridiag: int, tol: float, x0: np.ndarray | None = None):
    """Preconditioned mBCG on columns of rhs [n, C]; returns (x, iters, converged, diags, offs)."""
    n, C = rhs.shape
    x = np.zeros_like(rhs) if x0 is None else x0.copy()
    r = rhs - A @ x if x0 is not None else rhs.copy()
    z = P.apply(r) if P is not None else r
    p = z.copy()
    rz_old = np.sum(r * z, axis=0)
    ha, hb = [], []
    iters, converged = 0, False
    for it in range(max_iter):
        iters = it + 1
        Ap = A @ p
        pAp = np.sum(p * Ap, axis=0)
        bad = np.isnan(rz_old) | np.isnan(pAp) | (pAp < 1e-10)
        alpha = np.where(bad, 0.0, rz_old / np.where(bad, 1.0, pAp))
        active = (alpha != 0.0) & ~np.isnan(alpha)
        x[:, active] += alpha[active] * p[:, active]
        r[:, active] -= alpha[active] * Ap[:, active]
        z = P.apply(r) if P is not None else r
        rz_new = np.sum(r * z, axis=0)
        ok_b = ~np.isnan(rz_old) & ~np.isnan(rz_new) & (rz_old >= 1e-20)
        beta = np.where(ok_b, rz_new / (rz_old + 1e-20), 0.0)
        beta = np.where((beta < 0) | np.isnan(beta), 0.0, beta)
        rz_old = np.where(np.isnan(rz_new), 0.0, rz_new)
        p = np.where(beta == 0.0, z, z + beta * p)
        if it < max_tridiag:
            ha.append(alpha.copy())
            hb.append(beta.copy())
        if it >= 10 and ((it + 1) % 10 == 0 or it == max_iter - 1):
            mean_res = np.mean(np.sqrt(np.sum(r * r, axis=0)))
            if mean_res < tol and it >= max_tridiag - 1:
                converged = True
                break
    diags = [[] for _ in range(C)]
    offs = [[] for _ in range(C)]
    for k in range(len(ha)):
        max_off = 0.0
        for c in range(C):
            dv = _recip(ha[k][c])
            if k > 0:
                apr = _recip(ha[k - 1][c])
                dv += hb[k - 1][c] * apr
                off = np.sqrt(max(hb[k - 1][c], 0.0)) * apr
                offs[c].append(off)
                max_off = max(max_off, off)
            diags[c].append(dv)
        if k > 0 and max_off < 1e-6:
            break
    return x, iters, converged, diags, offs


def slq_logdet(diags, offs, n: int) -> float:
    """n * mean over probes of sum_i V0i^2 log(lambda_i) (native_numerics.mojo:403-536)."""
    from scipy.linalg import eigh_tridiagonal
    total, valid = 0.0, 0
    for d, e in zip(diags, offs):
        d = np.asarray(d, np.float64)
        e = np.asarray(e, np.float64)
        if d.size == 0 or np.any(np.isnan(d)) or np.any(np.isnan(e)):
            continue
        if d.size == 1:
            lam, V = d.copy(), np.ones((1, 1))
        else:
            lam, V = eigh_tridiagonal(d, e[: d.size - 1])
        clamp = max(1e-10, float(lam.max())) * 1e-6
        keep = (lam >= 0) & (lam >= clamp)
        total += float(np.sum(V[0, keep] ** 2 * np.log(lam[keep])))
        valid += 1
    return 0.0 if valid == 0 else n * total / valid


# ---------------------------------------------------------------- BBMM
def bbmm_step(kind: int, ard: bool, X, y_c, params, noise: float, P: Precond | None,
              num_probes: int, max_cg: int, max_tridiag: int, tol: float, iteration: int,
              x_warm: np.ndarray | None = None, noise_vec=None):
    """NLL, gradients [P+1] and the CG solution of one BBMM evaluation
    (noise_vec [n]: K + diag(noise_vec), the scalar noise ignored)."""
    X = np.asarray(X, np.float64)
    n = X.shape[0]
    K = ok.kernel_matrix(kind, X, X, params, ard)
    A = K + (np.diag(np.asarray(noise_vec, np.float64)) if noise_vec is not None
             else noise * np.eye(n))
    G = ok.kernel_gradients(kind, X, X, params, ard)
    return bbmm_dense(A, G, y_c, P, num_probes, max_cg, max_tridiag, tol, iteration, x_warm)


def bbmm_dense(A: np.ndarray, dAs, y_c, P: Precond | None, num_probes: int, max_cg: int,
               max_tridiag: int, tol: float, iteration: int,
               x_warm: np.ndarray | None = None):
    """One BBMM evaluation (bbmm_with_precond, combined_inv_quad_logdet.mojo:
    452-1140) of a dense operator A [N, N] with parameter derivatives dAs
    (each [N, N]); the last gradient is the one of a unit diagonal (the noise).
    Returns the NLL per entry, the gradients, alpha, the CG state and the
    factors U (probe solutions at the raw probe scale), W (P^-1 of the raw
    probes) and Zn (unit-norm probes)."""
    n = A.shape[0]
    T = num_probes
    seed = iteration * 104729 + 42
    if P is not None:
        Z = P.sample(T, seed)
    else:
        Z = gaussian(n * T, seed).astype(np.float64).reshape(T, n).T
    pnorm = np.linalg.norm(Z, axis=0)
    Zn = Z / pnorm
    rhs = np.concatenate([np.asarray(y_c, np.float64)[:, None], Zn], axis=1)
    rnorm = np.linalg.norm(rhs, axis=0)
    rhs = rhs / rnorm
    x, iters, conv, diags, offs = batched_cg(A, rhs, P, max_cg, max_tridiag, tol, x_warm)
    sol = x * rnorm
    alpha = sol[:, 0]
    inv_quad = float(np.dot(y_c, alpha))
    logdet = 0.0
    if max_tridiag > 0:
        logdet = slq_logdet(diags[1:], offs[1:], n)
        if P is not None:
            logdet += P.logdet
    nll = (0.5 * inv_quad + 0.5 * logdet + 0.5 * n * np.log(2 * np.pi)) / n
    U = sol[:, 1:] * pnorm
    W = Zn * pnorm
    if P is not None:
        W = P.apply(W)
    grads = []
    for g in dAs:
        data = alpha @ g @ alpha
        trace = np.sum(U * (g @ W)) if T > 0 else 0.0
        grads.append((-0.5 * data + 0.5 * trace / max(T, 1)) / n)
    noise_g = (-0.5 * alpha @ alpha + 0.5 * np.sum(U * W) / max(T, 1)) / n
    grads.append(noise_g)
    # per point: 0.5 (diag(A^-1) estimate - alpha_i^2) (jit_training.mojo:110-145)
    rowdot = -0.5 * alpha * alpha + (0.5 / max(T, 1)) * np.sum(U * W, axis=1)
    return {"nll": nll, "inv_quad": inv_quad, "logdet": logdet, "grads": np.array(grads),
            "alpha": alpha, "x": x, "cg_iterations": iters, "converged": conv,
            "rowdot": rowdot, "U": U, "W": W, "Zn": Zn}


# ---------------------------------------------------------------- learned noise
def learned_noise_vector(mode: int, raw, floor: float, groups=None, X=None) -> np.ndarray:
    """Per-point variances from the learned state (jit_training.mojo:41-84):
    mode 2 softplus(raw_i) + floor, 3 softplus(raw_{group_i}) + floor,
    4 softplus(raw_0 + sum_j raw_{j+1} x_ij) + floor."""
    raw = np.asarray(raw, F32)
    if mode == 2:
        r = raw
    elif mode == 3:
        r = raw[np.asarray(groups)]
    else:
        X = np.asarray(X, F32)
        r = np.full(X.shape[0], raw[0], F32)
        for j in range(X.shape[1]):
            r = (r + raw[j + 1] * X[:, j]).astype(F32)
    return np.array([_softplus(v) for v in r], F32) + F32(floor)


def learned_noise_grad(mode: int, raw, rowdot, floor: float, reg: float, target: float,
                       groups=None, X=None) -> np.ndarray:
    """Gradient of the objective with respect to the raw noise state
    (jit_training.mojo:110-228): per point g_i = rowdot_i / n plus, with
    reg > 0, reg log(noise / target) / (noise * count) (count n per point,
    the group count per group), through the softplus; mode 4 chains g_i to
    the intercept and the weights and adds reg w_p / max(d, 1)."""
    raw = np.asarray(raw, np.float64)
    rowdot = np.asarray(rowdot, np.float64)
    n = rowdot.shape[0]
    target = max(float(target), float(floor))

    def regg(noise, count):
        return reg * np.log(noise / target) / (noise * count) if reg > 0 else 0.0 * noise

    def sp(x):
        return np.logaddexp(0.0, x)

    def dsp(x):
        return 1.0 / (1.0 + np.exp(-x))

    if mode == 2:
        noise = sp(raw) + floor
        return (rowdot / n + regg(noise, n)) * dsp(raw)
    if mode == 3:
        groups = np.asarray(groups)
        G = raw.shape[0]
        s = np.bincount(groups, weights=rowdot / n, minlength=G)
        noise = sp(raw) + floor
        return (s + regg(noise, G)) * dsp(raw)
    X = np.asarray(X, np.float64)
    r = raw[0] + X @ raw[1:]
    noise = sp(r) + floor
    gr = (rowdot / n + regg(noise, n)) * dsp(r)
    g = np.concatenate([[gr.sum()], X.T @ gr])
    if reg > 0:
        g[1:] += reg * raw[1:] / max(X.shape[1], 1)
    return g


# ---------------------------------------------------------------- training
def _softplus(x):
    x = F32(x)
    if x > 20:
        return x
    if x < -20:
        return F32(np.exp(x))
    return F32(np.log(F32(1) + np.exp(x)))


def _inv_softplus(y):
    y = F32(y)
    if y > 20:
        return y
    if y < 1e-6:
        return F32(np.log(y))
    return F32(np.log(np.exp(y) - F32(1)))


def _softplus_deriv(x):
    x = F32(x)
    if x > 20:
        return F32(1)
    if x < -20:
        return F32(np.exp(x))
    return F32(1) / (F32(1) + np.exp(-x))


def _clip(g, m=100.0):
    g = F32(g)
    if np.isnan(g) or g > 1e30 or g < -1e30:
        return F32(0)
    return F32(min(max(g, -m), m))


def cosine_lr(lr_max, iteration: int, total: int):
    """Cosine annealing from lr_max to lr_max/20 (training_utils.mojo:23-40)."""
    lr_max = F32(lr_max)
    lr_min = lr_max / F32(20.0)
    frac = F32(iteration) / F32(max(total, 1))
    return F32(lr_min + F32(0.5) * (lr_max - lr_min) * (F32(1.0) + F32(np.cos(F32(np.pi) * frac))))


def adam_update(raw, m, v, t: int, grads, lr, chain=None):
    """One Adam step on raw (unconstrained) parameters, in fp32
    (training_utils.mojo:214-316): the gradient in constrained space is
    clipped to [-100, 100] (NaN / |g| > 1e30 -> 0), taken through the
    softplus chain rule (or the given d(constrained)/d(raw)), moments with
    beta = (0.9, 0.999), bias correction at step t + 1, eps 1e-8, and the
    new raw value clamped to [-20, 20].  Returns (raw, m, v, t + 1)."""
    raw = np.array(raw, F32)
    m = np.array(m, F32)
    v = np.array(v, F32)
    for q in range(len(raw)):
        d = _softplus_deriv(raw[q]) if chain is None else F32(chain[q])
        gr = _clip(grads[q]) * d
        m[q] = F32(0.9) * m[q] + F32(0.1) * gr
        v[q] = F32(0.999) * v[q] + F32(0.001) * gr * gr
    t += 1
    bc1 = F32(1) - F32(0.9) ** t
    bc2 = F32(1) - F32(0.999) ** t
    for q in range(len(raw)):
        nr = raw[q] - F32(lr) * (m[q] / bc1) / (np.sqrt(v[q] / bc2) + F32(1e-8))
        raw[q] = F32(min(max(nr, -20.0), 20.0))
    return raw, m, v, t


def adam_mean_update(raw_mean, mm, vm, t: int, grad, lr):
    """Adam step of the constant mean (jit_training.mojo:858-875): clipped
    gradient, no chain rule, bias correction with the kernel step's t (already
    incremented), no clamp.  Returns (raw_mean, mm, vm)."""
    mg = _clip(grad)
    mm = F32(0.9) * F32(mm) + F32(0.1) * mg
    vm = F32(0.999) * F32(vm) + F32(0.001) * mg * mg
    bc1 = F32(1) - F32(0.9) ** t
    bc2 = F32(1) - F32(0.999) ** t
    return F32(raw_mean - F32(lr) * (mm / bc1) / (np.sqrt(vm / bc2) + F32(1e-8))), mm, vm


def train(kind: int, ard: bool, X, y, init_params, init_noise: float, *, max_iterations=50,
          learning_rate=0.01, num_probes=10, max_cg=100, cg_tol=1e-2, precond_rank=0,
          max_tridiag=30, rebuild_threshold=0.5, init_mean=None, noise_vec=None,
          learned=None, use_cosine_lr=False, enable_early_stopping=False,
          early_stop_patience=10, early_stop_tol=1e-4, nan_iterations=(), evaluate=None):
    """Adam over raw (inverse-softplus) hyperparameters and the constant mean,
    with preconditioner rebuilds, NaN recovery and best-NLL restore
    (jit_training.mojo:274-1008).  With a fixed noise vector the noise is not
    learned (jit_training.mojo:524, 717, 947: operator noise 0 + the vector,
    noise slot frozen, reported noise 0).

    ``learned``: dict(mode=2|3|4, floor, reg, groups / X) for the learned
    per-point noise modes (jit_training.mojo:352-960): the vector is rebuilt
    from its raw state every iteration, the preconditioner rebuilt every
    iteration, the raw state updated by its own Adam after the kernel step.

    ``use_cosine_lr``: the step uses cosine_lr(learning_rate, it, max_iterations)
    (computed from the initial rate, so NaN halving does not change it;
    jit_training.mojo:697-699).  ``enable_early_stopping``: stop once the NLL
    has not improved on the best-so-far by more than early_stop_tol for
    early_stop_patience iterations (jit_training.mojo:884-905; converged).

    Test hooks: ``nan_iterations`` replaces the evaluated NLL of those
    iterations by NaN (the engine's forced-failure switch), and ``evaluate``
    replaces the BBMM evaluation: evaluate(it, params, noise, y_c, P, warm)
    returns a dict with nll, grads [P + 1], alpha [n], x, cg_iterations."""
    fixed = noise_vec is not None and learned is None
    if learned is not None:
        lmode, lfloor, lreg = learned["mode"], float(learned["floor"]), float(learned["reg"])
        lgroups, lX = learned.get("groups"), learned.get("X")
        S = {2: len(X), 3: int(np.max(lgroups)) + 1 if lgroups is not None else 0,
             4: (np.asarray(X).shape[1] + 1)}[lmode]
        r0 = _inv_softplus(max(F32(init_noise) - F32(lfloor), F32(1e-8)))
        lraw = np.full(S, r0 if lmode != 4 else 0.0, F32)
        lraw[0] = r0
        lm = np.zeros(S, F32)
        lv = np.zeros(S, F32)
        lbest = (lraw.copy(), lm.copy(), lv.copy())
        noise_vec = learned_noise_vector(lmode, lraw, lfloor, lgroups, lX).astype(np.float64)
    X = np.asarray(X, np.float64)
    y = np.asarray(y, np.float64)
    n = X.shape[0]
    Pn = len(init_params)
    init_mean = float(np.mean(y.astype(F32))) if init_mean is None else init_mean
    raw = np.array([_inv_softplus(v) for v in init_params] + [_inv_softplus(init_noise)], F32)
    raw_mean = F32(init_mean)
    m = np.zeros(Pn + 1, F32)
    v = np.zeros(Pn + 1, F32)
    mm = vm = F32(0)
    t = 0
    best = dict(nll=np.inf, raw=raw.copy(), mean=raw_mean, m=m.copy(), v=v.copy(), mm=mm, vm=vm, t=t,
                alpha=None)
    lr = F32(learning_rate)
    nan_iterations = set(int(i) for i in nan_iterations)

    scripted = evaluate is not None  # a scripted objective needs no preconditioner

    def build(params, noise):
        if precond_rank <= 0 or scripted:
            return None
        K = ok.kernel_matrix(kind, X, X, params, ard)
        L, _ = pivoted_cholesky(K, precond_rank)
        return Precond(L, np.asarray(noise_vec, np.float64) if noise_vec is not None else noise)

    if evaluate is None:
        def evaluate(it, params, noise, y_c, P, warm):
            return bbmm_step(kind, ard, X, y_c, params.astype(np.float64), float(noise), P,
                             num_probes, max_cg, max_tridiag, cg_tol, it, warm,
                             noise_vec=noise_vec)

    P = build(np.asarray(init_params, np.float64), init_noise)
    last_params, last_noise = np.asarray(init_params, F32).copy(), F32(init_noise)
    x_prev = None
    nll_hist, cg_hist, lr_hist, rebuild_steps = [], [], [], []
    best_es, no_improve, converged, iterations = F32(1e30), 0, False, 0
    for it in range(max_iterations):
        iterations = it + 1
        params = np.array([_softplus(r) for r in raw[:Pn]], F32)
        noise = F32(0.0) if fixed else _softplus(raw[Pn])
        if learned is not None:
            noise_vec = learned_noise_vector(lmode, lraw, lfloor, lgroups, lX).astype(np.float64)
        if it > 0:
            rel = np.abs(params - last_params) / np.maximum(np.abs(last_params), 1e-8)
            rel = float(rel.max())
            if not fixed:
                rel = max(rel, abs(noise - last_noise) / max(abs(last_noise), 1e-8))
            if learned is not None:
                rel = rebuild_threshold + 1.0
            if rel > rebuild_threshold:
                P = build(params, noise)
                rebuild_steps.append(it)
                last_params, last_noise = params.copy(), noise
        y_c = (y.astype(F32) - raw_mean).astype(np.float64)
        warm = None
        if it > 0 and x_prev is not None:
            warm = x_prev.copy()
            warm[:, 1:] = 0.0
        res = evaluate(it, params, noise, y_c, P, warm)
        x_prev = res.get("x")
        nll = F32(np.nan) if it in nan_iterations else res["nll"]
        cg_hist.append(res["cg_iterations"])
        if np.isnan(nll):
            lr = lr * F32(0.5)
            raw, raw_mean = best["raw"].copy(), best["mean"]
            m, v, mm, vm, t = best["m"].copy(), best["v"].copy(), best["mm"], best["vm"], best["t"]
            params = np.array([_softplus(r) for r in raw[:Pn]], F32)
            noise = F32(0.0) if fixed else _softplus(raw[Pn])
            last_params, last_noise = params.copy(), noise
            if learned is not None:
                lraw, lm, lv = (a.copy() for a in lbest)
                noise_vec = learned_noise_vector(lmode, lraw, lfloor, lgroups,
                                                 lX).astype(np.float64)
            P = build(params, noise)
            rebuild_steps.append(it)
            continue
        if nll < best["nll"]:
            best.update(nll=nll, raw=raw.copy(), mean=raw_mean, m=m.copy(), v=v.copy(), mm=mm,
                        vm=vm, t=t, alpha=np.asarray(res["alpha"]).copy())
            if learned is not None:
                lbest = (lraw.copy(), lm.copy(), lv.copy())
        lr_eff = cosine_lr(learning_rate, it, max_iterations) if use_cosine_lr else lr
        lr_hist.append(float(lr_eff))
        g = np.asarray(res["grads"], F32).copy()
        if fixed:
            g[Pn] = F32(0.0)
        raw, m, v, t = adam_update(raw, m, v, t, g, lr_eff)
        if learned is not None:
            bc1 = F32(1) - F32(0.9) ** t
            bc2 = F32(1) - F32(0.999) ** t
            lg = learned_noise_grad(lmode, lraw, res["rowdot"], lfloor, lreg, init_noise,
                                    lgroups, lX).astype(F32)
            lg[~np.isfinite(lg) | (np.abs(lg) > 1e6)] = 0.0
            lm = (F32(0.9) * lm + F32(0.1) * lg).astype(F32)
            lv = (F32(0.999) * lv + F32(0.001) * lg * lg).astype(F32)
            lraw = (lraw - lr_eff * (lm / bc1) / (np.sqrt(lv / bc2) + F32(1e-8))).astype(F32)
        raw_mean, mm, vm = adam_mean_update(raw_mean, mm, vm, t,
                                            -np.sum(res["alpha"]) / n, lr_eff)
        if np.isnan(raw_mean) or abs(raw_mean) > 1000:
            raw_mean = F32(init_mean)
        nll_hist.append(nll)
        if enable_early_stopping:
            if nll < best_es - F32(early_stop_tol):
                best_es, no_improve = F32(nll), 0
            else:
                no_improve += 1
                if no_improve >= early_stop_patience:
                    converged = True
                    break
    params = np.array([_softplus(r) for r in best["raw"][:Pn]], F32)
    extra = {}
    if learned is not None:
        extra["learned_noise"] = learned_noise_vector(lmode, lbest[0], lfloor, lgroups, lX)
        extra["noise_raw"] = lbest[0].copy()
    return {**extra, "params": params,
            "noise": 0.0 if fixed else float(_softplus(best["raw"][Pn])),
            "mean": float(best["mean"]), "final_nll": float(best["nll"]),
            "alpha": best["alpha"], "nll_history": np.array(nll_hist),
            "cg_iterations_history": np.array(cg_hist), "iterations": iterations,
            "converged": converged, "lr_history": np.array(lr_hist),
            "precond_rebuild_steps": rebuild_steps}


# ---------------------------------------------------------------- prediction
def solve_alpha(A: np.ndarray, rhs: np.ndarray, max_iter: int, tol: float) -> np.ndarray:
    """Unpreconditioned CG with relative-residual stop (jit_prediction.mojo:681-765)."""
    x = np.zeros_like(rhs)
    r = rhs.copy()
    p = r.copy()
    rr_old = float(r @ r)
    init = np.sqrt(rr_old)
    if init < 1e-20:
        init = 1.0
    for _ in range(max_iter):
        Ap = A @ p
        pAp = float(p @ Ap)
        if np.isnan(pAp) or pAp < 1e-10:
            break
        a = rr_old / pAp
        x += a * p
        r -= a * Ap
        rr_new = float(r @ r)
        if np.sqrt(rr_new) / init < tol:
            break
        beta = rr_new / (rr_old + 1e-20) if rr_old >= 1e-20 else 0.0
        if beta < 0 or np.isnan(beta):
            beta = 0.0
        p = r + beta * p
        rr_old = rr_new
    return x


def lanczos_start(n: int, r: int) -> np.ndarray:
    """Deterministic +-1 start vector (jit_prediction.mojo:999-1015), normalised."""
    i = np.arange(n, dtype=np.uint64)
    with np.errstate(over="ignore"):
        s = (np.uint64(0xC0FFEE1234567890) ^ (i * np.uint64(0x9E3779B97F4A7C15))
             ^ (np.uint64(r) * np.uint64(0xBF58476D1CE4E5B9)))
        s ^= s >> np.uint64(12)
        s ^= s << np.uint64(25)
        s ^= s >> np.uint64(27)
        s *= np.uint64(0x2545F4914F6CDD1D)
    z = np.where((s & np.uint64(0x20000)) != 0, 1.0, -1.0)
    return z / np.linalg.norm(z)


def lanczos_inv_root(A: np.ndarray, r: int, dtype=np.float64) -> np.ndarray:
    """S [n, r] with S S^T ~ A^{-1}: Lanczos with full re-orthogonalisation.

    ``dtype=np.float32`` runs the recurrence, the re-orthogonalisation and the
    root S = Q V diag(lambda^-1/2) V^T in fp32, as the reference does
    (jit_prediction.mojo:974-1177, 417-436); the tridiagonal eigensolve stays
    float64 (the reference's is an fp32 QL, native_numerics.mojo:271-400), so
    the fp32 result is if anything closer to exact than the reference's."""
    n = A.shape[0]
    A = np.asarray(A, dtype)
    Q = np.zeros((n, r), dtype)
    alpha = np.zeros(r, dtype)
    beta = np.zeros(max(r - 1, 0), dtype)
    Q[:, 0] = lanczos_start(n, r)
    b_prev = dtype(0.0)
    for j in range(r):
        v = Q[:, j]
        w = A @ v
        alpha[j] = v @ w
        w = w - alpha[j] * v
        if j > 0:
            w = w - b_prev * Q[:, j - 1]
        for _ in range(2):
            inner = Q[:, : j + 1].T @ w
            w = w - Q[:, : j + 1] @ inner
            if np.max(np.abs(inner)) < 1e-5:
                break
        b = np.linalg.norm(w)
        if j < r - 1:
            beta[j] = b
        if b < 1e-10:
            break
        if j + 1 < r:
            Q[:, j + 1] = w / b
        b_prev = b
    from scipy.linalg import eigh_tridiagonal
    al, be = alpha.astype(np.float64), beta.astype(np.float64)
    lam, V = eigh_tridiagonal(al, be) if r > 1 else (al.copy(), np.ones((1, 1)))
    clamp = max(1e-10, lam.max()) * 1e-6
    lam = np.maximum(lam, clamp)
    Tis = ((V / np.sqrt(lam)) @ V.T).astype(dtype)
    return Q @ Tis


def predict(kind: int, ard: bool, X, y, Xs, params, noise: float, mean: float, *,
            max_cg=300, tol=1e-3, lanczos_rank=100, noise_vec=None):
    """Mean and LOVE variance as the reference computes them (noise_vec [n]:
    K + diag(noise_vec) in place of the scalar noise)."""
    X = np.asarray(X, np.float64)
    n = X.shape[0]
    A = ok.kernel_matrix(kind, X, X, params, ard) + (
        np.diag(np.asarray(noise_vec, np.float64)) if noise_vec is not None
        else noise * np.eye(n))
    alpha = solve_alpha(A, np.asarray(y, np.float64) - mean, max_cg, tol)
    Ks = ok.kernel_matrix(kind, Xs, X, params, ard)
    mu = Ks @ alpha + mean
    S = lanczos_inv_root(A, lanczos_rank)
    V = Ks @ S
    var = np.maximum(_kdiag(kind, params, Xs) - np.sum(V * V, axis=1), 1e-10)
    return mu, var, alpha


def love_variance_fp32(kind: int, ard: bool, X, Xs, params, noise: float, *,
                       lanczos_rank=100) -> np.ndarray:
    """LOVE variance in the reference's fp32 arithmetic and order: fp32 kernel
    values (the exact values rounded once, more accurate than any fp32 kernel
    evaluation), the fp32 Lanczos root above, the fp32 cross product K(X*, X) S
    and var = k** - sum_j (K* S)_j^2 summed in fp32 with the 1e-10 floor
    (jit_prediction.mojo:1236-1350, kernel_love_variance :211-233).  Its
    distance from the float64 LOVE (predict) is the rounding floor any fp32
    implementation of the method carries."""
    X = np.asarray(X, np.float64)
    n = X.shape[0]
    A = (ok.kernel_matrix(kind, X, X, params, ard) + noise * np.eye(n)).astype(F32)
    S = lanczos_inv_root(A, lanczos_rank, dtype=F32)
    Ks = ok.kernel_matrix(kind, Xs, X, params, ard).astype(F32)
    W = Ks @ S
    kss = F32(_kdiag(kind, params, Xs))
    return np.maximum(kss - np.sum(W * W, axis=1, dtype=F32), F32(1e-10))


def exact_variance(kind: int, ard: bool, X, Xs, params, noise: float, *, max_cg=300,
                   tol=1e-3, precond_rank=10, block_cols=0, materialized=False, noise_vec=None):
    """Exact predictive variance as the reference computes it
    (jit_prediction.mojo:1357-1789): test columns in blocks (512 on the
    matrix-free route, all when materialized, or block_cols), right-hand sides
    K(X, x*_block) normalised per column, mBCG without tridiagonal under a
    Nystrom pivoted-Cholesky preconditioner (method 2, error_tol 1e-3,
    adaptive_tol 0.01, seed 42), then var = k** - <K_cross, solve> clamped at
    1e-10.  Returns (var, realised preconditioner rank, CG iterations per block).
    With noise_vec [n] the operator is K + diag(noise_vec) and the Nystrom stop
    sees the provider's 1e-6 noise floor (fn_ptr_module.py:673-679)."""
    X = np.asarray(X, np.float64)
    Xs = np.asarray(Xs, np.float64)
    n, m = X.shape[0], Xs.shape[0]
    K = ok.kernel_matrix(kind, X, X, params, ard)
    vec = noise_vec is not None
    A = K + (np.diag(np.asarray(noise_vec, np.float64)) if vec else noise * np.eye(n))
    prior = _kdiag(kind, params, Xs) * np.ones(m)
    # pivot error-ratio hint: k(x, x) of a stationary kernel, the last
    # parameter for trees with linear / polynomial leaves (get_diagonal_value)
    os_ = (float(np.asarray(params)[-1])
           if isinstance(kind, ok.TreeKernel) and kind.nonstationary else _kdiag(kind, params))
    if block_cols > 0:
        block = min(block_cols, m)
    elif materialized:
        block = m
    else:
        block = min(m, 512)
    P = None
    rank = 0
    if precond_rank > 0:
        L, rank = pivoted_cholesky(K, precond_rank, method=2, error_tol=1e-3,
                                   adaptive_tol=0.01, seed=42, noise=1e-6 if vec else noise,
                                   diag_value=os_)
        P = Precond(L, np.asarray(noise_vec, np.float64) if vec else noise)
    var = np.empty(m)
    iters = []
    for s0 in range(0, m, block):
        Kc = ok.kernel_matrix(kind, X, Xs[s0:s0 + block], params, ard)   # [n, C]
        norms = np.linalg.norm(Kc, axis=0)
        norms = np.where(norms > 0, norms, 1.0)
        x, it, _, _, _ = batched_cg(A, Kc / norms, P, max_cg, 0, tol)
        sol = x * norms
        var[s0:s0 + block] = np.maximum(prior[s0:s0 + block] - np.sum(Kc * sol, axis=0), 1e-10)
        iters.append(it)
    return var, rank, iters



# ---------------------------------------------------------------- mixed training
def train_mixed(node: dict, X, y, init_params, init_noise: float, cat_specs, init_cat_raw, *,
                default_dims=None, max_iterations=20, learning_rate=0.01, num_probes=10,
                max_cg=100, cg_tol=1e-2, precond_rank=10, max_tridiag=30,
                rebuild_threshold=0.5, use_cosine_lr=True, init_mean=0.0):
    """Split-Adam training of a mixed continuous x categorical tree
    (kernels/jit/jit_mixed.mojo:428-909, binding defaults of
    jit_engine_bindings.mojo:1241-1460: cosine rate, mean from 0, 30 Lanczos
    steps, rebuild threshold 0.5, preconditioner on).

    Continuous parameters, noise and mean step as in ``train`` (without the
    NaN restore); categorical raw parameters (cat_specs: (kind, L) per leaf,
    oracle.categorical codes) get dNLL/dtheta_k = -0.5 alpha^T dK_k alpha +
    (0.5/S) sum_s (K^-1 z_s)^T dK_k zn_s with the unit-norm probes zn_s, not
    divided by n, clipped, chained through their transforms and stepped by
    their own Adam (raw clamp +-20)."""
    from . import categorical as oc
    X = np.asarray(X, np.float64)
    y = np.asarray(y, np.float64)
    n = X.shape[0]
    Pn = len(init_params)
    sizes = [oc.num_params(k, L) for k, L in cat_specs]
    offs = np.cumsum([0] + sizes)

    def tables(rc):
        return [oc.correlation(k, L, oc.constrain(k, L, rc[offs[i]:offs[i + 1]]))
                for i, (k, L) in enumerate(cat_specs)]

    raw = np.array([_inv_softplus(v) for v in init_params] + [_inv_softplus(init_noise)], F32)
    rcat = np.asarray(init_cat_raw, F32).copy()
    raw_mean = F32(init_mean)
    m = np.zeros(Pn + 1, F32)
    v = np.zeros(Pn + 1, F32)
    mc = np.zeros(rcat.size, F32)
    vc = np.zeros(rcat.size, F32)
    mm = vm = F32(0)
    t = tc = 0
    best = dict(nll=np.inf, raw=raw.copy(), cat=rcat.copy(), mean=raw_mean)
    lr = F32(learning_rate)

    def tree(rc):
        return ok.TreeKernel(node, X.shape[1], tables(rc), default_dims)

    def build(T, params, noise):
        if precond_rank <= 0:
            return None
        L, _ = pivoted_cholesky(T.matrix(X, X, params), precond_rank)
        return Precond(L, noise)

    T0 = tree(rcat)
    P = build(T0, np.asarray(init_params, np.float64), init_noise)
    last_params, last_noise = np.asarray(init_params, F32).copy(), F32(init_noise)
    x_prev = None
    nll_hist = []
    for it in range(max_iterations):
        params = np.array([_softplus(r) for r in raw[:Pn]], F32)
        noise = _softplus(raw[Pn])
        T = tree(rcat)
        if it > 0:
            rel = float((np.abs(params - last_params)
                         / np.maximum(np.abs(last_params), 1e-8)).max())
            rel = max(rel, abs(noise - last_noise) / max(abs(last_noise), 1e-8))
            if rel > rebuild_threshold:
                P = build(T, params.astype(np.float64), float(noise))
                last_params, last_noise = params.copy(), noise
        y_c = (y.astype(F32) - raw_mean).astype(np.float64)
        warm = None
        if it > 0 and x_prev is not None:
            warm = x_prev.copy()
            warm[:, 1:] = 0.0
        res = bbmm_step(T, False, X, y_c, params.astype(np.float64), float(noise), P,
                        num_probes, max_cg, max_tridiag, cg_tol, it, warm)
        x_prev = res["x"]
        nll = res["nll"]
        if np.isnan(nll):
            lr = lr * F32(0.5)
            continue
        if nll < best["nll"]:
            best.update(nll=nll, raw=raw.copy(), cat=rcat.copy(), mean=raw_mean)
        lr_eff = lr
        if use_cosine_lr:
            lr_min = learning_rate / 20.0
            lr_eff = F32(lr_min + 0.5 * (learning_rate - lr_min)
                         * (1.0 + np.cos(np.pi * it / max(max_iterations, 1))))
        g = res["grads"].astype(F32)
        for q in range(Pn + 1):
            gr = _clip(g[q]) * _softplus_deriv(raw[q])
            m[q] = F32(0.9) * m[q] + F32(0.1) * gr
            v[q] = F32(0.999) * v[q] + F32(0.001) * gr * gr
        t += 1
        bc1 = F32(1) - F32(0.9) ** t
        bc2 = F32(1) - F32(0.999) ** t
        for q in range(Pn + 1):
            nr = raw[q] - lr_eff * (m[q] / bc1) / (np.sqrt(v[q] / bc2) + F32(1e-8))
            raw[q] = F32(min(max(nr, -20.0), 20.0))
        mg = _clip(-np.sum(res["alpha"]) / n)
        mm = F32(0.9) * mm + F32(0.1) * mg
        vm = F32(0.999) * vm + F32(0.001) * mg * mg
        raw_mean = F32(raw_mean - lr_eff * (mm / bc1) / (np.sqrt(vm / bc2) + F32(1e-8)))
        if np.isnan(raw_mean) or abs(raw_mean) > 1000:
            raw_mean = F32(init_mean)
        # categorical step
        D, lv = T.cat_leaf_derivatives(X, X, params.astype(np.float64))
        alpha, U, Zn = res["alpha"], res["U"], res["Zn"]
        gc = np.zeros(rcat.size, F32)
        for i, (kind, L) in enumerate(cat_specs):
            th = oc.constrain(kind, L, rcat[offs[i]:offs[i + 1]])
            dR = oc.correlation_gradients(kind, L, th)
            li, lj = lv[i]
            for k in range(sizes[i]):
                dK = D[i] * dR[k][li[:, None], lj[None, :]]
                val = -0.5 * alpha @ dK @ alpha
                if num_probes > 0:
                    val += 0.5 / num_probes * np.sum(U * (dK @ Zn))
                gc[offs[i] + k] = _clip(val)
        chain = np.concatenate([oc.chain_derivative(k, L, rcat[offs[i]:offs[i + 1]])
                                for i, (k, L) in enumerate(cat_specs)]).astype(F32)
        tc += 1
        cb1 = F32(1) - F32(0.9) ** tc
        cb2 = F32(1) - F32(0.999) ** tc
        gr = (gc * chain).astype(F32)
        mc = (F32(0.9) * mc + F32(0.1) * gr).astype(F32)
        vc = (F32(0.999) * vc + F32(0.001) * gr * gr).astype(F32)
        rcat = np.clip(rcat - lr_eff * (mc / cb1) / (np.sqrt(vc / cb2) + F32(1e-8)),
                       -20.0, 20.0).astype(F32)
        nll_hist.append(nll)
    return {"params": np.array([_softplus(r) for r in best["raw"][:Pn]], F32),
            "noise": float(_softplus(best["raw"][Pn])), "mean": float(best["mean"]),
            "final_nll": float(best["nll"]), "cat_raw": best["cat"].copy(),
            "nll_history": np.array(nll_hist)}
