"""float64 restatement of the reference kernel arithmetic (test infrastructure).

Reference semantics (caspbian/mojogp):
  * RBF       k = os * exp(-0.5 * sum_d (diff_d / l_d)^2)
  * Matern52  k = os * (1 + sqrt5 r + 5/3 r^2) * exp(max(-sqrt5 r, -20)),
              r = sqrt(max(sum_d (diff_d / l_d)^2 + 1e-20, 1e-20))
  * Matern12  k = os * exp(-r) (isotropic), os * exp(max(-r, -20)) (ARD)
  * Matern32  k = os * (1 + sqrt3 r) * exp(max(-sqrt3 r, -20))
    (codegen_engine/expressions.py:77-240: forward expressions;
     codegen_engine/passes/numerical_stability.py:29-41,62-85: sqrt(max(x,
     1e-20)), and exp(max(x, -20)) only where the post-pass exponent is
     syntactically negative -- a negative constant, a product with a negative
     constant as a direct operand, or c - y with c <= 0.  After from_sympy's
     left-nested products (ir.py:183-190) and CSE that holds for the Matern-3/2
     and 5/2 exponents (exp(max(-1 * u, -20))) and the ARD Matern-1/2 one, and
     not for RBF (iso: exp((-0.5 dist_sq) inv_l^2); ARD: a sum of terms), the
     isotropic Matern-1/2 (exp((-1 r_raw) inv_l)) or periodic leaves.)
  * isotropic kernels use a single lengthscale (params [ls, os]); ARD kernels
    use params [ls_0..ls_{d-1}, os] (kernel.py:324-365, 494-509).
  * forward product: out[c, i] = sum_j k(x_i, x_j) V[c, j] + noise V[c, i]
    (codegen_engine/emit/gpu_kernel.py:151-260).

Pinned by tests/test_oracle_kernels.py: the values and gradients of the
reference's own post-pass expressions at pairs on both sides of the -20 clamp
(tests/golden/ref_kernel_exprs.npz, written by tests/golden/gen_kernel_exprs.py
from the reference's code generator), scikit-learn RBF / Matern(nu=0.5, 1.5,
2.5) kernels, SymPy derivatives and central finite differences of the
gradients.
"""

from __future__ import annotations

import numpy as np

RBF = 0
MATERN52 = 1
MATERN12 = 2
MATERN32 = 3
KINDS = (RBF, MATERN52, MATERN12, MATERN32)

_SQRT5 = np.sqrt(5.0)
_SQRT3 = np.sqrt(3.0)


def _lengthscales(params: np.ndarray, d: int, ard: bool) -> np.ndarray:
    params = np.asarray(params, dtype=np.float64)
    return params[:d] if ard else np.full(d, params[0])


def sq_dist(X1: np.ndarray, X2: np.ndarray, ls: np.ndarray) -> np.ndarray:
    """sum_d ((x1_d - x2_d) / l_d)^2 from per-dimension differences (float64).

    Accumulated one dimension at a time so memory stays at n1*n2 doubles."""
    A = np.asarray(X1, dtype=np.float64) / ls
    B = np.asarray(X2, dtype=np.float64) / ls
    out = np.zeros((A.shape[0], B.shape[0]), dtype=np.float64)
    for k in range(A.shape[1]):
        diff = A[:, k, None] - B[None, :, k]
        out += diff * diff
    return out


def exp_clamped(kind: int, ard: bool) -> bool:
    """Whether the reference's generated code clamps this kernel's exponent at
    -20 (see the module docstring; recorded per kind, iso/ARD and dimension in
    tests/golden/ref_kernel_exprs.json)."""
    if kind == RBF:
        return False
    if kind == MATERN12:
        return bool(ard)
    return True


def _exp_guard(x: np.ndarray, clamp: bool) -> np.ndarray:
    """exp(max(x, -20)) where the reference clamps, exp(x) where it does not."""
    with np.errstate(under="ignore"):
        return np.exp(np.maximum(x, -20.0) if clamp else x)


def kernel_from_sq(kind: int, r2: np.ndarray, os: float, ard: bool = True) -> np.ndarray:
    """Kernel value from the scaled squared distance, with the reference guards
    (``ard`` matters for Matern-1/2 only: its exponent is clamped for ARD
    kernels and not for isotropic ones)."""
    clamp = exp_clamped(kind, ard)
    if kind == RBF:
        return os * _exp_guard(-0.5 * r2, clamp)
    r = np.sqrt(np.maximum(r2 + 1e-20, 1e-20))
    if kind == MATERN12:
        return os * _exp_guard(-r, clamp)
    if kind == MATERN32:
        return os * (1.0 + _SQRT3 * r) * _exp_guard(-_SQRT3 * r, clamp)
    return os * (1.0 + _SQRT5 * r + (5.0 / 3.0) * r * r) * _exp_guard(-_SQRT5 * r, clamp)


def kernel_matrix(kind: int, X1, X2, params, ard: bool) -> np.ndarray:
    """K(X1, X2) in float64 (``kind`` may be a TreeKernel; ``ard`` is then unused)."""
    if isinstance(kind, TreeKernel):
        return kind.matrix(X1, X2, params)
    X1 = np.atleast_2d(np.asarray(X1, dtype=np.float64))
    X2 = np.atleast_2d(np.asarray(X2, dtype=np.float64))
    d = X1.shape[1]
    ls = _lengthscales(params, d, ard)
    os = float(np.asarray(params, dtype=np.float64)[-1])
    return kernel_from_sq(kind, sq_dist(X1, X2, ls), os, ard)


def forward_matvec(kind: int, X, V, params, noise: float, ard: bool,
                   rows: np.ndarray | None = None, block: int = 256) -> np.ndarray:
    """(K + noise I) V for V of shape (ncols, n), optionally only for `rows`.

    Returns shape (ncols, len(rows)) (all rows by default).  Blocked so that
    n = 250 000 fits in memory.
    """
    X = np.asarray(X, dtype=np.float64)
    V = np.atleast_2d(np.asarray(V, dtype=np.float64))
    idx = np.arange(X.shape[0]) if rows is None else np.asarray(rows)
    out = np.empty((V.shape[0], idx.shape[0]), dtype=np.float64)
    for s in range(0, idx.shape[0], block):
        r = idx[s:s + block]
        Kb = kernel_matrix(kind, X[r], X, params, ard)
        out[:, s:s + block] = V @ Kb.T + noise * V[:, r]
    return out


def cross_matvec(kind: int, Xs, X, V, params, ard: bool, block: int = 256) -> np.ndarray:
    """K(Xs, X) V for V of shape (ncols, n); returns (ncols, m)."""
    Xs = np.asarray(Xs, dtype=np.float64)
    V = np.atleast_2d(np.asarray(V, dtype=np.float64))
    out = np.empty((V.shape[0], Xs.shape[0]), dtype=np.float64)
    for s in range(0, Xs.shape[0], block):
        Kb = kernel_matrix(kind, Xs[s:s + block], X, params, ard)
        out[:, s:s + block] = V @ Kb.T
    return out


def kernel_gradients(kind: int, X1, X2, params, ard: bool) -> np.ndarray:
    """dK/dtheta_p for every engine parameter p, shape (P, n1, n2), float64.

    The reference differentiates the unclamped forward expression with SymPy and
    then applies the same exp guard to the result (numerical_stability pass runs
    on gradients too, passes/numerical_stability.py:92-112; after CSE the
    gradients share the forward's exp let, so they are clamped exactly where
    the forward is); for Matern the r in d/dl cancels analytically
    (overrides.py:24-41).
      RBF:      dk/dl_d = k * diff_d^2 / l_d^3
      Matern52: dk/dl_d = (5/3) os (1 + sqrt5 r) exp(max(-sqrt5 r, -20)) diff_d^2 / l_d^3
      Matern32: dk/dl_d = 3 os exp(max(-sqrt3 r, -20)) diff_d^2 / l_d^3
      Matern12: dk/dl_d = os exp(-r) / r diff_d^2 / l_d^3 (r floored as above;
                exp(max(-r, -20)) for ARD)
      all:      dk/dos  = k / os
    Isotropic: dk/dl = sum_d of the per-dimension terms with l_d = l.
    """
    if isinstance(kind, TreeKernel):
        return kind.gradients(X1, X2, params)
    X1 = np.atleast_2d(np.asarray(X1, dtype=np.float64))
    X2 = np.atleast_2d(np.asarray(X2, dtype=np.float64))
    d = X1.shape[1]
    p = np.asarray(params, dtype=np.float64)
    ls = _lengthscales(p, d, ard)
    os = p[-1]
    diff2 = (X1[:, None, :] - X2[None, :, :]) ** 2          # raw differences
    r2 = diff2 @ (1.0 / ls**2)
    k = kernel_from_sq(kind, r2, os, ard)
    h = _grad_factor(kind, r2, os, ard, k)
    terms = diff2 / ls**3                                    # (n1, n2, d)
    if ard:
        g = [h * terms[:, :, q] for q in range(d)]
    else:
        g = [h * terms.sum(axis=2)]
    g.append(k / os)
    return np.stack(g, axis=0)


def _grad_factor(kind: int, r2: np.ndarray, os: float, ard: bool, k: np.ndarray) -> np.ndarray:
    """h with dk/dl_q = h diff_q^2 / l_q^3 (radial kinds; see kernel_gradients)."""
    if kind == RBF:
        return k
    r = np.sqrt(np.maximum(r2 + 1e-20, 1e-20))
    clamp = exp_clamped(kind, ard)
    if kind == MATERN12:
        return os * _exp_guard(-r, clamp) / r
    if kind == MATERN32:
        return 3.0 * os * _exp_guard(-_SQRT3 * r, clamp)
    return (5.0 / 3.0) * os * (1.0 + _SQRT5 * r) * _exp_guard(-_SQRT5 * r, clamp)


def gradient_matvec(kind: int, X, V, params, ard: bool, rows: np.ndarray | None = None,
                    block: int = 8) -> np.ndarray:
    """out[p, c, i] = sum_j dk_p(x_i, x_j) V[c, j] (reference fused_gradient_matvec
    layout out[p*n*C + c*n + i], gpu_kernel.py:382-484), optionally only for
    `rows` (shape (P, ncols, len(rows)), blocks of `block` rows so large n fits)."""
    V = np.atleast_2d(np.asarray(V, dtype=np.float64))
    if rows is None:
        G = kernel_gradients(kind, X, X, params, ard)
        return np.einsum("pij,cj->pci", G, V)
    X = np.asarray(X, dtype=np.float64)
    idx = np.asarray(rows)
    out = None
    for s in range(0, idx.shape[0], block):
        r = idx[s:s + block]
        G = kernel_gradients(kind, X[r], X, params, ard)          # (P, nr, n)
        P_, nr = G.shape[0], G.shape[1]
        part = (G.reshape(P_ * nr, -1) @ V.T).reshape(P_, nr, -1).transpose(0, 2, 1)
        if out is None:
            out = np.empty((G.shape[0], V.shape[0], idx.shape[0]), dtype=np.float64)
        out[:, :, s:s + block] = part
    return out


# ---------------------------------------------------------------------------
# Composite kernel trees
#
# Reference semantics: mojogp/kernel.py:722-803 (recursive evaluation, a
# node's active_dims slice its inputs, a scale factor follows its subtree in
# the parameter vector, kernel.py:528-568) with the leaf expressions of the
# engine (codegen_engine/expressions.py:77-326):
#   RQ        k = os (1 + r^2 / (2 alpha))^-alpha, r^2 = sum_q (dx_q / l_q)^2
#   Periodic  k = os exp(-2 S), S = sum_q sin^2(pi dx_q / period) / l_q (no clamp)
#             (isotropic: sum_q sin^2(pi dx_q / period) / l)
# and the radial leaves as above.  Pinned by tests/test_oracle_tree.py:
# scikit-learn RBF / Matern / RationalQuadratic / ExpSineSquared leaves,
# Sum / Product / ConstantKernel compositions, and central finite
# differences of the gradients.
# ---------------------------------------------------------------------------

RQ_LEAF = "RQ"
PERIODIC_LEAF = "PERIODIC"
_RADIAL_NAMES = {"RBF": RBF, "MATERN52": MATERN52, "MATERN12": MATERN12, "MATERN32": MATERN32}


CAT_LEAVES = ("GD", "CR", "EHH", "HH", "FE")


class TreeKernel:
    """A kernel tree given as nested dicts (``kernel_type`` or ``operator``,
    ``left`` / ``right``, ``ard_dim``, ``active_dims``, ``levels``) over ``dim``
    inputs.  Categorical leaves (mixed kernels, codegen_engine/expressions.py:
    493-516) take no tree parameters: their value is R[l_i, l_j] of the table
    in ``cat_tables`` (one L x L matrix per categorical leaf, tree order), the
    level index read from the leaf's input column.  Continuous leaves without
    active_dims see ``default_dims`` (default: all inputs)."""

    def __init__(self, node: dict, dim: int, cat_tables=None, default_dims=None):
        self.node = node
        self.dim = dim
        self.cat_tables = [np.asarray(t, np.float64) for t in (cat_tables or [])]
        self.default_dims = list(range(dim)) if default_dims is None else list(default_dims)
        self.nparams = self._count(node)

    def _count(self, nd) -> int:
        if nd.get("kernel_type") in CAT_LEAVES:
            return 0
        if nd.get("kernel_type") == "LINEAR":
            return (nd.get("ard_dim") or 1) + 1
        if nd.get("kernel_type") == "POLYNOMIAL":
            return 4 if nd.get("ard_dim") is None else nd["ard_dim"] + 3
        if "kernel_type" in nd:
            extra = 1 if nd["kernel_type"] in (RQ_LEAF, PERIODIC_LEAF) else 0
            return (nd.get("ard_dim") or 1) + extra + 1
        if nd["operator"] == "scale":
            return self._count(nd["left"]) + 1
        return self._count(nd["left"]) + self._count(nd["right"])

    @property
    def nonstationary(self) -> bool:
        """True when a linear or polynomial leaf makes k(x, x) vary with x."""
        def walk(nd):
            if "kernel_type" in nd:
                return nd["kernel_type"] in ("LINEAR", "POLYNOMIAL")
            return walk(nd["left"]) or ("right" in nd and walk(nd["right"]))
        return walk(self.node)

    def matrix(self, X1, X2, params) -> np.ndarray:
        return self._walk(X1, X2, params, False)[0]

    def gradients(self, X1, X2, params) -> np.ndarray:
        """dK/dtheta_p for every tree parameter, shape (P, n1, n2)."""
        return np.stack(self._walk(X1, X2, params, True)[1], axis=0)

    def diag(self, params) -> float:
        z = np.zeros((1, self.dim))
        return float(self.matrix(z, z, params)[0, 0])

    def _walk(self, X1, X2, params, grads):
        X1 = np.atleast_2d(np.asarray(X1, dtype=np.float64))
        X2 = np.atleast_2d(np.asarray(X2, dtype=np.float64))
        p = np.asarray(params, dtype=np.float64)
        if p.shape != (self.nparams,):
            raise ValueError(f"tree expects {self.nparams} parameters, got {p.shape}")
        self._cat_i = 0
        self._cat_d = []
        K, G, _ = self._node(self.node, X1[:, self.default_dims], X2[:, self.default_dims], p, 0,
                             grads, X1, X2)
        return K, G

    def cat_leaf_derivatives(self, X1, X2, params):
        """dK/dv_l per pair for every categorical leaf l (tree order), each
        (n1, n2), with the levels (l_i, l_j) of the leaf's column."""
        X1 = np.atleast_2d(np.asarray(X1, dtype=np.float64))
        X2 = np.atleast_2d(np.asarray(X2, dtype=np.float64))
        self._cat_i = 0
        self._cat_d = []
        _, _, _, D = self._nodeD(self.node, X1[:, self.default_dims], X2[:, self.default_dims],
                                 np.asarray(params, np.float64), 0, X1, X2)
        return [D[k] for k in sorted(D)], self._cat_d

    def _nodeD(self, nd, X1, X2, p, off, F1, F2):
        """(K, None, next_offset, {cat leaf index: dK/dv})."""
        if nd.get("kernel_type") in CAT_LEAVES:
            k = self._cat_i
            self._cat_i += 1
            col = int(nd["active_dims"][0])
            li, lj = F1[:, col].astype(int), F2[:, col].astype(int)
            self._cat_d.append((li, lj))
            K = self.cat_tables[k][li[:, None], lj[None, :]]
            return K, None, off, {k: np.ones_like(K)}
        if nd.get("active_dims") is not None:
            cols = list(nd["active_dims"])
            X1, X2 = F1[:, cols], F2[:, cols]
        if "kernel_type" in nd:
            n = self._count(nd)
            K, _ = _tree_leaf(nd, X1, X2, p[off:off + n], False)
            return K, None, off + n, {}
        A, _, mid, DA = self._nodeD(nd["left"], X1, X2, p, off, F1, F2)
        if nd["operator"] == "scale":
            c = p[mid]
            return c * A, None, mid + 1, {k: c * v for k, v in DA.items()}
        B, _, end, DB = self._nodeD(nd["right"], X1, X2, p, mid, F1, F2)
        if nd["operator"] == "sum":
            return A + B, None, end, {**DA, **DB}
        return (A * B, None, end, {**{k: v * B for k, v in DA.items()},
                                   **{k: A * v for k, v in DB.items()}})

    def _node(self, nd, X1, X2, p, off, grads, F1=None, F2=None):
        if nd.get("kernel_type") in CAT_LEAVES:
            k = self._cat_i
            self._cat_i += 1
            col = int(nd["active_dims"][0])
            li, lj = F1[:, col].astype(int), F2[:, col].astype(int)
            return self.cat_tables[k][li[:, None], lj[None, :]], ([] if grads else None), off
        if nd.get("active_dims") is not None:
            cols = list(nd["active_dims"])
            X1, X2 = F1[:, cols], F2[:, cols]
        if "kernel_type" in nd:
            n = self._count(nd)
            K, G = _tree_leaf(nd, X1, X2, p[off:off + n], grads)
            return K, G, off + n
        A, GA, mid = self._node(nd["left"], X1, X2, p, off, grads, F1, F2)
        if nd["operator"] == "scale":
            c = p[mid]
            return c * A, ([c * g for g in GA] + [A] if grads else None), mid + 1
        B, GB, end = self._node(nd["right"], X1, X2, p, mid, grads, F1, F2)
        if nd["operator"] == "sum":
            return A + B, (GA + GB if grads else None), end
        return A * B, ([g * B for g in GA] + [A * g for g in GB] if grads else None), end


def _tree_leaf(nd, X1, X2, p, grads):
    kt = nd["kernel_type"]
    q = X1.shape[1]
    ard = nd.get("ard_dim") is not None
    if ard and nd["ard_dim"] != q:
        raise ValueError("ARD leaf lengthscale count differs from its dimension count")
    nls = q if ard else 1
    if kt in ("LINEAR", "POLYNOMIAL"):
        # engine layout (kernel.py:462-568, expressions.py:327-421): linear
        # [variance | var_q], os; polynomial [variance | var_q], degree,
        # offset, os with the structural integer degree in the forward
        prod = X1[:, None, :] * X2[None, :, :]
        var = p[:nls]
        dot = (prod * var).sum(-1) if ard else var[0] * prod.sum(-1)
        if kt == "LINEAR":
            os = p[nls]
            k = os * dot
            if not grads:
                return k, None
            G = ([os * prod[:, :, j] for j in range(q)] if ard else [os * prod.sum(-1)])
            return k, G + [dot]
        D = int(round(float((nd.get("initial_values") or {}).get("degree", 2.0))))
        off, os = p[nls + 1], p[nls + 2]
        B = dot + off
        k = os * B**D
        if not grads:
            return k, None
        h = os * D * B ** (D - 1)
        G = ([h * prod[:, :, j] for j in range(q)] if ard else [h * prod.sum(-1)])
        return k, G + [np.zeros_like(k), h, B**D]
    ls = p[:nls] if ard else np.full(q, p[0])
    diff = X1[:, None, :] - X2[None, :, :]
    if kt == PERIODIC_LEAF:
        period, os = p[nls], p[nls + 1]
        ang = np.pi * diff / period
        s2 = np.sin(ang) ** 2
        S = (s2 / ls).sum(-1)
        k = os * _exp_guard(-2.0 * S, False)   # periodic: never clamped
        if not grads:
            return k, None
        G = ([2.0 * k * s2[:, :, j] / ls[j] ** 2 for j in range(q)] if ard
             else [2.0 * k * S / p[0]])
        G.append(4.0 * np.pi * k / period**2 * (np.sin(ang) * np.cos(ang) * diff / ls).sum(-1))
        G.append(k / os)
        return k, G
    d2 = diff**2
    r2 = (d2 / ls**2).sum(-1)
    if kt == RQ_LEAF:
        alpha, os = p[nls], p[nls + 1]
        B = 1.0 + r2 / (2.0 * alpha)
        k = os * B ** (-alpha)
        h = os * B ** (-alpha - 1.0)
        extra = [k * (-np.log(B) + r2 / (2.0 * alpha * B))]
    else:
        kind = _RADIAL_NAMES[kt]
        os = p[nls]
        k = kernel_from_sq(kind, r2, os, ard)
        h = _grad_factor(kind, r2, os, ard, k)
        extra = []
    if not grads:
        return k, None
    terms = d2 / ls**3
    G = [h * terms[:, :, j] for j in range(q)] if ard else [h * terms.sum(-1)]
    return k, G + extra + [k / os]
