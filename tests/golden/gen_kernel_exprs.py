"""Writes tests/golden/ref_kernel_exprs.json and ref_kernel_exprs.npz: the
post-pass kernel expressions the reference's code generator emits, and their
float64 values at chosen point pairs.  Run in the build container only.

For each kernel tree and input dimension the script runs the reference's own
pipeline up to the emitter (mojogp/codegen_engine/__init__.py:176-236):
KernelExprBuilder.from_kernel_node (expressions.py:474-650), the gradient
overrides and SymPy differentiation (overrides.py, differentiation.py), to_ir
(ir.py:213-252) and optimize (passes/__init__.py:14-35: cse, inv_ls, strength,
forward_hoist, gradient_sharing, dead_code, numerical_stability, simplify).
It records

* the let bindings, forward and gradient expressions as the emitter prints
  them (emit/mojo_printer.py:emit_ir);
* for every exp() in the lets / forward / gradients, whether the numerical
  stability pass wrapped its argument in max(., -20)
  (passes/numerical_stability.py:29-41,62-85);
* the forward value and every gradient at point pairs chosen so that the
  exponent of each radial or periodic leaf falls on both sides of -20,
  evaluated in float64 by the small IR evaluator below (this file's own code:
  the variables are bound as the emitter binds them, emit/gpu_kernel.py:18-52:
  diff_d = x_row_d - x_col_d, dist_sq = sum_d diff_d^2,
  dot_prod = sum_d x_row_d x_col_d).

The parameter vector of each case is in the generated code's own order
(the IR's Param indices).  For ``scale`` nodes the generator reads the scale
factor at the subtree's first index (expressions.py:642-648) while the
engine layout puts it after the subtree (kernel.py:561-566); the fixture keeps
the generator's order and the tests permute.
"""

import json
import sys
from pathlib import Path

import numpy as np

REF = "/root/reference"
HERE = Path(__file__).parent


def _tree(e, ir):
    """IR node -> nested list (JSON)."""
    if isinstance(e, ir.Var):
        return ["var", e.name]
    if isinstance(e, ir.Param):
        return ["param", e.index]
    if isinstance(e, ir.Const):
        return ["const", e.value]
    if isinstance(e, ir.BinOp):
        return [e.op, _tree(e.left, ir), _tree(e.right, ir)]
    if isinstance(e, ir.UnaryFn):
        return [e.fn, _tree(e.arg, ir)]
    if isinstance(e, ir.Pow):
        return ["pow", _tree(e.base, ir), _tree(e.exp, ir)]
    if isinstance(e, ir.MaxExpr):
        return ["max", _tree(e.left, ir), _tree(e.right, ir)]
    raise TypeError(type(e))


def _exps(t, out):
    """Collect (clamped, argument) for every exp node of a nested-list tree."""
    if not isinstance(t, list) or t[0] in ("var", "param", "const"):
        return
    if t[0] == "exp":
        a = t[1]
        clamped = a[0] == "max" and a[2] == ["const", -20.0]
        out.append(clamped)
    for c in t[1:]:
        _exps(c, out)


def _eval(t, env, p):
    """float64 value of a nested-list IR tree over arrays of pairs."""
    op = t[0]
    if op == "var":
        return env[t[1]]
    if op == "param":
        return p[t[1]]
    if op == "const":
        return np.float64(t[1])
    if op in ("+", "-", "*", "/"):
        a, b = _eval(t[1], env, p), _eval(t[2], env, p)
        with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
            return {"+": a + b, "-": a - b, "*": a * b, "/": a / b}[op]
    if op == "max":
        return np.maximum(_eval(t[1], env, p), _eval(t[2], env, p))
    if op == "pow":
        return np.power(_eval(t[1], env, p), _eval(t[2], env, p))
    fn = {"exp": np.exp, "sqrt": np.sqrt, "sin": np.sin, "cos": np.cos,
          "log": np.log, "abs": np.abs}[op]
    with np.errstate(over="ignore", under="ignore", invalid="ignore", divide="ignore"):
        return fn(_eval(t[1], env, p))


def _bind(X1, X2, lets, p):
    d = X1.shape[1]
    env = {}
    diff = X1 - X2
    for k in range(d):
        env[f"diff_{k}"] = diff[:, k]
        env[f"x_row_{k}"] = X1[:, k]
        env[f"x_col_{k}"] = X2[:, k]
    env["dist_sq"] = (diff * diff).sum(1)
    env["dot_prod"] = (X1 * X2).sum(1)
    for name, t in lets:
        env[name] = _eval(t, env, p)
    return env


# Parameter values by the IR's parameter names (lengthscales per dimension
# spread around the base value).
def _params(names, d, base_ls):
    p = []
    for i, nm in enumerate(names):
        if nm == "ls":
            p.append(base_ls)
        elif nm.startswith("l_"):
            k = int(nm[2:])
            p.append(base_ls * (0.7 + 0.6 * k / max(d - 1, 1)))
        elif nm == "os":
            p.append(1.3 + 0.1 * i)
        elif nm == "period":
            p.append(1.7)
        elif nm == "alpha":
            p.append(0.8)
        elif nm == "scale":
            p.append(2.0)
        elif nm in ("variance",) or nm.startswith("var_"):
            p.append(0.6)
        elif nm == "degree":
            p.append(2.0)
        elif nm == "offset":
            p.append(0.5)
        else:
            raise ValueError(nm)
    return np.array(p, np.float64)


def _pairs(rng, d, names, p):
    """Point pairs at scaled distances from 0 to 40 lengthscales along random
    directions: the exponents of RBF (-r^2/2), Matern (-sqrt(nu') r) and the
    periodic leaf cross -20 inside this range."""
    ls = np.ones(d)
    for i, nm in enumerate(names):
        if nm == "ls":
            ls[:] = p[i]
            break
        if nm.startswith("l_"):
            ls[int(nm[2:])] = p[i]
    radii = np.concatenate([[0.0, 1e-6, 0.3, 1.0, 2.5], np.linspace(5.0, 7.5, 11),
                            np.linspace(8.0, 12.5, 10), [15.0, 19.5, 20.5, 25.0, 40.0]])
    X1 = rng.normal(size=(radii.size, d))
    u = rng.normal(size=(radii.size, d))
    u /= np.linalg.norm(u, axis=1, keepdims=True)
    X2 = X1 + radii[:, None] * u * ls
    return X1, X2


def main() -> None:
    sys.path.insert(0, REF)
    from mojogp.codegen_engine import _resolve_ard
    from mojogp.codegen_engine import ir as rir
    from mojogp.codegen_engine.differentiation import compute_gradients
    from mojogp.codegen_engine.emit.mojo_printer import emit_ir
    from mojogp.codegen_engine.expressions import KernelExprBuilder
    from mojogp.codegen_engine.overrides import get_overrides_for_kernel
    from mojogp.codegen_engine.passes import optimize
    from mojogp.kernel import Kernel

    K = Kernel
    cases = []
    for fam in ("rbf", "matern12", "matern32", "matern52"):
        for ard in (False, True):
            for d in (1, 4, 8, 16):
                cases.append((f"{fam}_{'ard' if ard else 'iso'}_d{d}",
                              getattr(K, fam)(ard=ard), d, 1.0))
    for ard in (False, True):
        for d in (1, 4):
            tag = "ard" if ard else "iso"
            # small lengthscales put -2 S below -20 for part of the pairs
            cases.append((f"periodic_{tag}_d{d}", K.periodic(ard=ard), d, 0.05))
            cases.append((f"rq_{tag}_d{d}", K.rq(ard=ard), d, 1.0))
            cases.append((f"linear_{tag}_d{d}", K.linear(ard=ard), d, 1.0))
    cases.append(("polynomial_iso_d4", K.polynomial(), 4, 1.0))
    cases.append(("sum_rbf_matern52_d4", K.rbf() + K.matern52(), 4, 1.0))
    cases.append(("product_rbf_periodic_d2", K.rbf() * K.periodic(), 2, 1.0))
    cases.append(("product_matern12_matern32ard_d3", K.matern12() * K.matern32(ard=True), 3, 1.0))
    cases.append(("scale_rbf_d2", 2.0 * K.rbf(), 2, 1.0))
    cases.append(("product_sum_m12ard_rbf_matern52_d4",
                  (K.matern12(ard=True) + K.rbf()) * K.matern52(), 4, 1.0))

    rng = np.random.default_rng(11)
    meta, arrays = {}, {}
    for key, kern, d, base_ls in cases:
        kern = _resolve_ard(kern, d)
        ke = KernelExprBuilder(d).from_kernel_node(kern)
        ge = compute_gradients(ke, get_overrides_for_kernel(ke))
        irk = rir.to_ir(ge, d, needs_diffs=ke.needs_diffs, needs_dist_sq=ke.needs_dist_sq,
                        needs_dot=ke.needs_dot)
        irk = optimize(irk)
        lets = [(lb.name, _tree(lb.value, rir)) for lb in irk.lets]
        fwd = _tree(irk.forward, rir)
        grads = [_tree(irk.gradients[i], rir) for i in range(irk.num_params)]
        clamps = []
        for _, t in lets:
            _exps(t, clamps)
        _exps(fwd, clamps)
        for g in grads:
            _exps(g, clamps)
        p = _params(irk.param_names, d, base_ls)
        X1, X2 = _pairs(rng, d, irk.param_names, p)
        env = _bind(X1, X2, lets, p)
        F = np.broadcast_to(_eval(fwd, env, p), (X1.shape[0],)).astype(np.float64)
        G = np.stack([np.broadcast_to(_eval(g, env, p), (X1.shape[0],)) for g in grads])
        meta[key] = {
            "dim": d,
            "kernel": kern.to_dict(),
            "param_names": list(irk.param_names),
            "exp_clamped": clamps,
            "lets": [[n, emit_ir(lb.value)] for n, lb in zip([lb.name for lb in irk.lets], irk.lets)],
            "forward": emit_ir(irk.forward),
            "gradients": [emit_ir(irk.gradients[i]) for i in range(irk.num_params)],
        }
        arrays[f"{key}__params"] = p
        arrays[f"{key}__x1"] = X1
        arrays[f"{key}__x2"] = X2
        arrays[f"{key}__k"] = F
        arrays[f"{key}__grad"] = G
    (HERE / "ref_kernel_exprs.json").write_text(json.dumps(meta, indent=1, sort_keys=True) + "\n")
    np.savez_compressed(HERE / "ref_kernel_exprs.npz", **arrays)
    for key in meta:
        print(f"{key:40s} exp clamped: {meta[key]['exp_clamped']}")


if __name__ == "__main__":
    main()
