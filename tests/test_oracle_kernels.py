"""Pins the float64 kernel oracle (oracle/kernels.py) against independent facts:
the reference's own emitted kernel expressions (where the -20 exp clamp lands,
values and gradients on both sides of it), scikit-learn kernels, SymPy
derivatives and finite differences.  CPU only."""

import json
from pathlib import Path

import numpy as np
import pytest

from oracle import kernels as ok


def _sk_kernel(kind, ls):
    from sklearn.gaussian_process.kernels import RBF, Matern
    if kind == ok.RBF:
        return RBF(length_scale=ls)
    nu = {ok.MATERN12: 0.5, ok.MATERN32: 1.5, ok.MATERN52: 2.5}[kind]
    return Matern(length_scale=ls, nu=nu)


@pytest.mark.parametrize("kind", ok.KINDS)
@pytest.mark.parametrize("ard", [False, True])
def test_matches_sklearn_in_unclamped_region(kind, ard, rng):
    d = 4
    X1 = rng.uniform(-1, 1, size=(30, d))
    X2 = rng.uniform(-1, 1, size=(25, d))
    ls = rng.uniform(0.5, 2.0, size=d) if ard else np.array([0.9])
    os = 1.7
    params = np.concatenate([ls, [os]])
    K = ok.kernel_matrix(kind, X1, X2, params, ard)
    sk = _sk_kernel(kind, ls if ard else float(ls[0]))(X1, X2) * os
    np.testing.assert_allclose(K, sk, rtol=1e-10, atol=1e-13)


# ---------------------------------------------------------------------------
# The reference's own post-pass expressions (tests/golden/gen_kernel_exprs.py
# ran its code generator: KernelExprBuilder -> gradients -> to_ir -> optimize,
# codegen_engine/__init__.py:176-236) and their float64 values at point pairs
# whose exponents fall on both sides of -20.
# ---------------------------------------------------------------------------
GOLDEN = Path(__file__).parent / "golden"
_LEAF = {"rbf": ok.RBF, "matern12": ok.MATERN12, "matern32": ok.MATERN32,
         "matern52": ok.MATERN52}


@pytest.fixture(scope="module")
def exprs():
    meta = json.loads((GOLDEN / "ref_kernel_exprs.json").read_text())
    arrays = np.load(GOLDEN / "ref_kernel_exprs.npz")
    return meta, arrays


def _radial_cases(meta):
    out = []
    for key in sorted(meta):
        fam, tag, _ = key.split("_") if key.count("_") == 2 else (None, None, None)
        if fam in _LEAF:
            out.append((key, _LEAF[fam], tag == "ard"))
    return out


def test_fixture_covers_every_radial_kind_iso_ard_and_dimension(exprs):
    meta, _ = exprs
    cases = _radial_cases(meta)
    assert {(k, a) for _, k, a in cases} == {(k, a) for k in ok.KINDS for a in (False, True)}
    assert {meta[key]["dim"] for key, _, _ in cases} == {1, 4, 8, 16}


def test_clamp_placement_matches_reference_codegen(exprs):
    """exp_clamped(kind, ard) is what the reference's stability pass emitted
    for every radial leaf, iso and ARD, d in {1, 4, 8, 16}."""
    meta, _ = exprs
    for key, kind, ard in _radial_cases(meta):
        assert meta[key]["exp_clamped"] == [ok.exp_clamped(kind, ard)], key
    # RBF is never clamped, Matern-1/2 only for ARD: the distinction is real
    assert meta["rbf_ard_d16"]["exp_clamped"] == [False]
    assert meta["matern12_iso_d4"]["exp_clamped"] == [False]
    assert meta["matern12_ard_d4"]["exp_clamped"] == [True]
    assert meta["matern52_ard_d16"]["exp_clamped"] == [True]
    for key in ("periodic_iso_d1", "periodic_ard_d4", "product_rbf_periodic_d2"):
        assert not any(meta[key]["exp_clamped"]), key


def test_radial_values_and_gradients_match_reference_expressions(exprs):
    """Oracle K and dK/dtheta at the fixture pairs equal the reference's
    emitted expressions in float64 -- including far pairs where a wrongly
    placed clamp would give os e^-20 instead of the true tail."""
    meta, A = exprs
    far_seen = 0
    for key, kind, ard in _radial_cases(meta):
        p = A[f"{key}__params"]
        X1, X2 = A[f"{key}__x1"], A[f"{key}__x2"]
        want_k, want_g = A[f"{key}__k"], A[f"{key}__grad"]
        K = np.array([ok.kernel_matrix(kind, X1[i:i + 1], X2[i:i + 1], p, ard)[0, 0]
                      for i in range(X1.shape[0])])
        np.testing.assert_allclose(K, want_k, rtol=1e-12, atol=1e-300, err_msg=key)
        G = np.stack([ok.kernel_gradients(kind, X1[i:i + 1], X2[i:i + 1], p, ard)[:, 0, 0]
                      for i in range(X1.shape[0])], axis=1)
        # atol: the isotropic Matern-1/2 gradient at a coincident pair is
        # os 1e-10 / l^2 in the reference (r floored before the 1/l scale)
        np.testing.assert_allclose(G, want_g, rtol=1e-8, atol=1e-9, err_msg=key)
        far_seen += int(np.sum((want_k > 0) & (want_k < p[-1] * np.exp(-20.0))))
    assert far_seen > 50  # unclamped tails below os e^-20 are exercised


def _tree_params(meta, key, p):
    """Fixture parameters (the generated code's order) in the engine layout:
    a scale node's factor moves from before its subtree to after it."""
    names = meta[key]["param_names"]
    if names and names[0] == "scale":
        return np.concatenate([p[1:], p[:1]])
    return p


@pytest.mark.parametrize("key", [
    "periodic_iso_d1", "periodic_iso_d4", "periodic_ard_d1", "periodic_ard_d4",
    "rq_iso_d1", "rq_iso_d4", "rq_ard_d1", "rq_ard_d4",
    "linear_iso_d1", "linear_iso_d4", "linear_ard_d1", "linear_ard_d4",
    "polynomial_iso_d4", "sum_rbf_matern52_d4", "product_rbf_periodic_d2",
    "product_matern12_matern32ard_d3", "scale_rbf_d2", "product_sum_m12ard_rbf_matern52_d4"])
def test_tree_values_and_gradients_match_reference_expressions(exprs, key):
    meta, A = exprs
    tk = ok.TreeKernel(meta[key]["kernel"], meta[key]["dim"])
    p = A[f"{key}__params"]
    pe = _tree_params(meta, key, p)
    X1, X2 = A[f"{key}__x1"], A[f"{key}__x2"]
    K = np.array([tk.matrix(X1[i:i + 1], X2[i:i + 1], pe)[0, 0] for i in range(X1.shape[0])])
    np.testing.assert_allclose(K, A[f"{key}__k"], rtol=1e-11, atol=1e-300)
    G = np.stack([tk.gradients(X1[i:i + 1], X2[i:i + 1], pe)[:, 0, 0]
                  for i in range(X1.shape[0])], axis=1)
    want = A[f"{key}__grad"]
    if meta[key]["param_names"][0] == "scale":
        want = np.concatenate([want[1:], want[:1]])
    np.testing.assert_allclose(G, want, rtol=1e-8, atol=1e-9)


@pytest.mark.parametrize("kind", ok.KINDS)
def test_diagonal_is_outputscale(kind, rng):
    X = rng.normal(size=(10, 3))
    K = ok.kernel_matrix(kind, X, X, [0.7, 0.3, 1.1, 2.0], True)
    np.testing.assert_allclose(np.diag(K), 2.0, rtol=1e-9)


@pytest.mark.parametrize("kind", ok.KINDS)
@pytest.mark.parametrize("ard", [False, True])
def test_gradients_match_finite_differences(kind, ard, rng):
    d = 3
    X1 = rng.uniform(-1, 1, size=(8, d))
    X2 = rng.uniform(-1, 1, size=(7, d))
    params = np.concatenate([rng.uniform(0.6, 1.5, size=d if ard else 1), [1.3]])
    G = ok.kernel_gradients(kind, X1, X2, params, ard)
    assert G.shape == (params.size, 8, 7)
    h = 1e-6
    for p in range(params.size):
        up = params.copy(); up[p] += h
        dn = params.copy(); dn[p] -= h
        fd = (ok.kernel_matrix(kind, X1, X2, up, ard) - ok.kernel_matrix(kind, X1, X2, dn, ard)) / (2 * h)
        np.testing.assert_allclose(G[p], fd, rtol=1e-6, atol=1e-9)


def test_matern_gradient_matches_sympy():
    sp = pytest.importorskip("sympy")
    l0, l1, os, a0, a1 = sp.symbols("l0 l1 os a0 a1", positive=True)
    r = sp.sqrt((a0 / l0) ** 2 + (a1 / l1) ** 2)
    k = os * (1 + sp.sqrt(5) * r + sp.Rational(5, 3) * r**2) * sp.exp(-sp.sqrt(5) * r)
    vals = {l0: 0.8, l1: 1.3, os: 1.7, a0: 0.4, a1: -0.9}
    X1 = np.array([[0.4, -0.9]])
    X2 = np.zeros((1, 2))
    G = ok.kernel_gradients(ok.MATERN52, X1, X2, [0.8, 1.3, 1.7], True)
    for p, sym in enumerate([l0, l1, os]):
        ref = float(sp.diff(k, sym).subs(vals))
        assert G[p, 0, 0] == pytest.approx(ref, rel=1e-12)


@pytest.mark.parametrize("kind,nu_k", [(ok.MATERN12, "exp"), (ok.MATERN32, "m32")])
def test_low_order_matern_gradient_matches_sympy(kind, nu_k):
    """Matern-1/2 and 3/2 lengthscale derivatives of the forward expressions
    with the reference's r = sqrt(sum (a/l)^2 + 1e-20), as SymPy gives them."""
    sp = pytest.importorskip("sympy")
    l0, l1, os, a0, a1 = sp.symbols("l0 l1 os a0 a1", positive=True)
    r = sp.sqrt((a0 / l0) ** 2 + (a1 / l1) ** 2 + sp.Float(1e-20))
    if nu_k == "exp":
        k = os * sp.exp(-r)
    else:
        k = os * (1 + sp.sqrt(3) * r) * sp.exp(-sp.sqrt(3) * r)
    vals = {l0: 0.8, l1: 1.3, os: 1.7, a0: 0.4, a1: -0.9}
    G = ok.kernel_gradients(kind, np.array([[0.4, -0.9]]), np.zeros((1, 2)), [0.8, 1.3, 1.7], True)
    for p, sym in enumerate([l0, l1, os]):
        assert G[p, 0, 0] == pytest.approx(float(sp.diff(k, sym).subs(vals)), rel=1e-12)
    # coincident points: finite (the floored r), zero lengthscale derivative
    G0 = ok.kernel_gradients(kind, np.zeros((1, 2)), np.zeros((1, 2)), [0.8, 1.3, 1.7], True)
    assert np.all(np.isfinite(G0)) and G0[0, 0, 0] == 0.0
    assert G0[2, 0, 0] == pytest.approx(1.0, abs=1e-9)


def test_forward_matvec_matches_dense(rng):
    X = rng.normal(size=(60, 5))
    V = rng.normal(size=(3, 60))
    params = [0.9, 1.1, 0.8, 1.2, 1.0, 1.4]
    K = ok.kernel_matrix(ok.MATERN52, X, X, params, True)
    out = ok.forward_matvec(ok.MATERN52, X, V, params, 0.05, True, block=17)
    np.testing.assert_allclose(out, V @ K.T + 0.05 * V, rtol=1e-12)
    rows = np.array([3, 17, 59])
    part = ok.forward_matvec(ok.MATERN52, X, V, params, 0.05, True, rows=rows)
    np.testing.assert_allclose(part, out[:, rows], rtol=1e-12)


def test_gradient_matvec_layout(rng):
    X = rng.normal(size=(12, 2))
    V = rng.normal(size=(2, 12))
    params = [0.9, 1.2, 1.5]
    G = ok.kernel_gradients(ok.RBF, X, X, params, True)
    out = ok.gradient_matvec(ok.RBF, X, V, params, True)
    for p in range(3):
        np.testing.assert_allclose(out[p], V @ G[p].T, rtol=1e-12)
