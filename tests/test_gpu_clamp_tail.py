"""Device products at pairs beyond the reference's -20 exp clamp.

The reference's generated code clamps exp(x) at -20 only where its stability
pass recognises a negative exponent (passes/numerical_stability.py:62-85):
Matern-3/2, Matern-5/2 and ARD Matern-1/2 leaves are clamped; RBF, isotropic
Matern-1/2 and periodic leaves are not (tests/golden/ref_kernel_exprs.json,
pinned against the oracle in tests/test_oracle_kernels.py).

Two tight clusters A and B sit a distance D apart that puts the unclamped
exponent at -23.  With V = 0 on A and positive on B, the rows of A see only
cross-cluster pairs: their outputs are pure tail sums, n_B k(D) ~ e^-23 without
the clamp and the e^-20 floor with it -- a factor e^3 ~ 20 apart.  Every device
route (one-sided and symmetric tiles, direct pair loop, cross product, dense
fp16-split product, gradient products, compiled kernel trees) must put those
rows within 5% of the oracle (the fp16-split routes carry such values in fp16's
subnormal range: absolute error <= 2^-40 os per pair) and the whole columns
within the 1e-5 bar."""

import numpy as np
import pytest

from mojogp_amd import Matern12, Matern32, Matern52, RBF, make_ard_kernel
from mojogp_amd._provider import NativeProvider
from oracle import kernels as ok

pytestmark = pytest.mark.gpu

TAIL_EXP = 23.0
# |exponent| per unit scaled distance r: RBF 0.5 r^2, Matern-nu sqrt(2 nu) r
_DIST = {ok.RBF: np.sqrt(2.0 * TAIL_EXP), ok.MATERN12: TAIL_EXP,
         ok.MATERN32: TAIL_EXP / np.sqrt(3.0), ok.MATERN52: TAIL_EXP / np.sqrt(5.0)}
CASES = [(ok.RBF, False), (ok.RBF, True), (ok.MATERN12, False), (ok.MATERN12, True),
         (ok.MATERN32, True), (ok.MATERN52, False), (ok.MATERN52, True)]
_LEAF = {ok.RBF: RBF, ok.MATERN12: Matern12, ok.MATERN32: Matern32, ok.MATERN52: Matern52}


def _rel(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def _clusters(kind, ard, nA=1024, nB=1024, d=3, seed=0):
    rng = np.random.default_rng(seed + 10 * kind + int(ard))
    ls = np.array([0.8, 1.0, 1.25]) if ard else np.full(d, 1.0)
    u = rng.normal(size=d)
    u /= np.linalg.norm(u)
    XA = rng.uniform(-0.01, 0.01, size=(nA, d)) * ls
    XB = _DIST[kind] * u * ls + rng.uniform(-0.01, 0.01, size=(nB, d)) * ls
    X = np.concatenate([XA, XB]).astype(np.float32)
    params = np.concatenate([ls if ard else ls[:1], [1.3]]).astype(np.float32)
    V = np.zeros((2, nA + nB), np.float32)
    V[0, nA:] = 1.0
    V[1, nA:] = rng.uniform(0.5, 1.5, size=nB)
    return X, params, V, nA


def _check(name, got, ref, wrong, nA):
    tail, tail_ref, tail_wrong = got[:, :nA], ref[:, :nA], wrong[:, :nA]
    e_tail, e_full = _rel(tail, tail_ref), _rel(got, ref)
    sep = _rel(tail_wrong, tail_ref)
    print(f"  {name}: tail rows {e_tail:.2e} (other placement {sep:.2e}), columns {e_full:.2e}",
          flush=True)
    assert sep > 0.9                      # the placement is what the tail rows measure
    assert e_tail <= 0.05
    if got.shape[1] > nA:                 # columns that hold more than tail rows
        assert e_full <= 1e-5


def _oracles(kind, ard, X, V, params, noise):
    ref = ok.forward_matvec(kind, X, V, params, noise, ard)
    flip = ok.exp_clamped
    try:   # the other placement: clamped where the reference is not and vice versa
        ok.exp_clamped = lambda k, a: not flip(k, a)
        wrong = ok.forward_matvec(kind, X, V, params, noise, ard)
    finally:
        ok.exp_clamped = flip
    return ref, wrong


@pytest.mark.parametrize("kind,ard", CASES)
def test_tail_rows_follow_reference_clamp_placement(monkeypatch, kind, ard):
    X, params, V, nA = _clusters(kind, ard)
    noise = 0.05
    print(f"clamp tail kind={kind} ard={ard} n={X.shape[0]}", flush=True)
    ref, wrong = _oracles(kind, ard, X, V, params, noise)
    p = NativeProvider(kind, ard, X, params, noise)
    try:
        monkeypatch.setenv("MGP_SYM_MATVEC", "0")
        one_sided = p.forward_matvec(V)
        monkeypatch.setenv("MGP_SYM_MATVEC", "1")
        sym = p.forward_matvec(V)
        monkeypatch.delenv("MGP_SYM_MATVEC")
        direct = p.direct_matvec(V)
        cross = p.cross_matvec(X[:nA], V)
        grad = p.gradient_matvec(V)
        p.materialize()
        dense = p.forward_matvec(V)
    finally:
        p.close()
    for name, got in (("one-sided", one_sided), ("symmetric", sym), ("direct", direct),
                      ("dense", dense)):
        _check(name, got, ref, wrong, nA)
    # cross product K(X_A, X) V: the noise term does not apply
    refx = ref[:, :nA] - noise * V[:, :nA]
    wrongx = wrong[:, :nA] - noise * V[:, :nA]
    _check("cross", cross, refx, wrongx, nA)
    # gradient products: every parameter's tail rows.  (Their cluster-B rows
    # weigh pairs 0.01 lengthscales apart on coordinates ~5 lengthscales from
    # the centre, where fp32 coordinate differences -- in the reference's
    # kernels as here -- carry ~1e-5 relative error; column parity of the
    # gradient products is tested on ordinary data in test_gpu_matvec.py.)
    refg = ok.gradient_matvec(kind, X, V, params, ard)
    for q in range(refg.shape[0]):
        e_tail = _rel(grad[q][:, :nA], refg[q][:, :nA])
        print(f"  gradient p{q}: tail rows {e_tail:.2e}", flush=True)
        assert e_tail <= 0.05


@pytest.mark.parametrize("kind,ard", [(ok.RBF, False), (ok.MATERN12, False),
                                      (ok.MATERN12, True), (ok.MATERN52, True)])
def test_tree_leaf_tail_rows_follow_reference_clamp_placement(kind, ard):
    """The same tail rows through the compiled kernel-tree products (a scaled
    leaf) and their dense fill."""
    X, params, V, nA = _clusters(kind, ard, nA=512, nB=512)
    node = 2.0 * _LEAF[kind](ard=ard)
    if ard:
        node = make_ard_kernel(node, X.shape[1])
    T = ok.TreeKernel(node.to_dict(), X.shape[1])
    tp = np.concatenate([params, [2.0]]).astype(np.float32)   # scale after its subtree
    noise = 0.05
    ref = ok.forward_matvec(T, X, V, tp, noise, False)
    print(f"tree clamp tail kind={kind} ard={ard}", flush=True)
    p = NativeProvider(None, False, X, tp, noise, tree_spec=node.to_tree_spec(X.shape[1]))
    try:
        fwd = p.forward_matvec(V)
        p.materialize()
        dense = p.forward_matvec(V)
    finally:
        p.close()
    for name, got in (("tree", fwd), ("tree dense", dense)):
        e_tail, e_full = _rel(got[:, :nA], ref[:, :nA]), _rel(got, ref)
        print(f"  {name}: tail rows {e_tail:.2e}, columns {e_full:.2e}", flush=True)
        assert e_tail <= 0.05 and e_full <= 1e-5
