"""Parity of the gfx950 kernel products with the float64 oracle.

Bar (north star): norm-wise relative error <= 1e-5 per right-hand side,
against oracle/kernels.py which restates the reference arithmetic
(codegen_engine/expressions.py + passes/numerical_stability.py)."""

import math

import numpy as np
import pytest

from mojogp_amd._provider import NativeProvider
from oracle import kernels as ok

pytestmark = pytest.mark.gpu

TOL = 1e-5


def _relerr(got, ref):
    got = np.atleast_2d(np.asarray(got, dtype=np.float64))
    ref = np.atleast_2d(ref)
    num = np.linalg.norm(got - ref, axis=1)
    den = np.maximum(np.linalg.norm(ref, axis=1), 1e-30)
    return float(np.max(num / den))


def _params(rng, d, ard, lo=0.6, hi=1.6, os=1.3):
    ls = rng.uniform(lo, hi, size=d if ard else 1)
    return np.concatenate([ls, [os]]).astype(np.float32)


CASES = [
    # kind, ard, d, n, t
    (ok.RBF, False, 1, 2000, 11),
    (ok.RBF, True, 8, 3000, 16),
    (ok.MATERN52, True, 16, 2500, 16),
    (ok.MATERN52, False, 4, 1000, 1),
    (ok.RBF, True, 6, 777, 40),
    (ok.MATERN52, True, 3, 129, 3),
    (ok.RBF, False, 2, 17, 2),
    (ok.MATERN52, True, 30, 600, 5),
    (ok.RBF, True, 5, 1, 1),
]


@pytest.mark.parametrize("kind,ard,d,n,t", CASES)
def test_forward_matvec_parity(kind, ard, d, n, t):
    rng = np.random.default_rng(1000 + 7 * d + n)
    print(f"forward case kind={kind} ard={ard} d={d} n={n} t={t}", flush=True)
    X = rng.normal(size=(n, d)).astype(np.float32)
    V = rng.normal(size=(t, n)).astype(np.float32)
    params = _params(rng, d, ard)
    noise = 0.05
    ref = ok.forward_matvec(kind, X, V, params, noise, ard)
    with_p = NativeProvider(kind, ard, X, params, noise)
    try:
        got = with_p.forward_matvec(V)
        direct = with_p.direct_matvec(V)
    finally:
        with_p.close()
    assert got.shape == V.shape
    assert np.all(np.isfinite(got))
    assert _relerr(got, ref) <= TOL
    assert _relerr(direct, ref) <= TOL


@pytest.mark.parametrize("kind,ard,d", [(ok.RBF, True, 8), (ok.MATERN52, True, 16), (ok.RBF, False, 1)])
@pytest.mark.parametrize("t", [1, 16, 70])
def test_cross_matvec_parity(kind, ard, d, t):
    rng = np.random.default_rng(77 + d + t)
    n, m = 1500, 333
    print(f"cross case kind={kind} d={d} t={t}", flush=True)
    X = rng.uniform(-2, 2, size=(n, d)).astype(np.float32)
    Xs = rng.uniform(-2.5, 2.5, size=(m, d)).astype(np.float32)
    V = rng.normal(size=(t, n)).astype(np.float32)
    params = _params(rng, d, ard)
    ref = ok.cross_matvec(kind, Xs, X, V, params, ard)
    p = NativeProvider(kind, ard, X, params, 0.1)
    try:
        got = p.cross_matvec(Xs, V)
    finally:
        p.close()
    assert got.shape == (t, m)
    assert _relerr(got, ref) <= TOL


def test_short_lengthscale_and_update_params():
    """Gram-form cancellation stress: short lengthscales inflate |z|^2."""
    rng = np.random.default_rng(5)
    n, d, t = 2048, 16, 16
    X = rng.normal(size=(n, d)).astype(np.float32)
    V = rng.normal(size=(t, n)).astype(np.float32)
    p = NativeProvider(ok.MATERN52, True, X, _params(rng, d, True), 0.01)
    try:
        for lo, hi in [(0.25, 0.4), (2.0, 5.0), (0.6, 1.6)]:
            params = _params(rng, d, True, lo, hi, os=0.8)
            p.update_params(params)
            p.update_noise(0.02)
            ref = ok.forward_matvec(ok.MATERN52, X, V, params, 0.02, True)
            got = p.forward_matvec(V)
            print(f"ls range ({lo},{hi}) relerr {_relerr(got, ref):.3e}", flush=True)
            assert _relerr(got, ref) <= TOL
    finally:
        p.close()


@pytest.mark.parametrize("kind", [ok.RBF, ok.MATERN52])
def test_spread_far_beyond_lengthscale(kind):
    """Data spread of ~40 lengthscales: |z|^2 reaches ~1e5, where the Gram-form
    distance error (~2^-23 |z|^2) would exceed the bar; the provider must route
    the product through per-dimension differences and stay within it, for the
    training product and for the cross product."""
    rng = np.random.default_rng(11)
    n, m, d, t = 4000, 300, 2, 16
    X = rng.normal(size=(n, d)).astype(np.float32)
    Xs = rng.normal(size=(m, d)).astype(np.float32)
    V = rng.normal(size=(t, n)).astype(np.float32)
    params = np.array([0.05, 0.07, 1.3], dtype=np.float32)
    ref = ok.forward_matvec(kind, X, V, params, 0.05, True)
    refx = ok.cross_matvec(kind, Xs, X, V, params, True)
    p = NativeProvider(kind, True, X, params, 0.05)
    try:
        got = p.forward_matvec(V)
        gotx = p.cross_matvec(Xs, V)
    finally:
        p.close()
    print(f"spread/ls ~40: forward relerr {_relerr(got, ref):.3e}, "
          f"cross relerr {_relerr(gotx, refx):.3e}", flush=True)
    assert _relerr(got, ref) <= TOL
    assert _relerr(gotx, refx) <= TOL


# Gram-form bound on max|z_rows|^2 + max|z_cols|^2 per kernel and the base-2
# coordinate scale (z = (x - mean) * scale / lengthscale).
_GRAM_BOUND = {ok.RBF: (128.0, 0.84932180028801904272),
               ok.MATERN32: (512.0, 2.49882111064734320000),
               ok.MATERN52: (2048.0, 3.22596433305849393025)}


@pytest.mark.parametrize("kind", [ok.RBF, ok.MATERN32, ok.MATERN52])
@pytest.mark.parametrize("side", [0.95, 1.05])
def test_gram_routing_boundary(kind, side):
    """Points on an annulus whose outer radius puts max|z|^2 + max|z|^2 at
    side^2 x the kernel's Gram-form bound (X symmetric, so the centre is 0).
    Just below the bound the tile kernel runs (its output is not bit-equal to
    the difference path); just above, the product is the difference path's
    bit for bit.  Both sides, and the cross product from test points on the
    same annulus, stay within the product bar of the float64 oracle, with
    near-coincident pairs at the largest norms."""
    bound, scale = _GRAM_BOUND[kind]
    ls, n2, m, t = 0.1, 1500, 200, 16
    r_out = side * math.sqrt(bound / 2.0) * ls / scale
    rng = np.random.default_rng(17 + int(100 * side) + kind)

    def annulus(k):
        rad = np.sqrt(rng.uniform((0.7 * r_out) ** 2, r_out ** 2, size=k))
        ang = rng.uniform(0, 2 * np.pi, size=k)
        return np.stack([rad * np.cos(ang), rad * np.sin(ang)], 1)

    P = annulus(n2)
    P[0] = [r_out, 0.0]
    X = np.concatenate([P, -P]).astype(np.float32)
    Xs = annulus(m).astype(np.float32)
    n = X.shape[0]
    V = rng.normal(size=(t, n)).astype(np.float32)
    params = np.array([ls, 1.3], dtype=np.float32)
    print(f"gram boundary kind={kind} side={side} r_out={r_out:.4f}", flush=True)
    p = NativeProvider(kind, False, X, params, 0.05)
    try:
        got = p.forward_matvec(V)
        direct = p.direct_matvec(V)
        gotx = p.cross_matvec(Xs, V)
    finally:
        p.close()
    ref = ok.forward_matvec(kind, X, V, params, 0.05, False)
    refx = ok.cross_matvec(kind, Xs, X, V, params, False)
    e, ex = _relerr(got, ref), _relerr(gotx, refx)
    print(f"  forward relerr {e:.3e} cross relerr {ex:.3e} "
          f"bit-equal to difference path {np.array_equal(got, direct)}", flush=True)
    if side < 1.0:
        assert not np.array_equal(got, direct)
    else:
        assert np.array_equal(got, direct)
    assert e <= TOL
    assert ex <= TOL


@pytest.mark.parametrize("kind,ard,d,n,t", [(ok.RBF, False, 4, 3000, 16),
                                            (ok.MATERN52, True, 3, 2048, 1),
                                            (ok.RBF, True, 2, 1500, 40),
                                            (ok.MATERN32, False, 5, 1001, 130)])
def test_materialized_route_parity(kind, ard, d, n, t):
    """Dense K filled on the device and stored as a two-term fp16 split, products
    on the fp16 matrix cores (+ noise V): the 16-, 64- and 128-column block
    shapes, n not a multiple of 8; refilled after a parameter update."""
    rng = np.random.default_rng(40 + d + t)
    X = rng.uniform(-2, 2, size=(n, d)).astype(np.float32)
    V = rng.normal(size=(t, n)).astype(np.float32)
    params = _params(rng, d, ard)
    print(f"materialized case kind={kind} ard={ard} d={d} n={n} t={t}", flush=True)
    p = NativeProvider(kind, ard, X, params, 0.07)
    try:
        p.materialize()
        got = p.forward_matvec(V)
        params2 = _params(rng, d, ard, 0.3, 0.9, os=0.6)
        p.update_params(params2)
        got2 = p.forward_matvec(V)
    finally:
        p.close()
    ref = ok.forward_matvec(kind, X, V, params, 0.07, ard)
    ref2 = ok.forward_matvec(kind, X, V, params2, 0.07, ard)
    print(f"  relerr {_relerr(got, ref):.3e}, after update {_relerr(got2, ref2):.3e}", flush=True)
    assert _relerr(got, ref) <= TOL
    assert _relerr(got2, ref2) <= TOL


@pytest.mark.parametrize("kind,ard,d,n,t", [(ok.RBF, True, 3, 700, 5), (ok.MATERN52, True, 4, 900, 2),
                                            (ok.RBF, False, 2, 500, 3), (ok.MATERN52, False, 1, 600, 1)])
def test_gradient_matvec_parity(kind, ard, d, n, t):
    """Fused gradient products against the float64 closed-form derivatives."""
    rng = np.random.default_rng(60 + d + t)
    X = rng.normal(size=(n, d)).astype(np.float32)
    V = rng.normal(size=(t, n)).astype(np.float32)
    params = _params(rng, d, ard)
    print(f"gradient case kind={kind} ard={ard} d={d} n={n} t={t}", flush=True)
    p = NativeProvider(kind, ard, X, params, 0.05)
    try:
        got = p.gradient_matvec(V)
        times, _, out = p.benchmark_op(V, 2, 2, 1)
    finally:
        p.close()
    ref = ok.gradient_matvec(kind, X, V, params, ard)
    got = got.reshape(ref.shape)
    errs = [_relerr(got[q], ref[q]) for q in range(ref.shape[0])]
    print(f"  per-parameter relerr max {max(errs):.3e}", flush=True)
    assert max(errs) <= TOL
    assert np.array_equal(out.reshape(ref.shape), got)


def test_full_size_c3_sampled_rows():
    """BASELINE config 3 shape (N=250k, d=16, t=16, Matern-5/2 ARD): rows sampled
    across the matrix are compared with the float64 oracle."""
    rng = np.random.default_rng(0)
    n, d, t = 250_000, 16, 16
    X = rng.normal(size=(n, d)).astype(np.float32)
    V = rng.normal(size=(t, n)).astype(np.float32)
    V /= np.linalg.norm(V, axis=1, keepdims=True)
    params = np.concatenate([np.full(d, 1.0), [1.0]]).astype(np.float32)
    p = NativeProvider(ok.MATERN52, True, X, params, 0.1)
    try:
        got = p.forward_matvec(V)
    finally:
        p.close()
    rows = np.sort(rng.choice(n, size=192, replace=False))
    ref = ok.forward_matvec(ok.MATERN52, X, V, params, 0.1, True, rows=rows, block=64)
    err = _relerr(got[:, rows], ref)
    print(f"C3 sampled-row relerr {err:.3e}", flush=True)
    assert err <= TOL
