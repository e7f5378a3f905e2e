"""Parity of the symmetric K(X, X) V kernel (each off-diagonal kernel value
formed once, used for both of its entries) with the float64 oracle.

MGP_SYM_MATVEC=1 routes every square product with 1..16 right-hand sides
through it (any n), =0 keeps the one-sided tile kernel; unset, the symmetric
route is taken from 48 blocks of 512 points on.  Bar: norm-wise relative error
<= 1e-5 per right-hand side (the north star's matvec bar)."""

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


def _product(kind, ard, X, V, params, noise):
    p = NativeProvider(kind, ard, X, params, noise)
    try:
        return p.forward_matvec(V)
    finally:
        p.close()


# kind, ard, d, n, t: 1 .. 5 blocks of 512 points (odd and even), partial last
# blocks, every K=32 MFMA count (d = 1, 8, 16, 30), 1 .. 16 right-hand sides.
CASES = [
    (ok.MATERN52, True, 16, 17, 2),
    (ok.RBF, True, 8, 256, 16),
    (ok.MATERN52, True, 16, 300, 16),
    (ok.MATERN32, True, 4, 777, 11),
    (ok.RBF, False, 1, 1000, 16),
    (ok.MATERN52, True, 30, 1290, 5),
    (ok.RBF, True, 6, 2048, 3),
    (ok.MATERN52, True, 8, 1500, 1),
    (ok.MATERN52, False, 3, 2500, 16),
]


@pytest.mark.parametrize("kind,ard,d,n,t", CASES)
def test_symmetric_forward_parity(monkeypatch, kind, ard, d, n, t):
    rng = np.random.default_rng(4000 + 13 * d + n)
    print(f"symmetric case kind={kind} ard={ard} d={d} n={n} t={t}", flush=True)
    X = rng.normal(size=(n, d)).astype(np.float32)
    V = rng.normal(size=(t, n)).astype(np.float32)
    ls = rng.uniform(0.6, 1.6, size=d if ard else 1)
    params = np.concatenate([ls, [1.3]]).astype(np.float32)
    ref = ok.forward_matvec(kind, X, V, params, 0.05, ard)
    monkeypatch.setenv("MGP_SYM_MATVEC", "1")
    got = _product(kind, ard, X, V, params, 0.05)
    assert got.shape == V.shape and np.all(np.isfinite(got))
    err = _relerr(got, ref)
    print(f"  relerr {err:.3e}", flush=True)
    assert err <= TOL
    # A second product through the same workspaces (grown buffers reused).
    monkeypatch.setenv("MGP_SYM_MATVEC", "0")
    one_sided = _product(kind, ard, X, V, params, 0.05)
    assert _relerr(got, one_sided.astype(np.float64)) <= 2 * TOL


@pytest.mark.parametrize("kind,n,t", [(ok.MATERN52, 24_577, 16), (ok.RBF, 25_000, 9)])
def test_symmetric_auto_route_against_one_sided(monkeypatch, kind, n, t):
    """Above the block threshold the default route is symmetric: it agrees with
    the one-sided kernel on every entry and with the oracle on sampled rows."""
    rng = np.random.default_rng(n)
    d = 8
    print(f"symmetric auto case kind={kind} n={n} t={t}", flush=True)
    X = rng.normal(size=(n, d)).astype(np.float32)
    V = rng.normal(size=(t, n)).astype(np.float32)
    params = np.concatenate([rng.uniform(0.7, 1.4, size=d), [0.9]]).astype(np.float32)
    monkeypatch.delenv("MGP_SYM_MATVEC", raising=False)
    got = _product(kind, True, X, V, params, 0.1)
    monkeypatch.setenv("MGP_SYM_MATVEC", "0")
    one_sided = _product(kind, True, X, V, params, 0.1)
    rows = np.sort(rng.choice(n, size=128, replace=False))
    ref = ok.forward_matvec(kind, X, V, params, 0.1, True, rows=rows, block=64)
    e_ref = _relerr(got[:, rows], ref)
    e_one = _relerr(got, one_sided.astype(np.float64))
    print(f"  sampled-row relerr {e_ref:.3e}, vs one-sided {e_one:.3e}", flush=True)
    assert e_ref <= TOL
    assert e_one <= 2 * TOL


def test_symmetric_repeated_calls_bit_identical(monkeypatch):
    """Fixed-order reductions: the same product twice gives the same bits."""
    rng = np.random.default_rng(5)
    n, d, t = 3000, 5, 16
    X = rng.normal(size=(n, d)).astype(np.float32)
    V = rng.normal(size=(t, n)).astype(np.float32)
    params = np.array([1.1] * d + [1.0], dtype=np.float32)
    monkeypatch.setenv("MGP_SYM_MATVEC", "1")
    p = NativeProvider(ok.MATERN52, True, X, params, 0.1)
    try:
        a = p.forward_matvec(V)
        b = p.forward_matvec(V)
    finally:
        p.close()
    assert np.array_equal(a, b)


@pytest.mark.parametrize("kind,ard,d,n,t", [(ok.RBF, False, 4, 1100, 16),
                                            (ok.MATERN52, True, 3, 3000, 5),
                                            (ok.RBF, True, 2, 300, 1),
                                            (ok.MATERN32, False, 2, 200, 3),
                                            (ok.MATERN52, False, 32, 2000, 16),
                                            (ok.RBF, True, 7, 2001, 4)])
def test_materialized_symmetric_half(monkeypatch, kind, ard, d, n, t):
    """Materialized route, <= 16 columns: products from the symmetric half of K
    (5, 12, 2, 1 and 8 blocks of 256 points) against the oracle and against
    the full stored matrix (MGP_SYM_MATVEC=0), also after a parameter update.
    d = 32 is the largest input dimension the provider takes (the fill stages
    its points in LDS); n = 2001 packs the right-hand sides without 16-byte
    loads."""
    rng = np.random.default_rng(600 + n)
    X = rng.uniform(-2, 2, size=(n, d)).astype(np.float32)
    V = rng.normal(size=(t, n)).astype(np.float32)
    ls = rng.uniform(0.6, 1.4, size=d if ard else 1)
    params = np.concatenate([ls, [1.2]]).astype(np.float32)
    params2 = np.concatenate([ls * 0.7, [0.8]]).astype(np.float32)
    print(f"materialized symmetric case kind={kind} d={d} n={n} t={t}", flush=True)
    monkeypatch.delenv("MGP_SYM_MATVEC", raising=False)
    p = NativeProvider(kind, ard, X, params, 0.07)
    try:
        p.materialize()
        half = p.forward_matvec(V)
        monkeypatch.setenv("MGP_SYM_MATVEC", "0")
        full = p.forward_matvec(V)
        monkeypatch.delenv("MGP_SYM_MATVEC", raising=False)
        p.update_params(params2)
        half2 = p.forward_matvec(V)
    finally:
        p.close()
    ref = ok.forward_matvec(kind, X, V, params, 0.07, ard)
    ref2 = ok.forward_matvec(kind, X, V, params2, 0.07, ard)
    e, e_full, e2 = _relerr(half, ref), _relerr(half, full.astype(np.float64)), _relerr(half2, ref2)
    print(f"  relerr {e:.2e}, vs full {e_full:.2e}, after update {e2:.2e}", flush=True)
    assert e <= TOL and e2 <= TOL
    assert e_full <= 2 * TOL


@pytest.mark.parametrize("kind,ard,d,n,t", [(ok.RBF, True, 4, 17800, 16),
                                            (ok.MATERN52, False, 3, 20000, 7)])
def test_materialized_symmetric_multi_block_items(monkeypatch, kind, ard, d, n, t):
    """Sizes where a work item of the symmetric product covers several stored
    blocks (70 blocks, even: 18 splits of 2 offsets; 79 blocks, odd: 20 splits
    of 2), so the operand prefetch crosses blocks and some items are empty:
    every row against the full stored matrix (MGP_SYM_MATVEC=0), 128 sampled
    rows against the float64 oracle."""
    rng = np.random.default_rng(700 + n)
    X = rng.uniform(-2, 2, size=(n, d)).astype(np.float32)
    V = rng.normal(size=(t, n)).astype(np.float32)
    V[0] *= 1e-3                                      # columns of different scales
    ls = rng.uniform(0.6, 1.4, size=d if ard else 1)
    params = np.concatenate([ls, [1.1]]).astype(np.float32)
    rows = np.sort(rng.choice(n, size=128, replace=False))
    print(f"materialized symmetric multi-block case kind={kind} d={d} n={n} t={t}", flush=True)
    monkeypatch.delenv("MGP_SYM_MATVEC", raising=False)
    p = NativeProvider(kind, ard, X, params, 0.05)
    try:
        p.materialize()
        half = p.forward_matvec(V)
        monkeypatch.setenv("MGP_SYM_MATVEC", "0")
        full = p.forward_matvec(V)
        monkeypatch.delenv("MGP_SYM_MATVEC", raising=False)
    finally:
        p.close()
    ref = ok.forward_matvec(kind, X, V, params, 0.05, ard, rows=rows)
    e_full = _relerr(half, full.astype(np.float64))
    e = _relerr(half[:, rows], ref)
    print(f"  vs full {e_full:.2e}, sampled rows vs oracle {e:.2e}", flush=True)
    assert np.all(np.isfinite(half))
    assert e <= TOL and e_full <= 2 * TOL
