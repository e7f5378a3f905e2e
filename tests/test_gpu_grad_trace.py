"""Matrix-core gradient trace (Gram-form kernels) against the pair-loop trace
and the float64 oracle, through mgp_bbmm_eval.

MGP_GRAD_MFMA=1 takes the matrix-core trace for any n the route allows, =0
keeps the pair-loop trace.  The two device routes run the same mBCG solves,
so their gradients differ only by the trace arithmetic; the oracle bar is the
existing BBMM bar (1e-3 norm-wise, set by the stochastic probes' fp32 solves)."""

import ctypes as C

import numpy as np
import pytest

from mojogp_amd import _lib
from mojogp_amd._provider import NativeProvider
from oracle import engine as oe
from oracle import kernels as ok

pytestmark = pytest.mark.gpu


def _rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def _bbmm(kind, ard, X, y, params, noise, mean, T, it, rank):
    p = NativeProvider(kind, ard, X, params, noise)
    g = np.zeros(params.size + 1, np.float32)
    nll, iq, ld, ci, pl = C.c_float(), C.c_float(), C.c_float(), C.c_int(), C.c_float()
    try:
        _lib.call("mgp_bbmm_eval", p.handle, _lib.fptr(y), mean, T, 100, 30, 1e-2, it, rank,
                  C.byref(nll), C.byref(iq), C.byref(ld), _lib.fptr(g), C.byref(ci),
                  C.byref(pl), None)
    finally:
        p.close()
    return g, nll.value, ci.value


# kind, ard, d, n, probes, rank: 2 .. 11 blocks of 256 points (odd and even,
# partial last blocks), K=32 distance MFMA counts 1 and 2 (d = 1 .. 16).
CASES = [
    (ok.RBF, False, 1, 300, 10, 0),
    (ok.MATERN52, True, 4, 1000, 15, 30),
    (ok.RBF, True, 8, 777, 15, 50),
    (ok.MATERN32, True, 10, 1300, 15, 40),
    (ok.MATERN52, True, 16, 600, 7, 0),
    (ok.MATERN52, False, 3, 2600, 15, 20),
]


@pytest.mark.parametrize("kind,ard,d,n,T,rank", CASES)
def test_mfma_trace_matches_pair_loop_and_oracle(monkeypatch, kind, ard, d, n, T, rank):
    rng = np.random.default_rng(70 + d + n)
    X = rng.uniform(-2, 2, size=(n, d)).astype(np.float32)
    y = (np.sin(X).sum(1) + 0.1 * rng.normal(size=n)).astype(np.float32)
    params = np.concatenate([rng.uniform(0.7, 1.3, d if ard else 1), [1.1]]).astype(np.float32)
    noise, mean, it = 0.08, 0.05, 3
    print(f"trace case kind={kind} ard={ard} d={d} n={n} T={T} rank={rank}", flush=True)
    monkeypatch.setenv("MGP_GRAD_MFMA", "1")
    g_mfma, nll_m, ci_m = _bbmm(kind, ard, X, y, params, noise, mean, T, it, rank)
    monkeypatch.setenv("MGP_GRAD_MFMA", "0")
    g_loop, nll_l, ci_l = _bbmm(kind, ard, X, y, params, noise, mean, T, it, rank)
    assert ci_m == ci_l and nll_m == nll_l  # same solves
    e_loop = _rel(g_mfma[:-1], g_loop[:-1])
    P = None
    if rank > 0:
        K = ok.kernel_matrix(kind, X, X, params, ard)
        P = oe.Precond(oe.pivoted_cholesky(K, rank)[0], noise)
    y_c = (y - np.float32(mean)).astype(np.float64)
    r = oe.bbmm_step(kind, ard, X, y_c, params.astype(np.float64), noise, P, T, 100, 30, 1e-2, it)
    e_ref = _rel(g_mfma, r["grads"])
    print(f"  vs pair loop {e_loop:.2e}, vs oracle {e_ref:.2e} "
          f"(pair loop vs oracle {_rel(g_loop, r['grads']):.2e})", flush=True)
    assert e_loop <= 1e-4
    assert e_ref <= 1e-3
    assert g_mfma[-1] == g_loop[-1]  # the noise gradient has no trace


@pytest.mark.parametrize("kind,d", [(ok.MATERN52, 16), (ok.RBF, 8)])
def test_mfma_trace_auto_route_at_size(monkeypatch, kind, d):
    """From 4096 points on the default route is the matrix-core trace: its
    gradient matches the pair-loop trace of the same solves."""
    n = 20_000
    rng = np.random.default_rng(d)
    X = rng.normal(size=(n, d)).astype(np.float32)
    y = (np.sin(X).sum(1) + 0.1 * rng.normal(size=n)).astype(np.float32)
    params = np.concatenate([rng.uniform(0.8, 1.5, d), [1.0]]).astype(np.float32)
    print(f"trace auto case kind={kind} d={d} n={n}", flush=True)
    monkeypatch.delenv("MGP_GRAD_MFMA", raising=False)
    g_auto, nll_a, _ = _bbmm(kind, True, X, y, params, 0.1, 0.0, 15, 5, 50)
    monkeypatch.setenv("MGP_GRAD_MFMA", "0")
    g_loop, nll_l, _ = _bbmm(kind, True, X, y, params, 0.1, 0.0, 15, 5, 50)
    e = _rel(g_auto[:-1], g_loop[:-1])
    print(f"  vs pair loop {e:.2e}", flush=True)
    assert nll_a == nll_l
    assert e <= 1e-4
