"""The materialized route's full-matrix products (the fragment-ordered dense K)
against float64 at 1e-5, across the widths that pick each kernel: the narrow
product (<= 128 right-hand sides, per-wave operand loads, split partials) and
the wide one (> 128, LDS-staged 128 x 256 workgroup tiles, XCD-grouped
order), with ragged n and column counts (partial row and column blocks,
1, 2 and 4 column blocks per group)."""

import numpy as np
import pytest

from mojogp_amd._provider import NativeProvider
from oracle import kernels as ok

pytestmark = pytest.mark.gpu


def _rel(a, b):
    a = np.asarray(a, np.float64)
    return float(np.max(np.linalg.norm(a - b, axis=1) / np.linalg.norm(b, axis=1)))


@pytest.mark.parametrize("n,d,ncols", [(1000, 3, 17), (1000, 3, 70), (1000, 3, 129),
                                       (3001, 4, 300), (3001, 4, 513), (2304, 2, 1030)])
def test_full_dense_product_widths(monkeypatch, n, d, ncols):
    rng = np.random.default_rng(40 + n + ncols)
    X = rng.uniform(-2, 2, size=(n, d)).astype(np.float32)
    V = rng.normal(size=(ncols, n)).astype(np.float32)
    V[1] *= 1e-3                          # columns of different scales
    params = np.array([0.9, 1.3], np.float32)
    print(f"dense full product n={n} d={d} ncols={ncols}", flush=True)
    ref = ok.forward_matvec(ok.RBF, X, V, params, 0.05, False)
    p = NativeProvider(ok.RBF, False, X, params, 0.05)
    try:
        p.materialize()
        monkeypatch.setenv("MGP_SYM_MATVEC", "0")   # the full matrix for every width
        got = p.forward_matvec(V)
        monkeypatch.delenv("MGP_SYM_MATVEC")
    finally:
        p.close()
    err = _rel(got, ref)
    print(f"  max column relerr {err:.2e}", flush=True)
    assert np.all(np.isfinite(got))
    assert err <= 1e-5
