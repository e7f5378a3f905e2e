"""Pins the C restatement of the reference matvec (oracle/cpu_ref) against the
float64 oracle; it is the cpu_baseline of bench.py."""

import numpy as np
import pytest

from oracle import cpu_ref
from oracle import kernels as ok


@pytest.mark.parametrize("kind,ard,d", [(ok.RBF, False, 1), (ok.RBF, True, 8), (ok.MATERN52, True, 16)])
def test_cpu_ref_matches_float64(kind, ard, d):
    rng = np.random.default_rng(3 + d)
    n, t = 700, 5
    X = rng.normal(size=(n, d)).astype(np.float32)
    V = rng.normal(size=(t, n)).astype(np.float32)
    params = np.concatenate([rng.uniform(0.7, 1.5, size=d if ard else 1), [1.2]]).astype(np.float32)
    got = cpu_ref.forward_matvec_rows(kind, ard, X, params, 0.1, V, 100, 250)
    ref = ok.forward_matvec(kind, X, V, params, 0.1, ard, rows=np.arange(100, 350))
    err = np.linalg.norm(got - ref, axis=1) / np.linalg.norm(ref, axis=1)
    assert err.max() < 1e-5


def test_cpu_ref_rejects_bad_shapes():
    X = np.zeros((4, 2), dtype=np.float32)
    with pytest.raises(ValueError):
        cpu_ref.forward_matvec_rows(0, True, X, np.ones(3, np.float32), 0.1,
                                    np.zeros((65, 4), np.float32), 0, 4)
