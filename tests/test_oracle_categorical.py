"""Pins of the categorical correlation restatement (oracle.categorical):
closed forms (GD, CR), unit diagonals, symmetry, unit-norm hypersphere rows
and positive semi-definite HH matrices, the EHH / FE exponent ranges, the
reference's default initial values and transform derivatives."""

import numpy as np
import pytest

from oracle import categorical as oc


@pytest.mark.parametrize("kind", [oc.GD, oc.CR, oc.EHH, oc.HH, oc.FE])
@pytest.mark.parametrize("L", [2, 3, 5])
def test_correlation_structure(kind, L):
    rng = np.random.default_rng(L + 10 * kind)
    raw = rng.normal(size=oc.num_params(kind, L))
    th = oc.constrain(kind, L, raw)
    R = oc.correlation(kind, L, th)
    np.testing.assert_allclose(np.diag(R), 1.0, atol=1e-12)
    np.testing.assert_allclose(R, R.T, atol=1e-12)
    assert np.all(np.abs(R) <= 1.0 + 1e-12)
    if kind != oc.HH:
        assert np.all(R > 0.0)
    if kind == oc.HH:
        assert np.linalg.eigvalsh(R).min() >= -1e-12


def test_closed_forms():
    R = oc.correlation(oc.GD, 3, [0.7])
    np.testing.assert_allclose(R[0, 1], np.exp(-0.7))
    th = np.array([0.1, 0.4, 0.9])
    R = oc.correlation(oc.CR, 3, th)
    np.testing.assert_allclose(R[0, 2], np.exp(-1.0))
    np.testing.assert_allclose(R[1, 2], np.exp(-1.3))
    # hypersphere rows have unit norm; L = 2 gives R_01 = cos(t)
    C = oc.hypersphere_factor([0.3, 1.1, 2.0], 3)
    np.testing.assert_allclose(np.sum(C * C, axis=1), 1.0)
    np.testing.assert_allclose(oc.correlation(oc.HH, 2, [0.8])[0, 1], np.cos(0.8))
    # EHH with L = 2: exp(h (1 - cos t)); t = 0 gives 1, t = pi gives 1e-12
    np.testing.assert_allclose(oc.correlation(oc.EHH, 2, [0.0])[0, 1], 1.0)
    np.testing.assert_allclose(oc.correlation(oc.EHH, 2, [np.pi])[0, 1], 1e-12, rtol=1e-9)
    # FE with zero angles-distance: R_01 = exp(-(d0 + d1)) when cos t = 1
    np.testing.assert_allclose(oc.correlation(oc.FE, 2, [0.0, 0.2, 0.5])[0, 1], np.exp(-0.7))


def test_defaults_and_chain():
    raw = oc.default_raw(oc.FE, 3)
    th = oc.constrain(oc.FE, 3, raw)
    np.testing.assert_allclose(th[:3], 0.25 * np.pi)
    np.testing.assert_allclose(th[3:], 0.3)
    np.testing.assert_allclose(oc.constrain(oc.GD, 4, oc.default_raw(oc.GD, 4)), 0.5)
    r = np.array([-0.3, 0.8, 1.5, 0.2, -1.0, 0.4])
    h = 1e-6
    fd = (oc.constrain(oc.FE, 3, r + h) - oc.constrain(oc.FE, 3, r - h)) / (2 * h)
    np.testing.assert_allclose(oc.chain_derivative(oc.FE, 3, r), fd, rtol=1e-7)


@pytest.mark.parametrize("kind", [oc.GD, oc.CR, oc.EHH, oc.HH, oc.FE])
def test_gradient_closed_forms(kind):
    L = 3
    th = oc.constrain(kind, L, np.linspace(-0.5, 0.7, oc.num_params(kind, L)))
    G = oc.correlation_gradients(kind, L, th)
    R = oc.correlation(kind, L, th)
    assert np.allclose(G[:, np.arange(L), np.arange(L)], 0.0, atol=1e-8) or kind == oc.HH
    if kind == oc.GD:
        np.testing.assert_allclose(G[0][0, 1], -np.exp(-th[0]), rtol=1e-8)
    if kind == oc.CR:
        np.testing.assert_allclose(G[1][1, 2], -R[1, 2], rtol=1e-8)
        np.testing.assert_allclose(G[1][0, 2], 0.0, atol=1e-10)
