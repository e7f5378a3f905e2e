"""Pathwise prior draws against vectors written by the reference's own
mojogp/pathwise_prior.py (tests/golden/gen_pathwise_prior.py).

CPU: the seeded Generator is consumed in the reference's order (identical
weights) and the float64 restatement of the feature map reproduces the
reference's prior values.  GPU: the device evaluation does too."""

from pathlib import Path

import numpy as np
import pytest

from mojogp_amd._provider import KIND_MATERN12, KIND_MATERN32, KIND_MATERN52, KIND_RBF
from mojogp_amd.pathwise_prior import (build_feature_weights, build_pathwise_feature_map,
                                       sample_prior_values)
from oracle import lmc as ol

FIX = np.load(Path(__file__).parent / "golden" / "pathwise_prior.npz")
CASES = sorted({k.split("__")[0] for k in FIX.files})
KINDS = {"rbf": KIND_RBF, "m52": KIND_MATERN52, "m12": KIND_MATERN12, "m32": KIND_MATERN32}


def _case(name):
    seed, F, draws, d, ard = (int(v) for v in FIX[f"{name}__meta"])
    kind = KINDS[name.split("_")[0]]
    rng = np.random.default_rng(seed)
    fmap = build_pathwise_feature_map(kind, FIX[f"{name}__params"], input_dim=d, n_features=F,
                                      rng=rng, ard=bool(ard))
    w = build_feature_weights(fmap, draws, rng)
    return fmap, w, FIX[f"{name}__X"], FIX[f"{name}__values"]


@pytest.mark.parametrize("name", CASES)
def test_rng_order_and_values_match_reference(name):
    fmap, w, X, ref = _case(name)
    np.testing.assert_array_equal(w, FIX[f"{name}__weights"])
    vals = ol.rff_prior_values(X, fmap.lengthscales, fmap.W, fmap.phase, fmap.outputscale, w)
    np.testing.assert_allclose(vals, ref, rtol=1e-6, atol=1e-7)


@pytest.mark.gpu
@pytest.mark.parametrize("name", CASES)
def test_device_prior_values_match_reference(name):
    fmap, w, X, ref = _case(name)
    got = sample_prior_values(fmap, X, w)
    np.testing.assert_allclose(got, ref, rtol=1e-6, atol=1e-7)
