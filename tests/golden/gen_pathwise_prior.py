"""Writes tests/golden/pathwise_prior.npz from the reference's pathwise prior
(mojogp/pathwise_prior.py), run in the build container only.

Pins what no closed form fixes: the order in which a seeded
np.random.Generator is consumed by build_pathwise_feature_map (frequencies,
then phases) and build_feature_weights, and the scaling of
sample_prior_values.  Each case records the inputs (kernel, params, X, seed,
F, number of draws) and the reference's float32 prior values [draws, n].
"""

import sys
from pathlib import Path

import numpy as np

REF = "/root/reference"

CASES = [
    # name, kernel, ard, d, params, seed, F, draws, n
    ("rbf_iso_d3", "rbf", False, 3, [0.4, 1.3], 11, 64, 3, 7),
    ("m52_ard_d2", "matern52", True, 2, [0.3, 0.8, 1.7], 12, 96, 2, 9),
    ("m52_iso_d6", "matern52", False, 6, [0.7, 0.9], 13, 128, 4, 5),
    ("m12_ard_d3", "matern12", True, 3, [0.5, 0.9, 1.4, 0.8], 14, 80, 3, 6),
    ("m32_iso_d2", "matern32", False, 2, [0.6, 1.2], 15, 72, 2, 8),
]


def main() -> None:
    sys.path.insert(0, REF)
    from mojogp.kernel import Kernel, make_ard_kernel
    from mojogp.pathwise_prior import (build_feature_weights, build_pathwise_feature_map,
                                       sample_prior_values)
    out = {}
    for name, kname, ard, d, params, seed, F, draws, n in CASES:
        k = getattr(Kernel, kname)()
        if ard:
            k = make_ard_kernel(k, d)
        X = np.random.default_rng(100 + seed).uniform(0, 1, size=(n, d)).astype(np.float32)
        rng = np.random.default_rng(seed)
        fmap = build_pathwise_feature_map(k, np.asarray(params, np.float32), input_dim=d,
                                          n_features=F, rng=rng)
        w = build_feature_weights(fmap, draws, rng)
        vals = sample_prior_values(fmap, X, None, w)
        out[f"{name}__X"] = X
        out[f"{name}__params"] = np.asarray(params, np.float32)
        out[f"{name}__meta"] = np.array([seed, F, draws, d, int(ard)], np.int64)
        out[f"{name}__weights"] = w
        out[f"{name}__values"] = vals
    np.savez(Path(__file__).with_name("pathwise_prior.npz"), **out)


if __name__ == "__main__":
    main()
