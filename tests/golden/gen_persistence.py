"""Writes tests/golden/ref_single_output_* and ref_lmc_* ({config.json,
arrays.npz}): model files written by the reference's own SingleOutputGP.save
(mojogp/gp.py:3648-3733) and MultiOutputLMCGP.save
(mojogp/multi_output_gp.py:6638-6743), run in the build container only.

The reference's save is pure Python; the trained state it serialises is set
directly (no engine is needed to write the file).  The fixture pins the
schema-v1 file format (config keys, kernel_tree / kernel_mojo_type strings,
array names) that mojogp_amd reads and writes.
"""

import json
import sys
from pathlib import Path

import numpy as np

REF = "/root/reference"
HERE = Path(__file__).parent


def main() -> None:
    sys.path.insert(0, REF)
    from mojogp.gp import SingleOutputGP, TrainingResult
    from mojogp.kernel import Kernel, make_ard_kernel

    rng = np.random.default_rng(3)
    n, d = 40, 3
    X = rng.uniform(-1, 1, size=(n, d)).astype(np.float32)
    y = np.sin(2 * X).sum(1).astype(np.float32)
    gp = SingleOutputGP(Kernel.matern52(ard=True))
    gp.dim = d
    gp.kernel = make_ard_kernel(gp._kernel_pre_ard, d)
    gp._X_train, gp._y_train = X, y
    gp._training_method = "matrix_free"
    gp._engine_predict_mean = 0.125
    gp._backend_train_info = {"training_route": "matrix_free", "precond_rank": 0}
    gp._training_result = TrainingResult(
        params=np.array([0.7, 0.9, 1.1, 1.3], np.float32), noise=0.05, mean=0.125,
        nll=0.42, iterations=7, converged=False, lanczos_root=None, lanczos_rank=30)
    gp._is_trained = True
    gp.save(str(HERE / "ref_single_output"))
    # LMC model (mojogp/multi_output_gp.py:6638-6743)
    from mojogp.multi_output_gp import LMCTrainingResult, MultiOutputLMCGP
    T, R = 2, 2
    Y = np.stack([np.sin(3 * X[:, 0]), np.cos(2 * X[:, 1])], 1).astype(np.float32)
    lmc = MultiOutputLMCGP(kernels=["rbf", "matern52"], num_probes=7)
    lmc.method = "matrix_free"
    A = np.array([[[1.0, 0.2], [0.2, 0.5]], [[0.3, -0.1], [-0.1, 0.8]]], np.float32)
    B = A.sum(0)
    lam, Q = np.linalg.eigh(B.astype(np.float64))
    lmc._result = LMCTrainingResult(
        final_nll=0.31, nll_history=np.array([0.5, 0.4, 0.31], np.float32), iterations=3,
        converged=False, num_latents=R, num_tasks=T,
        noise_per_task=np.array([0.04, 0.06], np.float32),
        lengthscales=np.array([0.6, 0.8], np.float32),
        outputscales=np.array([1.2, 0.9], np.float32),
        params_per_latent=[[0.6, 1.2], [0.8, 0.9]], kernel_types=np.array([0, 1], np.int32),
        A_matrices=A, L_factors=np.linalg.cholesky(A).astype(np.float32), B=B,
        Q=Q.astype(np.float32), Lambda=lam.astype(np.float32),
        alpha=rng.normal(size=n * T).astype(np.float32), use_ard=False,
        mean_per_task=np.array([0.1, -0.2], np.float32),
        var_diag=np.full((R, T), 0.1, np.float32),
        iter_times_ms=np.array([3.0, 2.5, 2.4], np.float64))
    lmc._X_train, lmc._Y_train = X, Y
    lmc._fitted_mean = lmc._result.mean_per_task
    lmc._is_trained = True
    lmc.save(str(HERE / "ref_lmc"))
    # kernel DSL strings for a few trees
    trees = {
        "rbf": Kernel.rbf(),
        "matern52_ard8": make_ard_kernel(Kernel.matern52(ard=True), 8),
        "rbf_ls": Kernel.rbf(lengthscale=0.5, outputscale=2.0),
    }
    out = {k: {"dict": v.to_dict(), "mojo_type": v.to_mojo_type()} for k, v in trees.items()}
    (HERE / "ref_kernel_strings.json").write_text(json.dumps(out, indent=2, sort_keys=True))


if __name__ == "__main__":
    main()
