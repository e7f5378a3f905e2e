"""Model files against ones written by the reference's own SingleOutputGP.save
(tests/golden/gen_persistence.py): schema-v1 keys, kernel strings, arrays.

CPU: a reference-written file loads with the same state; our save writes the
reference's key set and array names; kernel_tree / kernel_mojo_type strings
match.  GPU: the loaded model predicts like the restated engine."""

import json
import shutil
from pathlib import Path

import numpy as np
import pytest

from mojogp_amd import Matern52, RBF, SingleOutputGP, make_ard_kernel
from mojogp_amd.kernel import KernelType

GOLD = Path(__file__).parent / "golden"
REF_CFG = json.loads((GOLD / "ref_single_output_config.json").read_text())


def _load_ref(tmp_path):
    for suffix in ("_config.json", "_arrays.npz"):
        shutil.copy(GOLD / f"ref_single_output{suffix}", tmp_path / f"m{suffix}")
    return SingleOutputGP.load(str(tmp_path / "m"))


def test_reference_file_loads(tmp_path):
    gp = _load_ref(tmp_path)
    tr = gp.training_result
    np.testing.assert_array_equal(tr.params, np.array([0.7, 0.9, 1.1, 1.3], np.float32))
    assert tr.noise == pytest.approx(0.05) and tr.mean == pytest.approx(0.125)
    assert tr.iterations == 7 and tr.lanczos_rank == 30 and not tr.converged
    assert gp.kernel.kernel_type == KernelType.MATERN52 and gp.kernel.ard_dim == 3
    arr = np.load(GOLD / "ref_single_output_arrays.npz")
    np.testing.assert_array_equal(gp._X_train, arr["X_train"])
    np.testing.assert_array_equal(gp._y_train, arr["y_train"])


def test_save_writes_reference_schema(tmp_path):
    gp = _load_ref(tmp_path)
    gp.save(str(tmp_path / "ours"))
    cfg = json.loads((tmp_path / "ours_config.json").read_text())
    assert set(cfg) == set(REF_CFG)
    for k, v in REF_CFG.items():
        if k != "mojogp_version":
            assert cfg[k] == v, k
    ours = np.load(tmp_path / "ours_arrays.npz")
    ref = np.load(GOLD / "ref_single_output_arrays.npz")
    assert set(ours.files) == set(ref.files)
    for k in ref.files:
        np.testing.assert_array_equal(ours[k], ref[k])


def test_kernel_strings_match_reference():
    ref = json.loads((GOLD / "ref_kernel_strings.json").read_text())
    ours = {"rbf": RBF(), "matern52_ard8": make_ard_kernel(Matern52(ard=True), 8),
            "rbf_ls": RBF(lengthscale=0.5, outputscale=2.0)}
    for name, k in ours.items():
        assert k.to_dict() == ref[name]["dict"], name
        assert k.to_mojo_type() == ref[name]["mojo_type"], name


@pytest.mark.gpu
def test_reference_file_predicts(tmp_path):
    from oracle import engine as oe
    from oracle import kernels as ok
    gp = _load_ref(tmp_path)
    Xs = np.random.default_rng(0).uniform(-1, 1, size=(20, 3)).astype(np.float32)
    mean, std = gp.predict(Xs, return_std=True, cg_tolerance=1e-6)
    tr = gp.training_result
    mu, var, _ = oe.predict(ok.MATERN52, True, gp._X_train, gp._y_train, Xs, tr.params,
                            tr.noise, 0.125, max_cg=300, tol=1e-6, lanczos_rank=200)
    np.testing.assert_allclose(mean, mu, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(std, np.sqrt(var), rtol=1e-4, atol=1e-5)


REF_LMC_CFG = json.loads((GOLD / "ref_lmc_config.json").read_text())


def _load_ref_lmc(tmp_path):
    from mojogp_amd import MultiOutputLMCGP
    for suffix in ("_config.json", "_arrays.npz"):
        shutil.copy(GOLD / f"ref_lmc{suffix}", tmp_path / f"l{suffix}")
    return MultiOutputLMCGP.load(str(tmp_path / "l"))


def test_reference_lmc_file_loads_and_resaves(tmp_path):
    gp = _load_ref_lmc(tmp_path)
    tr = gp.training_result
    ref = np.load(GOLD / "ref_lmc_arrays.npz")
    np.testing.assert_array_equal(tr.A_matrices, ref["A_matrices"])
    np.testing.assert_array_equal(tr.alpha, ref["alpha"])
    assert tr.params_per_latent == [ref["params_latent_0"].tolist(), ref["params_latent_1"].tolist()]
    assert gp.method == "matrix_free" and gp.num_probes == 7 and tr.num_tasks == 2
    gp.save(str(tmp_path / "ours"))
    cfg = json.loads((tmp_path / "ours_config.json").read_text())
    assert set(cfg) == set(REF_LMC_CFG)
    for k, v in REF_LMC_CFG.items():
        if k != "mojogp_version":
            assert cfg[k] == v, k
    ours = np.load(tmp_path / "ours_arrays.npz")
    assert set(ours.files) == set(ref.files)
    for k in ref.files:
        np.testing.assert_array_equal(ours[k], ref[k])


@pytest.mark.gpu
def test_reference_lmc_file_predicts(tmp_path):
    from oracle import kernels as ok
    from oracle import lmc as ol
    gp = _load_ref_lmc(tmp_path)
    tr = gp.training_result
    Xs = np.random.default_rng(1).uniform(-1, 1, size=(15, 3)).astype(np.float32)
    mean = gp.predict(Xs, variance_method="mean_only").mean
    params = [np.asarray(p, np.float64) for p in tr.params_per_latent]
    ref = ol.predict_mean([ok.RBF, ok.MATERN52], [False, False], gp._X_train, Xs, params,
                          tr.A_matrices, tr.alpha, tr.mean_per_task)
    np.testing.assert_allclose(mean, ref, rtol=1e-4, atol=1e-5)
