"""GPU parity of mixed continuous x categorical kernels (GD, CR, EHH, HH, FE
correlation tables as leaves of a kernel tree) against the float64
restatements (oracle.categorical, oracle.kernels.TreeKernel,
oracle.engine.train_mixed): products with every table family, the split-Adam
fit's trajectory (continuous parameters, noise, mean, raw categorical
parameters), and prediction with the trained tables."""

import numpy as np
import pytest

from mojogp_amd import CR, EHH, FE, GD, HH, RBF, Matern52, SingleOutputGP
from mojogp_amd._provider import NativeProvider
from oracle import categorical as oc
from oracle import engine as oe
from oracle import kernels as ok

pytestmark = pytest.mark.gpu


def _rel(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def _data(n, seed):
    rng = np.random.default_rng(seed)
    X = np.stack([rng.uniform(-2, 2, n), rng.uniform(-2, 2, n), rng.integers(0, 3, n),
                  rng.integers(0, 4, n)], 1).astype(np.float32)
    eff = np.array([0.0, 0.8, -0.6])[X[:, 2].astype(int)]
    y = (np.sin(X[:, 0]) + 0.5 * np.cos(X[:, 1]) + eff + 0.1 * rng.normal(size=n)).astype(np.float32)
    return X, y


CASES = {
    "rbf*ehh+m52*gd": (lambda: RBF(active_dims=[0]) * EHH(3, active_dims=[2])
                       + Matern52(active_dims=[1]) * GD(4, active_dims=[3])),
    "rbf*(cr+hh)": (lambda: RBF() * (CR(3, active_dims=[2]) + HH(4, active_dims=[3]))),
    "m52*fe": (lambda: Matern52(ard=True) * FE(3, active_dims=[2])),
}
_KIND = {"GD": oc.GD, "CR": oc.CR, "EHH": oc.EHH, "HH": oc.HH, "FE": oc.FE}


def _tables(kernel, raw):
    specs = [(_KIND[lf.kernel_type.name], lf.levels) for lf in kernel.categorical_leaves()]
    out, o = [], 0
    for kind, L in specs:
        k = oc.num_params(kind, L)
        out.append(oc.correlation(kind, L, oc.constrain(kind, L, raw[o:o + k])))
        o += k
    return specs, out


@pytest.mark.parametrize("name", list(CASES))
def test_mixed_products_match_oracle(name):
    from mojogp_amd import make_ard_kernel
    X, _ = _data(900, 3)
    node = CASES[name]()
    if node.has_ard():
        node = make_ard_kernel(node, 2)
    cont = [0, 1]
    rng = np.random.default_rng(4)
    P = node.engine_num_params()
    params = rng.uniform(0.6, 1.4, P).astype(np.float32)
    leaves = node.categorical_leaves()
    raw = rng.normal(0.0, 0.8, sum(lf.num_params() for lf in leaves)).astype(np.float32)
    specs, tabs = _tables(node, raw)
    print(f"mixed products {name}: {P} continuous params, {raw.size} categorical", flush=True)
    V = rng.normal(size=(6, X.shape[0])).astype(np.float32)
    p = NativeProvider(None, False, X, params, 0.15, tree_spec=node.to_tree_spec(4, cont))
    try:
        p.set_categorical_params([k for k, _ in specs], raw)
        got = p.forward_matvec(V)
        p.materialize()
        mat = p.forward_matvec(V)
    finally:
        p.close()
    T = ok.TreeKernel(node.to_dict(), 4, tabs, cont)
    ref = ok.forward_matvec(T, X, V, params, 0.15, False)
    print(f"  forward {_rel(got, ref):.2e} materialized {_rel(mat, ref):.2e}", flush=True)
    assert _rel(got, ref) <= 1e-5
    assert _rel(mat, ref) <= 1e-5


@pytest.mark.parametrize("name", ["rbf*ehh+m52*gd", "rbf*(cr+hh)"])
def test_mixed_fit_predict_match_oracle(name, tmp_path):
    X, y = _data(400, 11)
    kernel = CASES[name]()
    gp = SingleOutputGP(kernel)
    tr = gp.fit(X, y, max_iterations=8, method="matrix_free", preconditioner_rank=10,
                learning_rate=0.05)
    assert gp.backend_train_info["is_mixed"]
    init_pub = gp.kernel.get_initial_params()
    init_eng = gp.kernel.to_engine_params(init_pub)
    leaves = gp.kernel.categorical_leaves()
    cat_init = init_pub[~np.array(gp.kernel._public_slots())].astype(np.float32)
    specs = [(_KIND[lf.kernel_type.name], lf.levels) for lf in leaves]
    ref = oe.train_mixed(gp.kernel.to_dict(), X, y, init_eng, 0.1, specs, cat_init,
                         default_dims=[0, 1], max_iterations=8, learning_rate=0.05,
                         num_probes=10, precond_rank=10)
    eng = gp.kernel.to_engine_params(tr.params)
    print(f"mixed fit {name}: params {eng} vs {ref['params']}; noise {tr.noise} vs "
          f"{ref['noise']}; mean {tr.mean} vs {ref['mean']}; cat {tr.cat_params} vs "
          f"{ref['cat_raw']}; nll {tr.nll} vs {ref['final_nll']}", flush=True)
    assert _rel(eng, ref["params"]) <= 1e-3
    assert tr.noise == pytest.approx(ref["noise"], rel=1e-3)
    assert tr.mean == pytest.approx(ref["mean"], rel=1e-3, abs=1e-4)
    assert _rel(tr.cat_params, ref["cat_raw"]) <= 1e-3
    assert tr.nll == pytest.approx(ref["final_nll"], rel=1e-3, abs=1e-4)
    rng = np.random.default_rng(5)
    Xs = np.stack([rng.uniform(-2, 2, 50), rng.uniform(-2, 2, 50), rng.integers(0, 3, 50),
                   rng.integers(0, 4, 50)], 1).astype(np.float32)
    mean_t, std_t = gp.predict(Xs, return_std=True, cg_tolerance=1e-6)
    _, tabs = _tables(gp.kernel, tr.cat_params)
    T = ok.TreeKernel(gp.kernel.to_dict(), 4, tabs, [0, 1])
    mu, var, _ = oe.predict(T, False, X, y, Xs, eng.astype(np.float64), tr.noise, tr.mean,
                            max_cg=300, tol=1e-6, lanczos_rank=100)
    print(f"  predict mean {_rel(mean_t, mu):.2e} std {_rel(std_t, np.sqrt(var)):.2e}", flush=True)
    assert _rel(mean_t, mu) <= 1e-4
    assert _rel(std_t, np.sqrt(var)) <= 1e-4
    gp.save(tmp_path / "mixed")
    gp2 = SingleOutputGP.load(str(tmp_path / "mixed"))
    np.testing.assert_array_equal(gp2.training_result.cat_params, tr.cat_params)
    m2, s2 = gp2.predict(Xs, return_std=True, cg_tolerance=1e-6)
    np.testing.assert_allclose(m2, mean_t, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(s2, std_t, rtol=1e-5, atol=1e-6)
