"""Driver of the library's host layer for the sanitizer build.

Run in a child process that loads mojogp_amd/lib/asan/libmojogp_amd.so (host
code under AddressSanitizer + UndefinedBehaviorSanitizer) with the ASan
runtime preloaded; tests/test_sanitized_host.py starts it and fails on any
sanitizer report or non-zero exit.

    python tests/sanitized_host_calls.py cpu   # no GPU needed
    python tests/sanitized_host_calls.py gpu   # end-to-end on the GPU

cpu: argument validation of the C entry points, null / unknown handles, the
error-message buffer, the task-covariance initialiser, and a mutation fuzz
of the kernel-tree spec parser (every spec must be rejected or accepted
without a memory error).
gpu: fit / predict through every route (matrix-free, materialized, kernel
tree, LMC, ICM, mixed categorical ICM and LMC), the prediction cache, save /
load and stale-handle rejection after destruction.
"""

from __future__ import annotations

import ctypes as C
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

from mojogp_amd import _lib  # noqa: E402


def _status(name, *args) -> int:
    return int(getattr(_lib.load(), name)(*args))


def _expect_fail(name, *args, contains=""):
    st = _status(name, *args)
    msg = _lib.last_error()
    assert st != 0, f"{name} accepted invalid arguments"
    assert contains in msg, f"{name}: {msg!r} lacks {contains!r}"


def cpu() -> None:
    lib = _lib.load()
    assert lib.mgp_version()
    # error buffer: truncation and NUL termination at every small size
    _expect_fail("mgp_init_provider", 9, 0, 1, 1, None, None, 0, 0.1, C.byref(C.c_void_p()),
                 contains="kernel kind")
    for size in (1, 2, 7, 64):
        buf = C.create_string_buffer(size)
        lib.mgp_last_error(buf, size)
        assert len(buf.value) <= size - 1
    X = np.zeros((4, 2), np.float32)
    fp = _lib.fptr
    h = C.c_void_p()
    p2 = np.array([1.0, 1.0], np.float32)
    cases = [
        ((0, 0, 0, 4, fp(X), fp(p2), 2, 0.1, C.byref(h)), "input dimension"),
        ((0, 0, 2, 0, fp(X), fp(p2), 2, 0.1, C.byref(h)), "n must be"),
        ((0, 0, 2, 4, None, fp(p2), 2, 0.1, C.byref(h)), "null input"),
        ((0, 1, 2, 4, fp(X), fp(p2), 2, 0.1, C.byref(h)), "expected 3"),
        ((0, 0, 2, 4, fp(X), fp(p2), 2, -1.0, C.byref(h)), "noise"),
        ((0, 0, 2, 4, fp(X), fp(np.array([np.nan, 1.0], np.float32)), 2, 0.1, C.byref(h)),
         "finite"),
        ((0, 0, 2, 4, fp(X), fp(p2), 2, 0.1, None), "out_handle"),
    ]
    for args, needle in cases:
        _expect_fail("mgp_init_provider", *args, contains=needle)
    # stale / unknown / null handles are rejected without being dereferenced
    junk = C.c_void_p(0x1234560)
    V = np.zeros((1, 4), np.float32)
    _expect_fail("mgp_destroy_provider", junk, contains="unknown or destroyed provider")
    _expect_fail("mgp_destroy_provider", None, contains="null provider")
    _expect_fail("mgp_forward_matvec", junk, fp(V), 1, fp(V), contains="unknown or destroyed")
    _expect_fail("mgp_materialize", junk, contains="unknown or destroyed")
    _expect_fail("mgp_destroy_prediction_cache", junk, contains="prediction cache")
    # mixed multi-output entry points: argument checks before any device work
    _expect_fail("mgp_lmc_train_mixed", None, 1, 1, None, None, None, None, None, None, None,
                 None, 0, None, None, None, None, contains="need >= 1 latent")
    _expect_fail("mgp_icm_train_mixed", junk, 2, None, None, None, 1.0, None, None, 0, None, 0,
                 None, _lib.PROGRESS_CB(), None, None, None, contains="unknown or destroyed")
    # host task-covariance initialiser
    W = np.zeros(6, np.float32)
    assert _status("mgp_icm_task_covariance_init", 3, 2, 42, fp(W)) == 0
    assert np.all(np.isfinite(W)) and np.all((W >= 0.1) & (W <= 0.5))
    # kernel-tree spec parser: valid specs, then mutations and truncations
    from mojogp_amd import RBF, RQ, Matern32, Periodic, make_ard_kernel
    trees = [(RBF() + Matern32(), 3), (make_ard_kernel(RQ(ard=True), 3) * Periodic(), 3),
             (2.0 * RBF(active_dims=[1]), 2)]
    rng = np.random.default_rng(0)
    accepted = rejected = 0
    Xt = np.zeros((3, 4), np.float32)
    pbig = np.ones(64, np.float32)
    for node, d in trees:
        spec = np.asarray(node.to_tree_spec(d), np.int32)
        for trial in range(200):
            s = spec.copy()
            if trial % 4 == 0:
                s = s[: rng.integers(0, len(s))]
            else:
                for _ in range(rng.integers(1, 4)):
                    k = rng.integers(0, len(s))
                    s[k] = rng.choice([-1, 0, 1, 2, 7, 33, 1 << 20, -(1 << 30), s[k] + 1])
            out = C.c_void_p()
            st = _status("mgp_init_provider_tree",
                         s.ctypes.data_as(C.POINTER(C.c_int)), len(s), d, 3, fp(Xt),
                         fp(pbig), int(s[1]) if len(s) > 1 and 0 < s[1] <= 64 else 1, 0.1,
                         C.byref(out))
            if st == 0:  # accepted (only possible with a device)
                accepted += 1
                _lib.call("mgp_destroy_provider", out)
            else:
                rejected += 1
                assert _lib.last_error()
    print(f"cpu: tree-spec fuzz {rejected} rejected, {accepted} accepted", flush=True)


def gpu() -> None:
    from mojogp_amd import (RBF, Matern52, MultiOutputGP, MultiOutputLMCGP, SingleOutputGP,
                            make_ard_kernel)
    from mojogp_amd._provider import KIND_MATERN52, NativeProvider
    import tempfile
    rng = np.random.default_rng(0)
    n, d = 600, 3
    X = rng.uniform(-2, 2, size=(n, d)).astype(np.float32)
    y = (np.sin(X).sum(1) + 0.05 * rng.normal(size=n)).astype(np.float32)
    Xs = rng.uniform(-2, 2, size=(50, d)).astype(np.float32)
    for method in ("matrix_free", "materialized"):
        gp = SingleOutputGP(make_ard_kernel(Matern52(ard=True), d))
        gp.fit(X, y, max_iterations=8, method=method)
        m1, s1 = gp.predict(Xs, return_std=True, variance_method="love")
        m2, v2 = gp.predict(Xs, return_var=True, variance_method="exact")
        assert np.all(np.isfinite(m1)) and np.all(np.isfinite(s1)) and np.all(v2 > 0)
        print(f"gpu: {method} fit + LOVE / exact predict", flush=True)
    gp.prepare_prediction_cache(variance_method="love")
    mc, sc = gp.predict(Xs, return_std=True)  # through the cache
    assert gp.backend_predict_info["alpha_cache_used"]
    assert np.all(np.isfinite(mc)) and np.all(np.isfinite(sc))
    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, "m.npz")
        gp.save(path)
        g2 = SingleOutputGP.load(path)
        assert np.all(np.isfinite(g2.predict(Xs).mean))
    tree = SingleOutputGP(RBF() + Matern52())
    tree.fit(X, y, max_iterations=5, method="matrix_free")
    assert np.all(np.isfinite(tree.predict(Xs, return_std=True)[1]))
    print("gpu: prediction cache, save / load, kernel tree", flush=True)
    T = 3
    Y = np.stack([np.sin(X[:, 0] + t) for t in range(T)], 1).astype(np.float32)
    icm = MultiOutputGP(RBF())
    icm.fit(X, Y, max_iterations=5, method="matrix_free")
    assert np.all(np.isfinite(icm.predict(Xs).mean))
    lmc = MultiOutputLMCGP([RBF(), Matern52()])
    lmc.fit(X, Y, max_iterations=5, method="matrix_free")
    assert np.all(np.isfinite(lmc.predict(Xs).mean))
    print("gpu: ICM and LMC fit + predict", flush=True)
    from mojogp_amd import EHH
    Xm = np.c_[X[:, :2], rng.integers(0, 3, n)].astype(np.float32)
    mixed = RBF() * EHH(3, active_dims=[2])
    icm_m = MultiOutputGP(mixed)
    icm_m.fit(Xm, Y, max_iterations=4, method="matrix_free")
    Xsm = np.c_[Xs[:, :2], rng.integers(0, 3, Xs.shape[0])].astype(np.float32)
    assert np.all(np.isfinite(icm_m.predict(Xsm).mean))
    lmc_m = MultiOutputLMCGP([RBF(), mixed])
    lmc_m.fit(Xm, Y, max_iterations=4, method="materialized")
    assert np.all(np.isfinite(lmc_m.predict(Xsm).mean))
    print("gpu: mixed ICM and LMC fit + predict", flush=True)
    params = np.concatenate([np.ones(d), [1.0]]).astype(np.float32)
    p = NativeProvider(KIND_MATERN52, True, X, params, 0.1)
    V = rng.normal(size=(4, n)).astype(np.float32)
    out = p.forward_matvec(V)
    h = p.handle
    p.close()
    st = _status("mgp_forward_matvec", h, _lib.fptr(V), 4, _lib.fptr(out))
    assert st != 0 and "unknown or destroyed" in _lib.last_error()
    print("gpu: destroyed handle rejected", flush=True)


if __name__ == "__main__":
    mode = sys.argv[1] if len(sys.argv) > 1 else "cpu"
    {"cpu": cpu, "gpu": gpu}[mode]()
    print(f"sanitized host layer: {mode} OK", flush=True)
