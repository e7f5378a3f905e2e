#!/usr/bin/env python3
"""Headline benchmark of the MI355X exact-GP engine (one JSON line on stdout).

Metric: fused K.V matvec TFLOP/s at N=250k, d=16 (config 3:
Matern-5/2 ARD, t=16 right-hand sides).  One "step" is one fused forward
matvec (K + sigma^2 I) V over the 16 right-hand sides, inputs resident in HBM.

Work model (per (row, column) pair): F = 2d + 2t + c_k flops (c_k = 9 for
Matern-5/2, 5 for RBF) plus n_tr transcendentals (2 for Matern-5/2).
value = N^2 F / (host wall time per step); roofline.achieved uses the HIP-event
duration of the fused tile kernel measured on the provider's stream.  The
arithmetic is fp32-accurate (distances from an exact two-term fp16 split on
the fp16 matrix cores, the K.V product from a two-term fp16 split).
roofline.peak is the published dense fp16 MFMA peak (2.5 PFLOP/s) and frac =
achieved / peak.  The kernel is in fact bound by the mix of VALU (two
transcendentals and 5.5 other instructions per pair value) and 16-bit MFMA
issue, so roofline.pipe_model also reports the cycles per 16x16 tile that the
per-instruction costs measured live by mgp_pipe_probe give for the kernel's
instruction mix, expressed in the same algorithmic TFLOP/s.  At
config 3 the product runs on the symmetric kernel, which forms each
off-diagonal tile once for both of its entries (half the tiles, 1.5 more
MFMAs each); the model counts the tiles it forms, while value and achieved
stay per N^2 pairs.

The cpu_baseline leg times the C restatement of the reference matvec
(oracle/cpu_ref, OpenMP) on a bounded sample of rows of the same workload.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_FP16_MFMA_TFLOPS = 2500.0  # MI355X dense fp16 matrix peak (published)

N, D, T = 250_000, 16, 16
C_K = 9                        # Matern-5/2 epilogue flops per pair
N_TR = 2                       # sqrt + exp per pair
FLOPS_PER_PAIR = 2 * D + 2 * T + C_K
# HBM bytes per launch of the tile kernel at this workload (rocprofv3 FETCH_SIZE
# x 2.000 + WRITE_SIZE x 1.000, copy-kernel calibration): the symmetric kernel
# (profiles/symmetric_tile_c3_matvec.md: 1.610 GB read, 4.316 GB written, most
# of it the transposed partial sums) and the one-sided kernel
# (profiles/fused_tile_c3_matvec.md).
TILE_TRAFFIC_BYTES = {"symmetric": 5.926e9, "one_sided": 1.995e9}

# Instruction mix of the tile kernel k_fused_tile<Matern52, KB, NCG=1, R=4> per
# 16x16 tile (gfx950 ISA of this build): 4 pair values per lane, each with 2
# transcendentals (v_sqrt, v_exp) and 5.5 other VALU instructions (v_min, two
# FMAs, the product f*g, half a v_cvt_pk_f16_f32, one v_fma_mix); KB distance
# MFMAs plus 1.5 product MFMAs (v_mfma_f32_16x16x32_f16).
KB = -(-3 * (D + 2) // 32)
MFMA_PER_TILE = KB + 1.5
VALUES_PER_LANE = 4
TRANS_PER_VALUE, VALU_PER_VALUE = 2, 5.5
ROW_TILES, COL_TILES = -(-N // 16), 2 * -(-N // 32)


# Symmetric route (matvec.hip k_sym_tile / sym_route): square products with
# 1..16 right-hand sides over >= 48 blocks of 512 points form each
# off-diagonal 16x16 tile once and use it for both of its entries: the same
# VALU per tile, KB distance MFMAs plus 1.5 forward and 1.5 transposed product
# MFMAs.  The diagonal blocks are formed one-sided (both triangles).
SYM_ROWS, SYM_MIN_BLOCKS, SYM_MAX_BYTES = 512, 48, 16e9
SYM_MFMA_PER_TILE = KB + 3.0


def _sym_blocks(n, ncols=T):
    """(blocks, off-diagonal block pairs) when a square product of n points
    runs on the symmetric kernel, else None (the library's route rule,
    including the MGP_SYM_MATVEC switch)."""
    env = os.environ.get("MGP_SYM_MATVEC")
    if env is not None and env.startswith("0"):
        return None
    if not 1 <= ncols <= 16:
        return None
    nb = -(-n // SYM_ROWS)
    if env is None and nb < SYM_MIN_BLOCKS:
        return None
    if nb * (nb // 2) * SYM_ROWS * 16 * 4 > SYM_MAX_BYTES:
        return None
    return nb, nb * (nb - 1) // 2


def _pipe_model(probe):
    """Cycles per 16x16 tile (one-sided, symmetric) and the clock: VALU
    cycles plus the MFMA's measured cost inside a VALU stream (the two pipes
    overlap only partly on gfx950: out[4] of mgp_pipe_probe)."""
    ghz, c_tr, c_valu, c_mfma, c_mfma_mixed = probe[:5]
    valu = VALUES_PER_LANE * (TRANS_PER_VALUE * c_tr + VALU_PER_VALUE * c_valu)
    return valu + MFMA_PER_TILE * c_mfma_mixed, valu + SYM_MFMA_PER_TILE * c_mfma_mixed, ghz


def _tile_counts():
    """(one-sided tiles, symmetric tiles, MFMAs, kernel name) of one config-3 product."""
    sym = _sym_blocks(N)
    if sym is None:
        tiles = ROW_TILES * COL_TILES
        return tiles, 0, tiles * MFMA_PER_TILE, "k_fused_tile (one-sided)"
    nb, off = sym
    per_block = (SYM_ROWS // 16) ** 2
    diag, offt = nb * per_block, off * per_block
    return diag, offt, diag * MFMA_PER_TILE + offt * SYM_MFMA_PER_TILE, "k_sym_tile (symmetric)"


def _probe():
    import ctypes
    from mojogp_amd import _lib
    out = (ctypes.c_double * 6)()
    _lib.call("mgp_pipe_probe", out, 6)
    return [float(v) for v in out]


def _make_inputs():
    rng = np.random.default_rng(0)
    X = rng.normal(size=(N, D)).astype(np.float32)
    V = rng.normal(size=(T, N)).astype(np.float32)
    V /= np.linalg.norm(V, axis=1, keepdims=True)
    params = np.concatenate([np.ones(D), [1.0]]).astype(np.float32)
    return X, V, params, 0.1


def _mbcg_iteration_ms(X, params, noise, iterations: int = 20, kind=None, ard=True, rank=200):
    """One mBCG iteration over t=16 columns (y plus 15 probes) with a rank-`rank`
    greedy pivoted-Cholesky preconditioner and its Woodbury apply (config 3 by
    default: Matern-5/2 ARD, rank 200).  Returns (ms per iteration, wall
    seconds of the eval)."""
    import ctypes
    from mojogp_amd import _lib
    from mojogp_amd._provider import NativeProvider, KIND_MATERN52
    n = X.shape[0]
    rng = np.random.default_rng(1)
    y = rng.normal(size=n).astype(np.float32)
    prov = NativeProvider(KIND_MATERN52 if kind is None else kind, ard, X, params, noise)
    g = np.zeros(params.size + 1, np.float32)
    nll, iq, ld, pl = (ctypes.c_float() for _ in range(4))
    ci, loop_ms = ctypes.c_int(), ctypes.c_double()
    t0 = time.perf_counter()
    try:
        _lib.call("mgp_bbmm_eval", prov.handle, _lib.fptr(y), 0.0, T - 1, iterations,
                  iterations, 0.0, 0, rank, ctypes.byref(nll), ctypes.byref(iq),
                  ctypes.byref(ld), _lib.fptr(g), ctypes.byref(ci), ctypes.byref(pl),
                  ctypes.byref(loop_ms))
    finally:
        prov.close()
    return loop_ms.value / max(ci.value, 1), time.perf_counter() - t0


def _mbcg_iteration_ms_c2(iterations: int = 20):
    """One mBCG iteration at config 2: RBF ARD, N=50k, d=8, rank 100."""
    from mojogp_amd._provider import KIND_RBF
    rng = np.random.default_rng(0)
    X = rng.uniform(size=(50_000, 8)).astype(np.float32)
    params = np.concatenate([np.full(8, 0.5), [1.0]]).astype(np.float32)
    return _mbcg_iteration_ms(X, params, 0.01, iterations, kind=KIND_RBF, rank=100)[0]


def _c3_fit_predict_seconds():
    """Config 3 end to end: Matern-5/2 ARD, N=250k, d=16, 50 Adam steps, 15
    probes, rank-200 preconditioner (matrix-free), then mean + LOVE std at
    10 000 test points (the generator of tests/test_gpu_configs_at_size.py)."""
    from mojogp_amd import Matern52, SingleOutputGP
    rng = np.random.default_rng(0)
    X = rng.normal(size=(N, D)).astype(np.float32)
    W = rng.normal(size=(1024, D)) / 2.0
    b = rng.uniform(0, 2 * np.pi, size=1024)
    w = rng.normal(size=1024)
    y = (np.sqrt(2.0 / 1024) * np.cos(X @ W.T + b) @ w
         + 0.05 * rng.normal(size=N)).astype(np.float32)
    Xs = rng.normal(size=(10_000, D)).astype(np.float32)
    gp = SingleOutputGP(Matern52(ard=True))
    t0 = time.perf_counter()
    tr = gp.fit(X, y, method="matrix_free", max_iterations=50, num_probes=15,
                cg_tolerance=1e-2, preconditioner_rank=200)
    fit_s = time.perf_counter() - t0
    t0 = time.perf_counter()
    gp.predict(Xs, return_std=True, variance_method="love")
    pred_s = time.perf_counter() - t0
    info = gp.backend_train_info or {}
    return fit_s, pred_s, {"final_nll": tr.nll,
                           "cg_iterations_total": info.get("cg_iterations_total")}


def _fit_c2_seconds():
    """Config 2 end to end: RBF-ARD, N=50k, d=8, 30 Adam steps, 15 probes,
    rank-100 greedy preconditioner (matrix-free)."""
    from mojogp_amd import RBF, SingleOutputGP
    rng = np.random.default_rng(0)
    X = rng.uniform(size=(50_000, 8)).astype(np.float32)
    y = (np.sin(3 * X).sum(1) + 0.1 * rng.normal(size=50_000)).astype(np.float32)
    gp = SingleOutputGP(RBF(ard=True))
    t0 = time.perf_counter()
    tr = gp.fit(X, y, max_iterations=30, method="matrix_free", num_probes=15,
                preconditioner_rank=100, preconditioner="greedy")
    dt = time.perf_counter() - t0
    info = gp.backend_train_info or {}
    return dt, {"final_nll": tr.nll, "cg_iterations_total": info.get("cg_iterations_total")}


def _c4_product_only():
    """The config-4 16-column dense product alone (profiling): one materialize
    of K(X, X) (RBF, lengthscale 1.5, outputscale 1, noise 0.01, X ~ U(-2, 2)^4,
    seed 0), then 3 warm-up and 30 timed products."""
    from mojogp_amd._provider import NativeProvider, KIND_RBF
    rng = np.random.default_rng(0)
    n = 40_000
    X = rng.uniform(-2, 2, size=(n, 4)).astype(np.float32)
    prov = NativeProvider(KIND_RBF, False, X, np.array([1.5, 1.0], np.float32), 0.01)
    try:
        prov.materialize()
        V = rng.normal(size=(16, n)).astype(np.float32)
        t, _, _ = prov.benchmark_forward(V, 30, 3)
    finally:
        prov.close()
    return {"dense_matvec_ms_16_mean": round(float(np.mean(t)), 4),
            "dense_matvec_ms_16_min": round(float(np.min(t)), 4)}


def _c4_wide_product_only():
    """The config-4 4096-column dense product alone (profiling): one
    materialize (as _c4_product_only), the full K filled by a warm-up
    product, then 3 timed products of 4096 columns (the exact-variance
    block)."""
    from mojogp_amd._provider import NativeProvider, KIND_RBF
    rng = np.random.default_rng(0)
    n = 40_000
    X = rng.uniform(-2, 2, size=(n, 4)).astype(np.float32)
    prov = NativeProvider(KIND_RBF, False, X, np.array([1.5, 1.0], np.float32), 0.01)
    try:
        prov.materialize()
        V = rng.normal(size=(4096, n)).astype(np.float32)
        t, _, _ = prov.benchmark_forward(V, 3, 1)
    finally:
        prov.close()
    return {"dense_matvec_ms_4096_mean": round(float(np.mean(t)), 3),
            "dense_matvec_ms_4096_min": round(float(np.min(t)), 3)}


def _c3_gradient_trace_only():
    """The config-3 gradient trace alone (profiling): the matrix-core trace
    sum_ab dK_p[a,b] (Lf Rf^T)_ab over N = 250k, d = 16, Matern-5/2 ARD with
    16 weight columns (the BBMM gradient step's shape: alpha and 15 probe
    solves), 1 warm-up and 5 timed calls through mgp_gradient_trace."""
    from mojogp_amd._provider import NativeProvider, KIND_MATERN52
    X, _, params, noise = _make_inputs()
    rng = np.random.default_rng(1)
    L = rng.normal(size=(T, N)).astype(np.float32)
    R = rng.normal(size=(T, N)).astype(np.float32)
    prov = NativeProvider(KIND_MATERN52, True, X, params, noise)
    try:
        prov.gradient_trace(L, R)
        t = []
        for _ in range(5):
            t0 = time.perf_counter()
            prov.gradient_trace(L, R)
            t.append((time.perf_counter() - t0) * 1e3)
    finally:
        prov.close()
    return {"gradient_trace_ms_mean": round(float(np.mean(t)), 3),
            "gradient_trace_ms_min": round(float(np.min(t)), 3)}


def _c4_materialized():
    """Config 4: RBF (isotropic) N=40k d=4 on the materialized route (dense K as a
    two-term fp16 split: the symmetric half, 3.25 GB, for products of <= 16
    columns, the full 6.46 GB layout for wider ones), default fit, exact
    variance at 4096 test points (the generator of
    tests/test_gpu_configs_at_size.py), and the dense product alone at 16 and
    4096 right-hand sides (wall time per call, column maxima + packing + MFMA
    product + reduction, inputs resident on the device)."""
    from mojogp_amd import RBF, SingleOutputGP
    from mojogp_amd._provider import NativeProvider, KIND_RBF
    rng = np.random.default_rng(0)
    n, d, m = 40_000, 4, 4096
    X = rng.uniform(-2, 2, size=(n, d)).astype(np.float32)
    y = (np.prod(np.cos(X), axis=1) + 0.05 * rng.normal(size=n)).astype(np.float32)
    Xs = rng.uniform(-2, 2, size=(m, d)).astype(np.float32)
    gp = SingleOutputGP(RBF())
    t0 = time.perf_counter()
    tr = gp.fit(X, y, method="materialized")
    fit_s = time.perf_counter() - t0
    info = gp.backend_train_info or {}
    t0 = time.perf_counter()
    gp.predict(Xs, return_var=True, variance_method="exact")
    ev_s = time.perf_counter() - t0
    einfo = gp.backend_predict_info or {}
    params = np.asarray(gp.kernel.to_engine_params(np.asarray(tr.params, np.float32)),
                        np.float32)
    prov = NativeProvider(KIND_RBF, False, X, params, float(tr.noise))
    try:
        prov.materialize()
        # The 16-column product reads the stored symmetric half of K: the
        # diagonal and cyclic-half blocks of 256 points, 4 B per entry.
        nbk = -(-n // 256)
        kbytes = 4.0 * 256 * 256 * nbk * (nbk + 1) / 2
        t16, _, _ = prov.benchmark_forward(rng.normal(size=(16, n)).astype(np.float32), 10, 2)
        ms16 = float(np.median(t16))
        tw, _, _ = prov.benchmark_forward(rng.normal(size=(m, n)).astype(np.float32), 3, 1)
        msw = float(np.median(tw))
    finally:
        prov.close()
    flops_w = 2.0 * n * n * m
    return {
        "workload": "config 4: RBF N=40000 d=4, materialized route, default fit, exact "
                    "variance at 4096 test points",
        "fit_seconds": round(fit_s, 3),
        "fit_iterations": len(tr.nll_history),
        "cg_iterations_total": info.get("cg_iterations_total"),
        "exact_variance_seconds": round(ev_s, 3),
        "exact_cg_total_iterations": einfo.get("exact_cg_total_iterations"),
        "lengthscale": float(params[0]),
        "dense_matvec_ms_16": round(ms16, 4),
        "dense_matvec_bytes_16": kbytes,
        "dense_matvec_GBps_16": round(kbytes / (ms16 * 1e-3) / 1e9, 1),
        "dense_matvec_ms_4096": round(msw, 3),
        "dense_matvec_fp32_equiv_tflops_4096": round(flops_w / (msw * 1e-3) / 1e12, 2),
        "dense_matvec_fp16_mfma_tflops_4096": round(3 * flops_w / (msw * 1e-3) / 1e12, 2),
    }


C5_N, C5_D, C5_T, C5_PROBES = 20_000, 6, 4, 15
C5_C = C5_PROBES + 1                   # columns per task block (t = 16)


def _c5_data(seed: int = 0):
    """Config 5 generator: X ~ U[0,1]^{20000 x 6}; latent f1 = RBF (l = 0.2) and
    f2 = Matern-5/2 (l = 0.7) random-Fourier-feature draws (1024 features, the
    Matern frequencies multivariate-t with 5 degrees of freedom); W ~ N(0,1)^{4x2};
    Y = [f1 f2] W^T + 0.05 N(0,1)."""
    rng = np.random.default_rng(seed)
    X = rng.uniform(0, 1, size=(C5_N, C5_D)).astype(np.float32)

    def rff(ls, matern):
        Wf = rng.standard_normal((1024, C5_D))
        if matern:
            Wf = Wf / np.sqrt(rng.chisquare(5, size=(1024, 1)) / 5.0)
        b = rng.uniform(0, 2 * np.pi, size=1024)
        w = rng.standard_normal(1024)
        return lambda Z: np.sqrt(2.0 / 1024) * np.cos(Z / ls @ Wf.T + b) @ w

    f1, f2 = rff(0.2, False), rff(0.7, True)
    Wm = rng.standard_normal((C5_T, 2))
    Y = (np.stack([f1(X), f2(X)], 1) @ Wm.T
         + 0.05 * rng.standard_normal((C5_N, C5_T))).astype(np.float32)
    Xs = rng.uniform(0, 1, size=(1000, C5_D)).astype(np.float32)
    return X, Y, Xs, Wm


def _c5_flops_per_pair():
    """Structured product work per (i, j) pair summed over the two latents:
    per latent 2d + 2 T C + c_k (RBF 5, Matern-5/2 9)."""
    return (2 * C5_D + 2 * C5_T * C5_C + 5) + (2 * C5_D + 2 * C5_T * C5_C + 9)


def _lmc_c5(repeats: int, warmup: int):
    """Config 5 legs: the structured product (K_full V over 16 task-blocked
    columns = 64 columns per latent, inputs resident), one LMC mBCG iteration
    (15 probes, rank-15 greedy preconditioner per latent), and the end-to-end
    MultiOutputLMCGP fit (matrix-free, 15 probes, reference defaults otherwise)
    plus 64 pathwise posterior samples at 1000 test points."""
    import ctypes
    from mojogp_amd import MultiOutputLMCGP, _lib
    from mojogp_amd._provider import KIND_MATERN52, KIND_RBF, NativeProvider
    X, Y, Xs, Wm = _c5_data()
    A = np.stack([np.outer(Wm[:, s], Wm[:, s]) + 0.1 * np.eye(C5_T)
                  for s in range(2)]).astype(np.float32)
    noise = np.full(C5_T, 0.0025, np.float32)
    provs = [NativeProvider(KIND_RBF, False, X, np.array([0.2, 1.0], np.float32), 0.0),
             NativeProvider(KIND_MATERN52, False, X, np.array([0.7, 1.0], np.float32), 0.0)]
    rng = np.random.default_rng(2)
    V = rng.standard_normal((C5_C, C5_T * C5_N)).astype(np.float32)
    times = np.zeros(repeats, np.float64)
    y = np.ascontiguousarray((Y - Y.mean(0)).T.reshape(-1), dtype=np.float32)
    nll, iq, ld, pl = (ctypes.c_float() for _ in range(4))
    ci, loop_ms = ctypes.c_int(), ctypes.c_double()
    try:
        _lib.call("mgp_lmc_benchmark_forward", _lib.handles(provs), 2, C5_T, _lib.fptr(A),
                  _lib.fptr(noise), _lib.fptr(V), C5_C, repeats, warmup, _lib.dptr(times), None)
        _lib.call("mgp_lmc_bbmm_eval", _lib.handles(provs), 2, C5_T, _lib.fptr(A),
                  _lib.fptr(noise), None, _lib.fptr(y), C5_PROBES, 200, 30, 1.0, 0, 15, 0,
                  ctypes.byref(nll), ctypes.byref(iq), ctypes.byref(ld), None, None, None, None,
                  ctypes.byref(ci), ctypes.byref(pl), ctypes.byref(loop_ms))
    finally:
        for p in provs:
            p.close()
    ms = float(np.median(times))
    flops = float(C5_N) * C5_N * _c5_flops_per_pair()
    gp = MultiOutputLMCGP(kernels=["rbf", "matern52"], num_probes=C5_PROBES)
    t0 = time.perf_counter()
    res = gp.fit(X, Y, method="matrix_free")
    fit_s = time.perf_counter() - t0
    t0 = time.perf_counter()
    gp.sample_posterior(Xs, n_samples=64, method="pathwise", rng=np.random.default_rng(1))
    samp_s = time.perf_counter() - t0
    return {
        "workload": "config 5: LMC N=20000 d=6 T=4 Q=2 (RBF l=0.2, Matern-5/2 l=0.7), "
                    "t=16 task-blocked columns (64 per latent), synthetic RFF data seed 0",
        "structured_matvec_ms": round(ms, 4),
        "structured_matvec_tflops": round(flops / (ms * 1e-3) / 1e12, 3),
        "mbcg_iter_ms": round(loop_ms.value / max(ci.value, 1), 3),
        "mbcg_iterations": ci.value,
        "fit_seconds": round(fit_s, 3),
        "fit_iterations": res.iterations,
        "pathwise_64_samples_seconds": round(samp_s, 3),
    }, (X, V[:1])


def _c5_product_only(repeats: int = 30, warmup: int = 3):
    """The config-5 structured product alone (profiling): K_full V over 16
    task-blocked columns through mgp_lmc_benchmark_forward, inputs resident,
    `warmup` untimed and `repeats` timed calls."""
    from mojogp_amd import _lib
    from mojogp_amd._provider import KIND_MATERN52, KIND_RBF, NativeProvider
    X, _, _, Wm = _c5_data()
    A = np.stack([np.outer(Wm[:, s], Wm[:, s]) + 0.1 * np.eye(C5_T)
                  for s in range(2)]).astype(np.float32)
    noise = np.full(C5_T, 0.0025, np.float32)
    provs = [NativeProvider(KIND_RBF, False, X, np.array([0.2, 1.0], np.float32), 0.0),
             NativeProvider(KIND_MATERN52, False, X, np.array([0.7, 1.0], np.float32), 0.0)]
    V = np.random.default_rng(2).standard_normal((C5_C, C5_T * C5_N)).astype(np.float32)
    times = np.zeros(repeats, np.float64)
    try:
        _lib.call("mgp_lmc_benchmark_forward", _lib.handles(provs), 2, C5_T, _lib.fptr(A),
                  _lib.fptr(noise), _lib.fptr(V), C5_C, repeats, warmup, _lib.dptr(times), None)
    finally:
        for p in provs:
            p.close()
    return {"structured_matvec_ms_median": round(float(np.median(times)), 4),
            "structured_matvec_ms_min": round(float(np.min(times)), 4)}


def _cpu_model() -> str:
    """The host CPU's model name (first /proc/cpuinfo "model name" line)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _cpu_baseline_c5(X, V1, target_s: float):
    """Reference-order fp32 C restatement of the config-5 structured product on
    a bounded sample of rows: both latents' (K_s V) rows for the 64 columns
    (the T x T mixing is negligible next to it)."""
    from oracle import cpu_ref
    threads = cpu_ref.num_threads()
    Vc = np.ascontiguousarray(np.tile(V1.reshape(C5_T, C5_N), (C5_C, 1))[:C5_T * C5_C])
    lat = [(0, np.array([0.2, 1.0], np.float32)), (1, np.array([0.7, 1.0], np.float32))]

    def run(rows):
        for kind, p in lat:
            cpu_ref.forward_matvec_rows(kind, False, X, p, 0.0, Vc, 0, rows)

    probe = 64
    t0 = time.perf_counter()
    run(probe)
    dt = max(time.perf_counter() - t0, 1e-3)
    rows = int(min(C5_N, max(probe, target_s / dt * probe)))
    t0 = time.perf_counter()
    run(rows)
    dt = time.perf_counter() - t0
    return {
        "value": rows * C5_N * _c5_flops_per_pair() / dt / 1e12,
        "unit": "TFLOP/s",
        "cores": threads,
        "cpu_model": _cpu_model(),
        "kind": "port",
        "sample": f"rows [0,{rows}) of both latents' products (64 columns each) of the "
                  f"config-5 structured matvec; {dt:.1f} s on {threads} threads",
    }


def _c1_data():
    """Config 1: X = linspace(-3, 3, 2000), y = sin(2x) + 0.05 N(0, 1) (seed 0);
    test points linspace(-4, 4, 128)."""
    rng = np.random.default_rng(0)
    X = np.linspace(-3, 3, 2000, dtype=np.float32)[:, None]
    y = (np.sin(2 * X[:, 0]) + 0.05 * rng.normal(size=2000)).astype(np.float32)
    Xs = np.linspace(-4, 4, 128, dtype=np.float32)[:, None]
    return X, y, Xs


def _c1_gpu_seconds():
    """Config 1 on the GPU: 50-step matrix-free fit + LOVE predict at 128 points."""
    from mojogp_amd import RBF, SingleOutputGP
    X, y, Xs = _c1_data()
    gp = SingleOutputGP(RBF())
    t0 = time.perf_counter()
    gp.fit(X, y, max_iterations=50, method="matrix_free")
    gp.predict(Xs, return_std=True, variance_method="love")
    return time.perf_counter() - t0


def _row_sample_seconds(run, total_rows: int, target_s: float, probe: int = 64):
    """Seconds of run(rows) for all total_rows, extrapolated linearly from a
    timed prefix sized to about target_s.  Returns (seconds, rows timed)."""
    t0 = time.perf_counter()
    run(probe)
    dt = max(time.perf_counter() - t0, 1e-4)
    rows = int(min(total_rows, max(probe, target_s / dt * probe)))
    t0 = time.perf_counter()
    run(rows)
    dt = time.perf_counter() - t0
    return dt * total_rows / rows, rows


def _cpu_legs(gpu: dict, target_s: float) -> dict:
    """CPU timings of configs 1-4 on this host (the oracle restatements: the
    numpy training loop, the fp32 reference-order C product, numpy fp32 dense
    algebra), each beside the GPU figure of the same work.  Config 1 runs in
    full; the others time a prefix of rows of their products and extrapolate."""
    from oracle import cpu_ref
    from oracle import engine as oe
    from oracle import kernels as ok
    threads = cpu_ref.num_threads()
    legs = {}
    # config 1: the whole fit + predict
    X, y, Xs = _c1_data()
    t0 = time.perf_counter()
    ref = oe.train(ok.RBF, False, X, y, [1.0, 1.0], 0.1, max_iterations=50, num_probes=10,
                   max_cg=100, cg_tol=1e-2, precond_rank=0, max_tridiag=30)
    oe.predict(ok.RBF, False, X, y, Xs, np.asarray(ref["params"], np.float64), ref["noise"],
               ref["mean"], max_cg=300, tol=1e-3, lanczos_rank=100)
    c1 = time.perf_counter() - t0
    legs["c1"] = {"cpu_seconds": round(c1, 3), "gpu_seconds": gpu.get("c1"),
                  "work": "50-step fit + LOVE predict at 128 points, measured in full",
                  "kind": "port (numpy restatement of the training loop)"}
    # config 2: one 16-column product per CG iteration, times the GPU fit's CG count
    rng = np.random.default_rng(0)
    X2 = rng.uniform(size=(50_000, 8)).astype(np.float32)
    p2 = np.concatenate([np.full(8, 0.5), [1.0]]).astype(np.float32)
    V2 = rng.normal(size=(16, 50_000)).astype(np.float32)
    mv2, rows2 = _row_sample_seconds(
        lambda r: cpu_ref.forward_matvec_rows(0, True, X2, p2, 0.01, V2, 0, r), 50_000,
        target_s / 4)
    cg2 = gpu.get("c2_cg_iterations") or 0
    legs["c2"] = {"cpu_seconds_per_product": round(mv2, 3),
                  "cpu_fit_seconds_extrapolated": round(mv2 * cg2, 1) if cg2 else None,
                  "gpu_fit_seconds": gpu.get("c2_fit"),
                  "work": f"(K + s^2 I) V, 16 columns, rows [0,{rows2}) timed; fit = product x "
                          f"the GPU fit's {cg2} CG iterations (vector work and gradients "
                          f"not counted: a lower bound)",
                  "kind": "port (fp32 reference-order C restatement)"}
    # config 3: one mBCG iteration = product (row sample) + Woodbury apply (numpy)
    X3, _, p3, noise3 = _make_inputs()
    V3 = np.random.default_rng(1).normal(size=(16, N)).astype(np.float32)
    mv3, rows3 = _row_sample_seconds(
        lambda r: cpu_ref.forward_matvec_rows(1, True, X3, p3, noise3, V3, 0, r), N,
        target_s / 4)
    L = np.random.default_rng(2).normal(size=(200, N)).astype(np.float32)
    Minv = np.eye(200, dtype=np.float32)
    t0 = time.perf_counter()
    w = L @ V3.T
    z = (V3 - (L.T @ (Minv @ w)).T) / np.float32(noise3)
    wb3 = time.perf_counter() - t0
    legs["c3"] = {"cpu_ms_per_mbcg_iteration": round((mv3 + wb3) * 1e3, 1),
                  "gpu_ms_per_mbcg_iteration": gpu.get("c3_mbcg_ms"),
                  "work": f"product rows [0,{rows3}) timed and extrapolated, plus the rank-200 "
                          f"Woodbury apply in numpy fp32 ({wb3 * 1e3:.0f} ms); the gradient "
                          f"pass has no CPU restatement at this size",
                  "kind": "port (C restatement + numpy)"}
    del L, z, w
    # config 4: dense K fill and one 16-column product (row samples), and the
    # 4096-column exact-variance product
    rng4 = np.random.default_rng(0)
    n4 = 40_000
    X4 = rng4.uniform(-2, 2, size=(n4, 4)).astype(np.float32)
    ls, os_ = np.float32(gpu.get("c4_lengthscale") or 1.0), np.float32(1.0)
    blk = {}

    def fill(r):
        d2 = np.zeros((r, n4), np.float32)
        for k in range(X4.shape[1]):
            d2 += ((X4[:r, k, None] - X4[None, :, k]) / ls) ** 2
        blk["K"] = os_ * np.exp(np.maximum(np.float32(-0.5) * d2, np.float32(-20.0)))
    fill_s, rows4 = _row_sample_seconds(fill, n4, target_s / 8, probe=16)
    Kb = blk["K"]
    V16 = rng4.normal(size=(n4, 16)).astype(np.float32)
    t0 = time.perf_counter()
    Kb @ V16
    p16 = (time.perf_counter() - t0) * n4 / Kb.shape[0]
    Vw = rng4.normal(size=(n4, 512)).astype(np.float32)
    t0 = time.perf_counter()
    Kb @ Vw
    pw = (time.perf_counter() - t0) * n4 / Kb.shape[0] * (4096 / 512)
    cg4 = gpu.get("c4_cg_iterations") or 0
    legs["c4"] = {"cpu_fill_seconds": round(fill_s, 2),
                  "cpu_ms_per_product_16": round(p16 * 1e3, 1),
                  "gpu_ms_per_product_16": gpu.get("c4_ms_16"),
                  "cpu_seconds_per_product_4096": round(pw, 2),
                  "gpu_seconds_per_product_4096": gpu.get("c4_s_4096"),
                  "cpu_fit_seconds_extrapolated": round(p16 * cg4 + 100 * fill_s, 1) if cg4 else None,
                  "gpu_fit_seconds": gpu.get("c4_fit"),
                  "cpu_exact_variance_seconds_extrapolated": round(50 * pw, 1),
                  "gpu_exact_variance_seconds": gpu.get("c4_exact"),
                  "work": f"K rows [0,{rows4}) filled (numpy fp32, per-dimension differences) "
                          f"and multiplied by 16 and 512 columns (numpy fp32 GEMM), all "
                          f"extrapolated to N=40000 (and 4096 columns); fit = 100 fills + one "
                          f"16-column product per GPU CG iteration ({cg4}); exact variance = "
                          f"50 products of 4096 columns",
                  "kind": "port (numpy fp32)"}
    for leg in legs.values():
        leg["threads"] = threads
    return legs


def _cpu_baseline(X, V, params, noise, target_s: float):
    from oracle import cpu_ref
    threads = cpu_ref.num_threads()
    probe_rows = 256
    t0 = time.perf_counter()
    cpu_ref.forward_matvec_rows(1, True, X, params, noise, V, 0, probe_rows)
    dt = max(time.perf_counter() - t0, 1e-3)
    rows = int(min(N, max(probe_rows, target_s / dt * probe_rows)))
    t0 = time.perf_counter()
    cpu_ref.forward_matvec_rows(1, True, X, params, noise, V, 0, rows)
    dt = time.perf_counter() - t0
    flops = rows * N * FLOPS_PER_PAIR
    return {
        "value": flops / dt / 1e12,
        "unit": "TFLOP/s",
        "cores": threads,
        "cpu_model": _cpu_model(),
        "kind": "port",
        "sample": f"rows [0,{rows}) of the config-3 matvec ({rows}x{N} pairs, t={T}); "
                  f"{dt:.1f} s on {threads} threads",
    }


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="target duration of the CPU baseline sample")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--c4-only", action="store_true",
                    help="only the config-4 materialized leg (fit, exact variance, dense "
                         "products)")
    ap.add_argument("--c4-product", action="store_true",
                    help="only the config-4 16-column dense product (profiling)")
    ap.add_argument("--c4-wide", action="store_true",
                    help="only the config-4 4096-column dense product (profiling)")
    ap.add_argument("--c3-grad", action="store_true",
                    help="only the config-3 gradient trace, 16 columns (profiling)")
    ap.add_argument("--no-extras", action="store_true",
                    help="skip the mBCG-iteration and fit() measurements")
    ap.add_argument("--mbcg-only", action="store_true",
                    help="only time one mBCG iteration at configs 3 and 2 (profiling)")
    ap.add_argument("--c5-only", action="store_true",
                    help="only the config-5 LMC leg (structured product, mBCG iteration, "
                         "fit, pathwise samples)")
    ap.add_argument("--c5-product", action="store_true",
                    help="only the config-5 structured product (30 timed calls; profiling)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="BYTES",
                    help="only run the plain copy kernel of BYTES (HBM counter calibration)")
    args = ap.parse_args(argv)

    if args.calibrate_copy:
        import ctypes
        from mojogp_amd import _lib
        ms = ctypes.c_double(0.0)
        _lib.call("mgp_calibration_copy", int(args.calibrate_copy), 3, ctypes.byref(ms))
        gbs = 2 * args.calibrate_copy / (ms.value * 1e-3) / 1e9
        print(json.dumps({"calibration_copy_bytes": args.calibrate_copy,
                          "ms": ms.value, "GB/s": gbs}), flush=True)
        return 0

    if args.c4_only:
        print(json.dumps(_c4_materialized()), flush=True)
        return 0
    if args.c4_product:
        print(json.dumps(_c4_product_only()), flush=True)
        return 0
    if args.c4_wide:
        print(json.dumps(_c4_wide_product_only()), flush=True)
        return 0
    if args.c3_grad:
        print(json.dumps(_c3_gradient_trace_only()), flush=True)
        return 0
    if args.c5_product:
        print(json.dumps(_c5_product_only()), flush=True)
        return 0
    if args.c5_only:
        c5, _ = _lmc_c5(repeats=10, warmup=2)
        print(json.dumps(c5), flush=True)
        return 0
    if args.mbcg_only:
        X, _, params, noise = _make_inputs()
        c3, _ = _mbcg_iteration_ms(X, params, noise)
        print(json.dumps({"mbcg_iter_ms_c3": round(c3, 4),
                          "mbcg_iter_ms_c2": round(_mbcg_iteration_ms_c2(), 4)}), flush=True)
        return 0

    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); "
              "the multi-GPU design is described in DESIGN.md and not run here.",
              file=sys.stderr)
        return 2
    if args.steps < 1 or args.warmup < 0:
        print("--steps must be >= 1 and --warmup >= 0", file=sys.stderr)
        return 2

    from mojogp_amd._provider import NativeProvider, KIND_MATERN52

    X, V, params, noise = _make_inputs()
    prov = NativeProvider(KIND_MATERN52, True, X, params, noise)
    try:
        times_ms, tile_ms, _ = prov.benchmark_forward(V, repeats=args.steps, warmup=args.warmup)
    finally:
        prov.close()

    pairs = float(N) * float(N)
    ms_per_step = float(np.mean(times_ms))
    value = pairs * FLOPS_PER_PAIR / (ms_per_step * 1e-3) / 1e12
    achieved = pairs * FLOPS_PER_PAIR / (tile_ms * 1e-3) / 1e12
    probe = _probe()
    cycles, sym_cycles, ghz = _pipe_model(probe)
    simds = 4 * int(probe[5])
    one_tiles, sym_tiles, mfmas, kernel = _tile_counts()
    t_model_ms = (one_tiles * cycles + sym_tiles * sym_cycles) / simds / (ghz * 1e9) * 1e3
    peak = pairs * FLOPS_PER_PAIR / (t_model_ms * 1e-3) / 1e12
    mfma_tflops = mfmas * 16384 / (tile_ms * 1e-3) / 1e12

    result = {
        "metric": "fused K.V matvec TFLOP/s (N=250k, d=16, t=16, Matern-5/2 ARD)",
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (X ~ N(0,I), seed 0; 16 unit-norm random right-hand sides)",
        "config": {"workload": "config 3 forward matvec: (K + 0.1 I) V, N=250000, d=16, t=16, "
                               "Matern-5/2 ARD, lengthscales 1, outputscale 1",
                   "N": N, "d": D, "t": T},
        "roofline": {
            "bound": "mfma",
            "achieved": round(achieved, 3),
            "peak": PEAK_FP16_MFMA_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_FP16_MFMA_TFLOPS, 4),
            "traffic": TILE_TRAFFIC_BYTES["symmetric" if sym_tiles else "one_sided"],
            "peak_kind": "published MI355X dense fp16 MFMA peak; achieved counts the "
                         "algorithmic fp32-equivalent flops (F per pair x N^2)",
            "kernel": kernel,
            "issued_fp16_mfma_tflops": round(mfma_tflops, 2),
            "issued_fp16_mfma_frac": round(mfma_tflops / PEAK_FP16_MFMA_TFLOPS, 4),
            "pipe_model": {
                "what": "VALU + 16-bit MFMA cycles per 16x16 tile formed (symmetric tiles "
                        "carry 1.5 more MFMAs) from per-instruction costs measured live "
                        "(mgp_pipe_probe); the kernel is issue bound",
                "peak": round(peak, 3),
                "frac": round(t_model_ms / tile_ms, 4),
                "model_ms": round(t_model_ms, 3),
                "tiles_formed": {"one_sided": one_tiles, "symmetric": sym_tiles,
                                 "all_pairs_equivalent": ROW_TILES * COL_TILES},
                "cycles_per_tile": round(cycles, 2),
                "cycles_per_symmetric_tile": round(sym_cycles, 2),
                "instruction_cycles": {"clock_ghz": round(probe[0], 3),
                                       "v_exp_f32": round(probe[1], 2),
                                       "v_fma_f32": round(probe[2], 2),
                                       "mfma_f16_k32": round(probe[3], 2),
                                       "mfma_f16_k32_in_valu_stream": round(probe[4], 2)},
            },
        },
        "fp32_equivalent_tflops": round(achieved, 3),
        "tile_kernel_ms": round(tile_ms, 4),
    }
    if not args.no_extras:
        it_ms, _ = _mbcg_iteration_ms(X, params, noise)
        result["mbcg_iter_ms"] = round(it_ms, 3)
        result["mbcg_iter_ms_c2"] = round(_mbcg_iteration_ms_c2(), 3)
        c3_fit, c3_pred, c3_info = _c3_fit_predict_seconds()
        result["fit_seconds_c3"] = round(c3_fit, 3)
        result["predict_love_seconds_c3"] = round(c3_pred, 3)
        result["fit_c3_info"] = c3_info
        fit_s, fit_info = _fit_c2_seconds()
        result["fit_seconds"] = round(fit_s, 3)
        result["fit_config"] = ("config 2: RBF-ARD N=50000 d=8, 30 Adam steps, 15 probes, "
                                "rank-100 greedy preconditioner")
        result["fit_info"] = fit_info
        result["materialized_c4"] = _c4_materialized()
        result["fit_predict_seconds_c1"] = round(_c1_gpu_seconds(), 3)
        c5, c5_inputs = _lmc_c5(repeats=10, warmup=2)
        result["lmc_c5"] = c5
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = _cpu_baseline(X, V, params, noise, args.cpu_seconds)
        if not args.no_extras:
            result["lmc_c5"]["cpu_baseline"] = _cpu_baseline_c5(*c5_inputs, args.cpu_seconds / 2)
            c4 = result["materialized_c4"]
            gpu = {"c1": result["fit_predict_seconds_c1"],
                   "c2_fit": result["fit_seconds"],
                   "c2_cg_iterations": (result.get("fit_info") or {}).get("cg_iterations_total"),
                   "c3_mbcg_ms": result["mbcg_iter_ms"],
                   "c4_ms_16": c4["dense_matvec_ms_16"],
                   "c4_s_4096": round(c4["dense_matvec_ms_4096"] / 1e3, 4),
                   "c4_fit": c4["fit_seconds"], "c4_exact": c4["exact_variance_seconds"],
                   "c4_cg_iterations": c4["cg_iterations_total"],
                   "c4_lengthscale": c4.get("lengthscale")}
            result["cpu_baseline"]["legs"] = _cpu_legs(gpu, args.cpu_seconds)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
