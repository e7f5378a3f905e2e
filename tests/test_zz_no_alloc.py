"""The allocation-free forward matvec (mgp_forward_matvec_device_noalloc)
against the allocating one (mgp_forward_matvec_device) through the C ABI.

The allocation-free call always runs the one-sided tile kernel, so it is
compared with the allocating call on that same kernel (MGP_SYM_MATVEC=0), and
separately with the allocating call's automatic route, which above
n = 24065 is the symmetric kernel (a different summation, 1e-6 apart).
Calls in a row with decreasing inputs share one fixed scratch array that keeps
the previous call's bytes, so each call must rebuild everything it reads:
* config 3 (N = 250k, d = 16, t = 16, Matern-5/2 ARD): its split partials do
  not all fit the 64 MiB array, so fewer splits run; the product then differs
  from the one-sided allocating call's by summation order only (<= 1e-6);
* N = 30000, d = 8, t = 16 (above the symmetric threshold): same splits as
  the one-sided allocating call, bit-identical output;
* N = 20000, d = 8, t = 16: same splits, bit-identical output;
* N = 3000, d = 5, t = 5, RBF with a fixed noise vector: bit-identical.
An input whose packed right-hand sides exceed the array is rejected before any
launch, free device memory is unchanged across an allocation-free call on a
fresh provider (whose own workspace would otherwise grow on first use), and
calls from two threads on two providers -- which share the device's array --
give each its own sequential result bit for bit (a per-device lock orders
them).
Device buffers for inputs and outputs come from the HIP runtime the library
itself loaded, through ctypes.
"""

import ctypes as C
import os
import sys
import threading

import numpy as np
import pytest

from mojogp_amd import _lib
from mojogp_amd._provider import KIND_MATERN52, KIND_RBF, NativeProvider

pytestmark = pytest.mark.gpu

_H2D, _D2H = 1, 2


def _log(msg):
    print(msg, flush=True)
    sys.__stderr__.write(msg + "\n")
    sys.__stderr__.flush()


def _hip():
    """The libamdhip64 already mapped into this process by the library."""
    _lib.load()
    with open("/proc/self/maps") as f:
        paths = sorted({ln.split()[-1] for ln in f if "libamdhip64.so" in ln})
    assert paths, "libamdhip64 is not loaded"
    h = C.CDLL(paths[0])
    h.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
    h.hipFree.argtypes = [C.c_void_p]
    h.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    h.hipMemGetInfo.argtypes = [C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]
    h.hipDeviceSynchronize.argtypes = []
    for fn in (h.hipMalloc, h.hipFree, h.hipMemcpy, h.hipMemGetInfo, h.hipDeviceSynchronize):
        fn.restype = C.c_int
    return h


class _Dev:
    """One device buffer of nbytes."""

    def __init__(self, hip, nbytes):
        self.hip, self.nbytes = hip, int(nbytes)
        self.ptr = C.c_void_p()
        assert hip.hipMalloc(C.byref(self.ptr), self.nbytes) == 0

    def put(self, a):
        a = np.ascontiguousarray(a)
        assert a.nbytes == self.nbytes
        assert self.hip.hipMemcpy(self.ptr, a.ctypes.data, a.nbytes, _H2D) == 0

    def get(self, shape):
        out = np.empty(shape, np.float32)
        assert out.nbytes == self.nbytes
        assert self.hip.hipMemcpy(out.ctypes.data, self.ptr, out.nbytes, _D2H) == 0
        return out

    def free(self):
        if self.ptr.value:
            self.hip.hipFree(self.ptr)
            self.ptr = C.c_void_p()


def _free_mem(hip):
    fr, tot = C.c_size_t(), C.c_size_t()
    assert hip.hipDeviceSynchronize() == 0
    assert hip.hipMemGetInfo(C.byref(fr), C.byref(tot)) == 0
    return fr.value


def _allocating(prov, src, dst, t, sym):
    """mgp_forward_matvec_device with the symmetric route allowed or not."""
    old = os.environ.get("MGP_SYM_MATVEC")
    try:
        if sym:
            os.environ.pop("MGP_SYM_MATVEC", None)
        else:
            os.environ["MGP_SYM_MATVEC"] = "0"
        _lib.call("mgp_forward_matvec_device", prov.handle, src.ptr, t, dst.ptr)
    finally:
        if old is None:
            os.environ.pop("MGP_SYM_MATVEC", None)
        else:
            os.environ["MGP_SYM_MATVEC"] = old


def _case(hip, kind, n, d, t, seed, noise_vec=False, check_memory=False):
    """(no-alloc output, one-sided allocating output, automatic-route output)."""
    rng = np.random.default_rng(seed)
    X = rng.normal(size=(n, d)).astype(np.float32)
    V = rng.normal(size=(t, n)).astype(np.float32)
    params = np.concatenate([rng.uniform(0.7, 1.4, size=d), [1.1]]).astype(np.float32)
    nbytes = 4 * n * t
    _log(f"no-alloc case: kind {kind} n={n} d={d} t={t} seed {seed} noise_vec={noise_vec}")
    prov = NativeProvider(kind, True, X, params, 0.1)
    bufs = [_Dev(hip, nbytes) for _ in range(3)]
    try:
        if noise_vec:
            nv = rng.uniform(0.05, 0.2, size=n).astype(np.float32)
            _lib.call("mgp_set_noise_vector", prov.handle, _lib.fptr(nv))
        bufs[0].put(V)
        # sentinel contents: the no-alloc output must overwrite every entry
        bufs[2].put(np.full((t, n), np.nan, np.float32))
        before = _free_mem(hip)
        _lib.call("mgp_forward_matvec_device_noalloc", prov.handle, bufs[0].ptr, t, bufs[2].ptr)
        after = _free_mem(hip)
        got = bufs[2].get((t, n))
        _allocating(prov, bufs[0], bufs[1], t, sym=False)
        ref = bufs[1].get((t, n))
        grown = before - _free_mem(hip)
        _allocating(prov, bufs[0], bufs[1], t, sym=True)
        auto = bufs[1].get((t, n))
        if check_memory:
            _log(f"  free memory: no-alloc call {before - after} B, allocating call {grown} B")
            assert abs(before - after) < (1 << 20)
        assert np.all(np.isfinite(got))
        return got, ref, auto
    finally:
        for b in bufs:
            b.free()
        prov.close()


def _colrel(a, b):
    return float(np.max(np.linalg.norm(a - b, axis=1) / np.linalg.norm(b, axis=1)))


def test_noalloc_matches_allocating_entry_point():
    hip = _hip()
    got, ref, auto = _case(hip, KIND_MATERN52, 250_000, 16, 16, 0, check_memory=True)
    _log(f"  config 3: vs one-sided {_colrel(got, ref):.2e}, vs symmetric {_colrel(got, auto):.2e}")
    assert _colrel(got, ref) <= 1e-6       # fewer splits: summation order only
    assert _colrel(got, auto) <= 5e-6      # the symmetric kernel's own summation
    got, ref, auto = _case(hip, KIND_MATERN52, 30_000, 8, 16, 4)
    _log(f"  n=30000: vs symmetric {_colrel(got, auto):.2e}")
    np.testing.assert_array_equal(got, ref)
    assert _colrel(got, auto) <= 5e-6
    got, ref, _ = _case(hip, KIND_MATERN52, 20_000, 8, 16, 1)
    np.testing.assert_array_equal(got, ref)
    got, ref, _ = _case(hip, KIND_RBF, 3000, 5, 5, 2, noise_vec=True)
    np.testing.assert_array_equal(got, ref)


def test_noalloc_calls_from_two_threads_are_ordered():
    """Two providers on one GPU share its scratch array; calls from two threads
    (ctypes releases the GIL during the call) must each reproduce their own
    sequential result bit for bit."""
    hip = _hip()
    rng = np.random.default_rng(9)
    jobs = []
    for n, d, t, kind in ((20_000, 8, 16, KIND_MATERN52), (12_000, 4, 8, KIND_RBF)):
        X = rng.normal(size=(n, d)).astype(np.float32)
        V = rng.normal(size=(t, n)).astype(np.float32)
        params = np.concatenate([rng.uniform(0.7, 1.4, size=d), [1.1]]).astype(np.float32)
        prov = NativeProvider(kind, True, X, params, 0.1)
        src, dst = _Dev(hip, 4 * n * t), _Dev(hip, 4 * n * t)
        src.put(V)
        jobs.append((prov, src, dst, t, n))
    try:
        seq = []
        for prov, src, dst, t, n in jobs:
            _lib.call("mgp_forward_matvec_device_noalloc", prov.handle, src.ptr, t, dst.ptr)
            seq.append(dst.get((t, n)))
        _log("no-alloc threads: two providers, 6 calls each")
        errors = []

        def run(k):
            prov, src, dst, t, n = jobs[k]
            try:
                for _ in range(6):
                    _lib.call("mgp_forward_matvec_device_noalloc", prov.handle, src.ptr, t,
                              dst.ptr)
                    if not np.array_equal(dst.get((t, n)), seq[k]):
                        errors.append(f"provider {k}: output differs from its sequential call")
            except Exception as exc:  # reported after the join
                errors.append(f"provider {k}: {exc}")

        threads = [threading.Thread(target=run, args=(k,)) for k in range(2)]
        for th in threads:
            th.start()
        for th in threads:
            th.join(timeout=120)
        assert not any(th.is_alive() for th in threads)
        assert not errors, errors
    finally:
        for prov, src, dst, _, _ in jobs:
            src.free()
            dst.free()
            prov.close()


def test_noalloc_rejects_inputs_beyond_the_scratch():
    hip = _hip()
    n, d, t = 300_000, 2, 64      # packed right-hand sides: ~77 MB > 64 MiB
    rng = np.random.default_rng(3)
    X = rng.normal(size=(n, d)).astype(np.float32)
    prov = NativeProvider(KIND_RBF, False, X, np.array([1.0, 1.0], np.float32), 0.1)
    bufs = [_Dev(hip, 4 * n * t) for _ in range(2)]
    try:
        with pytest.raises(_lib.NativeCallError, match="at most 67108864"):
            _lib.call("mgp_forward_matvec_device_noalloc", prov.handle, bufs[0].ptr, t,
                      bufs[1].ptr)
    finally:
        for b in bufs:
            b.free()
        prov.close()
