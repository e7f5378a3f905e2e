"""Python handle over a native device-resident kernel provider."""

from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib

KIND_RBF = 0
KIND_MATERN52 = 1
KIND_MATERN12 = 2
KIND_MATERN32 = 3
_KIND_NAMES = {"rbf": KIND_RBF, "matern52": KIND_MATERN52, "matern12": KIND_MATERN12,
               "matern32": KIND_MATERN32}


# Provider kind reported for composite kernel trees.
TREE_KIND = -1


def kind_code(kind) -> int:
    if isinstance(kind, str):
        try:
            return _KIND_NAMES[kind.lower()]
        except KeyError:
            raise ValueError(f"unsupported kernel kind {kind!r}") from None
    return int(kind)


def _cols(V: np.ndarray, n: int) -> tuple[np.ndarray, bool]:
    """Normalise right-hand sides to column-major [ncols][n] float32."""
    V = _lib.f32(V)
    if V.ndim == 1:
        if V.shape[0] != n:
            raise ValueError(f"vector has length {V.shape[0]}, expected {n}")
        return V.reshape(1, n), True
    if V.ndim != 2 or V.shape[1] != n:
        raise ValueError(f"right-hand sides must have shape (ncols, {n}), got {V.shape}")
    return V, False


class NativeProvider:
    """Owns one ``mgp_init_provider`` handle (training inputs live in HBM)."""

    def __init__(self, kind, ard: bool, X: np.ndarray, params: np.ndarray, noise: float,
                 tree_spec=None):
        """``tree_spec``: flat kernel-tree spec (``KernelNode.to_tree_spec``);
        ``kind`` and ``ard`` are then ignored."""
        X = _lib.f32(X)
        if X.ndim != 2:
            raise ValueError("X must be 2-D")
        params = _lib.f32(params).ravel()
        self.n, self.d = X.shape
        self.nparams = params.shape[0]
        h = C.c_void_p()
        if tree_spec is not None:
            spec = np.ascontiguousarray(np.asarray(tree_spec, dtype=np.int32).ravel())
            self.kind, self.ard, self.tree_spec = TREE_KIND, False, spec
            _lib.call("mgp_init_provider_tree", spec.ctypes.data_as(C.POINTER(C.c_int)),
                      int(spec.size), self.d, self.n, _lib.fptr(X), _lib.fptr(params),
                      self.nparams, float(noise), C.byref(h))
        else:
            self.kind = kind_code(kind)
            self.ard = bool(ard)
            self.tree_spec = None
            _lib.call("mgp_init_provider", self.kind, int(self.ard), self.d, self.n,
                      _lib.fptr(X), _lib.fptr(params), self.nparams, float(noise),
                      C.byref(h))
        self._h = h
        self.params = params.copy()
        self.noise = float(noise)

    @property
    def handle(self) -> C.c_void_p:
        if self._h is None or not self._h.value:
            raise RuntimeError("provider has been destroyed")
        return self._h

    def close(self) -> None:
        if getattr(self, "_h", None) is not None and self._h.value:
            _lib.call("mgp_destroy_provider", self._h)
        self._h = None

    def __del__(self):  # pragma: no cover - best effort
        try:
            self.close()
        except Exception:
            pass

    def update_params(self, params) -> None:
        params = _lib.f32(params).ravel()
        _lib.call("mgp_update_params", self.handle, _lib.fptr(params), params.shape[0])
        self.params = params.copy()

    def update_noise(self, noise: float) -> None:
        _lib.call("mgp_update_noise", self.handle, float(noise))
        self.noise = float(noise)

    def set_noise_vector(self, noise_vec) -> None:
        """Fixed per-point noise variances [n] (K + diag(noise_vec)), or None."""
        if noise_vec is None:
            _lib.call("mgp_set_noise_vector", self.handle, None)
            self.noise_vec = None
            return
        v = _lib.f32(noise_vec).ravel()
        if v.shape != (self.n,):
            raise ValueError(f"noise vector must have shape ({self.n},), got {v.shape}")
        _lib.call("mgp_set_noise_vector", self.handle, _lib.fptr(v))
        self.noise_vec = v.copy()

    def set_categorical_params(self, kinds, raw) -> None:
        """Correlation tables of the categorical leaves (tree order) from raw
        parameters (kinds: 0 GD, 1 CR, 2 EHH, 3 HH, 4 FE)."""
        k = np.ascontiguousarray(np.asarray(kinds, dtype=np.int32).ravel())
        r = _lib.f32(raw).ravel()
        _lib.call("mgp_set_categorical_params", self.handle, k.ctypes.data_as(C.POINTER(C.c_int)),
                  int(k.size), _lib.fptr(r), int(r.size))

    def set_learned_noise(self, mode: int, group_ids=None, num_groups=None) -> None:
        """Learned per-point noise for training (modes 2 per point, 3 per group,
        4 linear in the inputs; 0 clears).  The current noise vector is the
        initial state."""
        gp_ = None
        ng = 0
        if int(mode) == 3:
            if group_ids is None:
                raise ValueError("grouped noise needs group ids")
            g = np.ascontiguousarray(np.asarray(group_ids, dtype=np.int32).ravel())
            if g.shape != (self.n,):
                raise ValueError(f"group ids must have shape ({self.n},)")
            ng = int(num_groups) if num_groups is not None else int(g.max()) + 1
            self._groups = g
            gp_ = g.ctypes.data_as(C.POINTER(C.c_int))
        _lib.call("mgp_set_learned_noise", self.handle, int(mode), gp_, ng)

    def forward_matvec(self, V) -> np.ndarray:
        Vc, vec = _cols(V, self.n)
        out = np.empty_like(Vc)
        _lib.call("mgp_forward_matvec", self.handle, _lib.fptr(Vc), Vc.shape[0],
                  _lib.fptr(out))
        return out[0] if vec else out

    def direct_matvec(self, V) -> np.ndarray:
        Vc, vec = _cols(V, self.n)
        out = np.empty_like(Vc)
        _lib.call("mgp_direct_matvec", self.handle, _lib.fptr(Vc), Vc.shape[0],
                  _lib.fptr(out))
        return out[0] if vec else out

    def materialize(self) -> None:
        """Switch to the dense-K route (K held on the device, 4 n^2 bytes)."""
        _lib.call("mgp_materialize", self.handle)

    def cross_matvec(self, Xs, V) -> np.ndarray:
        Xs = _lib.f32(Xs)
        if Xs.ndim != 2 or Xs.shape[1] != self.d:
            raise ValueError(f"test inputs must have shape (m, {self.d})")
        Vc, vec = _cols(V, self.n)
        m = Xs.shape[0]
        out = np.empty((Vc.shape[0], m), dtype=np.float32)
        _lib.call("mgp_cross_matvec", self.handle, _lib.fptr(Xs), m, _lib.fptr(Vc),
                  Vc.shape[0], _lib.fptr(out))
        return out[0] if vec else out

    def extract_diagonal(self) -> np.ndarray:
        out = np.empty(self.n, dtype=np.float32)
        _lib.call("mgp_extract_diagonal", self.handle, _lib.fptr(out))
        return out

    def benchmark_forward(self, V, repeats: int, warmup: int):
        """(per-call wall ms array, mean tile-kernel ms, output)."""
        return self.benchmark_op(V, 0, repeats, warmup)

    def benchmark_op(self, V, op: int, repeats: int, warmup: int):
        """benchmark_provider_ops: op 0 forward, 1 gradient products, 2 gradient
        products + dots, 3 dots only.  Returns (wall ms per call, mean tile ms
        (op 0), last output ([C, n] for op 0, [P, C, n] otherwise))."""
        Vc, _ = _cols(V, self.n)
        times = np.zeros(repeats, dtype=np.float64)
        tile = C.c_double(0.0)
        shape = Vc.shape if op == 0 else (self.nparams,) + Vc.shape
        out = np.empty(shape, dtype=np.float32)
        _lib.call("mgp_benchmark_provider_ops", self.handle, _lib.fptr(Vc), Vc.shape[0],
                  int(op), int(repeats), int(warmup), _lib.dptr(times), C.byref(tile),
                  _lib.fptr(out))
        return times, float(tile.value), out

    def gradient_trace(self, Lf, Rf) -> np.ndarray:
        """g[p] = sum_ab dK_p[a, b] sum_c Lf[c, a] Rf[c, b] (float64, [P]): the
        BBMM gradient step's trace routine on given weight columns."""
        L, _ = _cols(Lf, self.n)
        R, _ = _cols(Rf, self.n)
        if L.shape != R.shape:
            raise ValueError("Lf and Rf must have the same shape")
        out = np.zeros(self.nparams, dtype=np.float64)
        _lib.call("mgp_gradient_trace", self.handle, _lib.fptr(L), _lib.fptr(R), L.shape[0],
                  _lib.dptr(out))
        return out

    def gradient_matvec(self, V) -> np.ndarray:
        """out[p, c, i] = sum_j dk_p(x_i, x_j) V[c, j] for the P engine parameters."""
        Vc, vec = _cols(V, self.n)
        out = np.empty((self.nparams, Vc.shape[0], self.n), dtype=np.float32)
        _lib.call("mgp_gradient_matvec", self.handle, _lib.fptr(Vc), Vc.shape[0],
                  _lib.fptr(out))
        return out[:, 0, :] if vec else out
