"""Kernel specification surface (subset served by the gfx950 engine).

Mirrors the reference's kernel DSL for the hot-path kernels
(mojogp/kernel.py): ``RBF``, ``Matern12``, ``Matern32`` and ``Matern52``,
isotropic or ARD, with the same
parameter names, initial values and engine parameter layout
(``kernel.py:324-509``):

  isotropic  [lengthscale, outputscale]
  ARD        [ls_0 .. ls_{d-1}, outputscale]

Composite trees (sum / product / scale) and the other kernel families are
accepted for construction and serialisation but the engine rejects them at
``fit`` time: they are outside the accelerated path.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from enum import Enum
from typing import Any, Dict, List, Optional

import numpy as np


class KernelType(Enum):
    RBF = "RBFComposable"
    MATERN12 = "Matern12Composable"
    MATERN32 = "Matern32Composable"
    MATERN52 = "Matern52Composable"
    PERIODIC = "PeriodicComposable"
    LINEAR = "LinearComposable"
    RQ = "RQComposable"
    POLYNOMIAL = "PolynomialComposable"


# Families the native kernels implement (value = native kind code).
NATIVE_KINDS = {KernelType.RBF: 0, KernelType.MATERN52: 1, KernelType.MATERN12: 2,
                KernelType.MATERN32: 3}


@dataclass
class KernelNode:
    kernel_type: Optional[KernelType] = None
    operator: Optional[str] = None
    left: Optional["KernelNode"] = None
    right: Optional["KernelNode"] = None
    scale_factor: Optional[float] = None
    ard_dim: Optional[int] = None
    initial_values: Optional[Dict[str, float]] = None
    ard: bool = False
    active_dims: Optional[tuple] = None

    # ---------------------------------------------------------- composition
    def __add__(self, other: "KernelNode") -> "KernelNode":
        return KernelNode(operator="sum", left=self, right=other)

    def __mul__(self, other):
        if isinstance(other, (int, float)):
            return KernelNode(operator="scale", left=self, scale_factor=float(other))
        return KernelNode(operator="product", left=self, right=other)

    def __rmul__(self, other):
        return self.__mul__(other)

    # ---------------------------------------------------------- structure
    def has_ard(self) -> bool:
        if self.ard:
            return True
        return bool((self.left and self.left.has_ard()) or (self.right and self.right.has_ard()))

    def is_native_leaf(self) -> bool:
        return self.kernel_type in NATIVE_KINDS and self.operator is None and self.active_dims is None

    def native_kind(self) -> int:
        if not self.is_native_leaf():
            raise NotImplementedError(
                f"kernel {self!r} is outside the gfx950 engine (supported: RBF, Matern12, "
                "Matern32, Matern52, "
                "isotropic or ARD, no composition / active_dims)")
        return NATIVE_KINDS[self.kernel_type]

    def num_params(self) -> int:
        if self.kernel_type is not None:
            if self.ard_dim is not None:
                if self.kernel_type in (KernelType.PERIODIC, KernelType.RQ):
                    return self.ard_dim + 2
                if self.kernel_type == KernelType.POLYNOMIAL:
                    return self.ard_dim + 3
                return self.ard_dim + 1
            if self.kernel_type in (KernelType.PERIODIC, KernelType.RQ, KernelType.POLYNOMIAL):
                return 3
            return 2
        if self.operator in ("sum", "product"):
            return self.left.num_params() + self.right.num_params()
        if self.operator == "scale":
            return self.left.num_params() + 1
        raise ValueError(f"Unknown operator: {self.operator}")

    def get_param_names(self, prefix: str = "") -> List[str]:
        if self.kernel_type is not None:
            base = self.kernel_type.name.lower()
            if prefix:
                base = f"{prefix}_{base}"
            if self.ard_dim is not None:
                names = [f"{base}_ls_{d}" for d in range(self.ard_dim)]
                if self.kernel_type == KernelType.PERIODIC:
                    names.append(f"{base}_period")
                elif self.kernel_type == KernelType.RQ:
                    names.append(f"{base}_alpha")
                elif self.kernel_type == KernelType.POLYNOMIAL:
                    names += [f"{base}_degree", f"{base}_offset"]
                names.append(f"{base}_outputscale")
                return names
            if self.kernel_type == KernelType.POLYNOMIAL:
                return [f"{base}_degree", f"{base}_offset", f"{base}_outputscale"]
            if self.kernel_type == KernelType.LINEAR:
                return [f"{base}_variance", f"{base}_outputscale"]
            if self.kernel_type in (KernelType.PERIODIC, KernelType.RQ):
                extra = "period" if self.kernel_type == KernelType.PERIODIC else "alpha"
                return [f"{base}_lengthscale", f"{base}_{extra}", f"{base}_outputscale"]
            return [f"{base}_lengthscale", f"{base}_outputscale"]
        if self.operator in ("sum", "product"):
            return (self.left.get_param_names(f"{prefix}left" if prefix else "left")
                    + self.right.get_param_names(f"{prefix}right" if prefix else "right"))
        if self.operator == "scale":
            return self.left.get_param_names(prefix) + [f"{prefix}_scale" if prefix else "scale"]
        raise ValueError(f"Unknown operator: {self.operator}")

    def get_initial_params(self) -> np.ndarray:
        """Initial values matched by name suffix, default 1.0.

        As in the reference (kernel.py:631-660) an ARD leaf's ``ls_d`` names do
        not match the ``lengthscale`` key, so ARD lengthscales start at 1.0."""
        values = np.ones(self.num_params(), dtype=np.float32)
        self._fill_initial(values, 0)
        return values

    def _fill_initial(self, values: np.ndarray, offset: int) -> int:
        if self.kernel_type is not None:
            n = self.num_params()
            if self.initial_values:
                for i, name in enumerate(self.get_param_names()):
                    for key, val in self.initial_values.items():
                        if name.endswith(f"_{key}") or name == key:
                            values[offset + i] = val
                            break
            return offset + n
        if self.operator in ("sum", "product"):
            return self.right._fill_initial(values, self.left._fill_initial(values, offset))
        if self.operator == "scale":
            mid = self.left._fill_initial(values, offset)
            if self.initial_values and "scale" in self.initial_values:
                values[mid] = self.initial_values["scale"]
            elif self.scale_factor is not None:
                values[mid] = self.scale_factor
            return mid + 1
        return offset

    def to_engine_params(self, public_params) -> np.ndarray:
        p = np.asarray(public_params, dtype=np.float32)
        if p.shape != (self.num_params(),):
            raise ValueError(f"public_params must have shape ({self.num_params()},), got {p.shape}")
        return p.copy()

    def from_engine_params(self, engine_params) -> np.ndarray:
        p = np.asarray(engine_params, dtype=np.float32)
        if p.shape != (self.num_params(),):
            raise ValueError(f"engine_params must have shape ({self.num_params()},), got {p.shape}")
        return p.copy()

    # ---------------------------------------------------------- serialisation
    # Type names written into saved model configs ("kernel_mojo_type"); the
    # strings are the reference's (kernel.py:273-321) so saved files match.
    _ARD_TYPE_NAMES = {
        KernelType.RBF: "RBFComposableARD", KernelType.MATERN12: "Matern12ComposableARD",
        KernelType.MATERN32: "Matern32ComposableARD",
        KernelType.MATERN52: "Matern52ComposableARD",
        KernelType.PERIODIC: "PeriodicComposableARD", KernelType.RQ: "RQComposableARD",
        KernelType.LINEAR: "LinearComposableARD",
        KernelType.POLYNOMIAL: "PolynomialComposableARD",
    }

    def to_mojo_type(self) -> str:
        if self.kernel_type is not None:
            if self.ard_dim is not None:
                return f"{self._ARD_TYPE_NAMES[self.kernel_type]}[{self.ard_dim}]"
            return self.kernel_type.value
        if self.operator == "sum":
            return f"SumKernel[{self.left.to_mojo_type()}, {self.right.to_mojo_type()}]"
        if self.operator == "product":
            return f"ProductKernel[{self.left.to_mojo_type()}, {self.right.to_mojo_type()}]"
        if self.operator == "scale":
            return f"ScaleKernel[{self.left.to_mojo_type()}]"
        raise ValueError(f"Unknown operator: {self.operator}")

    def to_dict(self) -> Dict[str, Any]:
        d: Dict[str, Any] = {}
        if self.kernel_type is not None:
            d["kernel_type"] = self.kernel_type.name
        if self.operator is not None:
            d["operator"] = self.operator
        if self.left is not None:
            d["left"] = self.left.to_dict()
        if self.right is not None:
            d["right"] = self.right.to_dict()
        if self.scale_factor is not None:
            d["scale_factor"] = self.scale_factor
        if self.ard_dim is not None:
            d["ard_dim"] = self.ard_dim
        if self.initial_values is not None:
            d["initial_values"] = self.initial_values
        if self.ard:
            d["ard"] = True
        if self.active_dims is not None:
            d["active_dims"] = list(self.active_dims)
        return d

    @staticmethod
    def from_dict(d: Dict[str, Any]) -> "KernelNode":
        return KernelNode(
            kernel_type=KernelType[d["kernel_type"]] if "kernel_type" in d else None,
            operator=d.get("operator"),
            left=KernelNode.from_dict(d["left"]) if "left" in d else None,
            right=KernelNode.from_dict(d["right"]) if "right" in d else None,
            scale_factor=d.get("scale_factor"),
            ard_dim=d.get("ard_dim"),
            initial_values=d.get("initial_values"),
            ard=d.get("ard", False),
            active_dims=tuple(d["active_dims"]) if "active_dims" in d else None,
        )

    # ---------------------------------------------------------- evaluation
    def evaluate(self, X, X2=None, params=None) -> np.ndarray:
        """K(X, X2) in float64 arithmetic, returned as float32 (kernel.py:722-923)."""
        X = np.asarray(X, dtype=np.float64)
        X2 = X if X2 is None else np.asarray(X2, dtype=np.float64)
        p = np.ones(self.num_params()) if params is None else np.asarray(params, np.float64)
        if self.kernel_type not in (KernelType.RBF, KernelType.MATERN12, KernelType.MATERN32,
                                    KernelType.MATERN52) or self.operator is not None:
            raise NotImplementedError("evaluate() covers RBF and Matern leaves")
        if self.ard_dim is not None:
            ls, extra = p[: self.ard_dim], self.ard_dim
        else:
            ls, extra = np.array([p[0]]), 1
        A, B = X / ls, X2 / ls
        sq = (np.sum(A * A, 1)[:, None] + np.sum(B * B, 1)[None, :] - 2 * A @ B.T)
        sq = np.maximum(sq, 0.0)
        dist = np.sqrt(sq + 1e-20)
        os = p[extra]
        if self.kernel_type == KernelType.RBF:
            K = os * np.exp(-0.5 * sq)
        elif self.kernel_type == KernelType.MATERN12:
            K = os * np.exp(-dist)
        elif self.kernel_type == KernelType.MATERN32:
            K = os * (1 + np.sqrt(3.0) * dist) * np.exp(-np.sqrt(3.0) * dist)
        else:
            K = os * (1 + np.sqrt(5.0) * dist + 5.0 / 3.0 * sq) * np.exp(-np.sqrt(5.0) * dist)
        return K.astype(np.float32)

    def __repr__(self) -> str:
        if self.kernel_type is not None:
            tag = "ARD" if (self.ard or self.ard_dim is not None) else ""
            return f"{self.kernel_type.name}{tag}()"
        if self.operator == "scale":
            return f"{self.scale_factor} * {self.left!r}"
        sym = "+" if self.operator == "sum" else "*"
        return f"({self.left!r} {sym} {self.right!r})"


def make_ard_kernel(kernel: KernelNode, dim: int) -> KernelNode:
    """Resolve ARD leaves to ``dim`` per-dimension lengthscales (kernel.py:1520-1583)."""
    if kernel.kernel_type is not None:
        ard_dim = len(kernel.active_dims) if kernel.active_dims is not None else dim
        return KernelNode(kernel_type=kernel.kernel_type, ard_dim=ard_dim,
                          initial_values=kernel.initial_values, ard=kernel.ard,
                          active_dims=kernel.active_dims)
    return KernelNode(operator=kernel.operator,
                      left=make_ard_kernel(kernel.left, dim) if kernel.left else None,
                      right=make_ard_kernel(kernel.right, dim) if kernel.right else None,
                      scale_factor=kernel.scale_factor, active_dims=kernel.active_dims)


def _leaf(kt: KernelType, ard: bool, active_dims, **init) -> KernelNode:
    return KernelNode(kernel_type=kt, ard=ard, initial_values=dict(init),
                      active_dims=tuple(sorted(active_dims)) if active_dims is not None else None)


def RBF(lengthscale: float = 1.0, outputscale: float = 1.0, ard: bool = False,
        active_dims: Optional[List[int]] = None) -> KernelNode:
    return _leaf(KernelType.RBF, ard, active_dims, lengthscale=lengthscale, outputscale=outputscale)


def Matern52(lengthscale: float = 1.0, outputscale: float = 1.0, ard: bool = False,
             active_dims: Optional[List[int]] = None) -> KernelNode:
    return _leaf(KernelType.MATERN52, ard, active_dims, lengthscale=lengthscale,
                 outputscale=outputscale)


def Matern32(lengthscale: float = 1.0, outputscale: float = 1.0, ard: bool = False,
             active_dims: Optional[List[int]] = None) -> KernelNode:
    return _leaf(KernelType.MATERN32, ard, active_dims, lengthscale=lengthscale,
                 outputscale=outputscale)


def Matern12(lengthscale: float = 1.0, outputscale: float = 1.0, ard: bool = False,
             active_dims: Optional[List[int]] = None) -> KernelNode:
    return _leaf(KernelType.MATERN12, ard, active_dims, lengthscale=lengthscale,
                 outputscale=outputscale)
