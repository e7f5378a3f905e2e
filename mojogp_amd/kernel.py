"""Kernel specification surface served by the gfx950 engine.

Mirrors the reference's kernel DSL (mojogp/kernel.py): ``RBF``, ``Matern12``,
``Matern32``, ``Matern52``, ``RQ`` and ``Periodic`` leaves, isotropic or ARD,
optionally restricted to ``active_dims``, composed with ``+`` (sum), ``*``
(product) and ``c * K`` (scale), with the reference's parameter names, initial
values and parameter layout (``kernel.py:324-660``):

  RBF / Matern   [lengthscale | ls_0 .. ls_{q-1}], outputscale
  RQ             [lengthscale | ls_0 .. ls_{q-1}], alpha, outputscale
  Periodic       [lengthscale | ls_0 .. ls_{q-1}], period, outputscale
  sum / product  left params, then right params
  scale          inner params, then the scale factor

A single RBF / Matern leaf on all input dimensions runs on the fused MFMA
tile path; every other tree is compiled by ``to_tree_spec`` into the flat
integer form the native kernel-tree products take.  ``Linear`` and
``Polynomial`` leaves are accepted for construction and serialisation but
rejected at ``fit`` time (non-stationary leaves are outside the served path).
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
    GD = "GDCategorical"
    CR = "CRCategorical"
    EHH = "EHHCategorical"
    HH = "HHCategorical"
    FE = "FECategorical"


# Categorical families (kernel.py:63-69 parameter counts; native kind codes of
# the mixed training entry point: 0 GD, 1 CR, 2 EHH, 3 HH, 4 FE).
CATEGORICAL_KINDS = {KernelType.GD: 0, KernelType.CR: 1, KernelType.EHH: 2, KernelType.HH: 3,
                     KernelType.FE: 4}
_CAT_PARAM_COUNTS = {
    KernelType.GD: lambda L: 1,
    KernelType.CR: lambda L: L,
    KernelType.EHH: lambda L: L * (L - 1) // 2,
    KernelType.HH: lambda L: L * (L - 1) // 2,
    KernelType.FE: lambda L: L * (L + 1) // 2,
}


def _inv_softplus(x: float) -> float:
    return float(np.log(np.expm1(x)))


def _inv_sigmoid(x: float) -> float:
    return float(np.log(x / (1.0 - x)))


def cat_default_raw_param(kernel_type: KernelType, param_index: int, L: int) -> float:
    """Default raw categorical parameter (kernel.py:84-101)."""
    if kernel_type == KernelType.GD:
        return _inv_softplus(0.5)
    if kernel_type == KernelType.CR:
        return _inv_softplus(0.3)
    if kernel_type in (KernelType.EHH, KernelType.HH):
        return _inv_sigmoid(0.25)
    if kernel_type == KernelType.FE:
        return _inv_sigmoid(0.25) if param_index < L * (L - 1) // 2 else _inv_softplus(0.3)
    return 0.0


def cat_raw_from_constrained(kernel_type: KernelType, L: int, theta) -> np.ndarray:
    """Raw parameters of one categorical leaf from its constrained values: the
    inverse of the transforms of categorical_prediction_params
    (kernel.py:132-174): softplus for GD / CR and the FE diagonal, pi *
    sigmoid for the EHH / HH angles and the first L(L-1)/2 FE entries.  Angles
    are kept inside (0, pi) by 1e-7 of a half-turn."""
    th = np.asarray(theta, np.float64).ravel()
    n_angles = {KernelType.EHH: len(th), KernelType.HH: len(th),
                KernelType.FE: L * (L - 1) // 2}.get(kernel_type, 0)
    out = np.empty_like(th)
    u = np.clip(th[:n_angles] / np.pi, 1e-7, 1.0 - 1e-7)
    out[:n_angles] = np.log(u / (1.0 - u))
    v = np.maximum(th[n_angles:], 1e-30)
    out[n_angles:] = np.where(v > 20.0, v, np.log(np.expm1(np.minimum(v, 20.0))))
    return out.astype(np.float32)


# Families the native kernels implement (value = native kind code).
NATIVE_KINDS = {KernelType.RBF: 0, KernelType.MATERN52: 1, KernelType.MATERN12: 2,
                KernelType.MATERN32: 3}
# Leaf codes of the kernel-tree spec (radial kinds keep their codes).
TREE_LEAF_CODES = {**NATIVE_KINDS, KernelType.RQ: 4, KernelType.PERIODIC: 5,
                   KernelType.LINEAR: 7, KernelType.POLYNOMIAL: 8}
_CAT_LEAF_CODE = 6
_TN_LEAF, _TN_ADD, _TN_MUL, _TN_SCALE = 0, 1, 2, 3


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
    levels: Optional[int] = None  # categorical leaves

    # ---------------------------------------------------------- composition
    def __add__(self, other: "KernelNode") -> "KernelNode":
        return KernelNode(operator="sum", left=self, right=other)

    def __radd__(self, other):
        if isinstance(other, (int, float)) and other == 0:
            return self  # sum() starts from 0
        return KernelNode(operator="sum", left=other, right=self)

    def with_active_dims(self, dims) -> "KernelNode":
        """Copy of this (possibly composite) kernel restricted to ``dims``
        (kernel.py:224-242); leaves inside without their own active_dims see
        exactly these input columns."""
        import copy
        node = copy.deepcopy(self)
        node.active_dims = tuple(sorted(int(x) for x in dims))
        return node

    def has_active_dims(self) -> bool:
        return bool(self.active_dims is not None
                    or (self.left and self.left.has_active_dims())
                    or (self.right and self.right.has_active_dims()))

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

    def is_categorical(self) -> bool:
        return self.kernel_type in CATEGORICAL_KINDS

    def has_categorical(self) -> bool:
        if self.kernel_type is not None:
            return self.is_categorical()
        return bool((self.left and self.left.has_categorical())
                    or (self.right and self.right.has_categorical()))

    def categorical_leaves(self) -> List["KernelNode"]:
        """Categorical leaves in tree order."""
        if self.kernel_type is not None:
            return [self] if self.is_categorical() else []
        out = self.left.categorical_leaves() if self.left else []
        return out + (self.right.categorical_leaves() if self.right else [])

    def structural_degree(self) -> int:
        """Fixed integer degree of a polynomial leaf (expressions.py:57-71)."""
        deg = float((self.initial_values or {}).get("degree", 2.0))
        d = int(round(deg))
        if abs(deg - d) > 1e-5 or d < 1:
            raise ValueError("Polynomial kernel degree must be a fixed positive integer, "
                             f"got {deg:.6g}.")
        return d

    def engine_num_params(self) -> int:
        """Continuous parameters only (categorical leaves train separately);
        an isotropic polynomial carries a hidden variance slot
        (kernel.py:462-480)."""
        if self.kernel_type is not None:
            if self.is_categorical():
                return 0
            if self.kernel_type == KernelType.POLYNOMIAL and self.ard_dim is None:
                return 4
            return self.num_params()
        if self.operator == "scale":
            return self.left.engine_num_params() + 1
        return self.left.engine_num_params() + self.right.engine_num_params()

    def is_tree_servable(self) -> bool:
        """Every leaf is one of the stationary families the tree products serve."""
        if self.kernel_type is not None:
            return self.kernel_type in TREE_LEAF_CODES or self.is_categorical()
        return bool(self.left.is_tree_servable()
                    and (self.operator == "scale" or self.right.is_tree_servable()))

    def to_tree_spec(self, dim: int, default_dims=None) -> List[int]:
        """Flat integer spec of the native kernel-tree products.

        Layout: [d, nparams, nleaves, nnodes, per leaf (tree order): code, ard,
        ndim, p0, dims..., per node (children first, root last): code, a, b].
        A leaf's dimensions are its own active_dims, else those of its nearest
        ancestor with active_dims, else all ``dim`` inputs.  ARD leaves must
        carry one lengthscale per dimension (``make_ard_kernel``)."""
        if not self.is_tree_servable():
            raise NotImplementedError(
                f"kernel {self!r} has leaves outside the gfx950 engine (served: RBF, Matern12, "
                "Matern32, Matern52, RQ, Periodic under sum / product / scale)")
        leaves: List[List[int]] = []
        nodes: List[List[int]] = []
        table = [0]

        def walk(node: "KernelNode", dims: tuple, offset: int):
            dims = node.active_dims if node.active_dims is not None else dims
            for x in dims:
                if not 0 <= x < dim:
                    raise ValueError(f"active_dims index {x} out of range for {dim}-dimensional input")
            if node.is_categorical():
                if node.active_dims is None or len(node.active_dims) != 1 or not node.levels:
                    raise ValueError("categorical kernels need levels and one active dim")
                L = int(node.levels)
                leaves.append([_CAT_LEAF_CODE, L, 1, table[0], int(node.active_dims[0])])
                table[0] += L * L
                nodes.append([_TN_LEAF, len(leaves) - 1, 0])
                return len(nodes) - 1, offset
            if node.kernel_type is not None:
                ard = node.ard_dim is not None
                if ard and node.ard_dim != len(dims):
                    raise ValueError(f"ARD leaf {node!r} has {node.ard_dim} lengthscales for "
                                     f"{len(dims)} active dimensions")
                code = TREE_LEAF_CODES[node.kernel_type]
                extra = [node.structural_degree()] if code == 8 else []
                leaves.append([code, int(ard), len(dims), offset, *extra, *dims])
                nodes.append([_TN_LEAF, len(leaves) - 1, 0])
                return len(nodes) - 1, offset + node.engine_num_params()
            if node.operator in ("sum", "product"):
                a, mid = walk(node.left, dims, offset)
                b, end = walk(node.right, dims, mid)
                nodes.append([_TN_ADD if node.operator == "sum" else _TN_MUL, a, b])
                return len(nodes) - 1, end
            if node.operator == "scale":
                if node.left.has_categorical():
                    raise ValueError("Cannot apply scale to a kernel tree containing categorical "
                                     "nodes (kernel.py:1118-1128)")
                a, mid = walk(node.left, dims, offset)
                nodes.append([_TN_SCALE, a, mid])
                return len(nodes) - 1, mid + 1
            raise ValueError(f"Unknown operator: {node.operator}")

        start = tuple(range(dim)) if default_dims is None else tuple(default_dims)
        _, nparams = walk(self, start, 0)
        if (len(leaves) > 8 or len(nodes) > 16 or nparams > 48 or dim > 32
                or sum(lf[2] for lf in leaves if lf[0] != _CAT_LEAF_CODE) > 64):
            raise NotImplementedError("kernel trees are served up to 8 leaves, 16 nodes, "
                                      "48 parameters, 32 input dimensions and 64 leaf "
                                      "dimensions in total")
        spec = [dim, nparams, len(leaves), len(nodes)]
        for lf in leaves:
            spec += lf
        for nd in nodes:
            spec += nd
        return spec

    def native_kind(self) -> int:
        if not self.is_native_leaf():
            raise NotImplementedError(
                f"kernel {self!r} is outside the gfx950 engine (supported: RBF, Matern12, "
                "Matern32, Matern52, "
                "isotropic or ARD, no composition / active_dims)")
        return NATIVE_KINDS[self.kernel_type]

    def num_params(self) -> int:
        if self.is_categorical():
            if self.levels is None:
                raise ValueError(f"Categorical kernel {self.kernel_type.name} requires levels")
            return _CAT_PARAM_COUNTS[self.kernel_type](self.levels)
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
            if self.is_categorical():
                col = (f"_col{self.active_dims[0]}"
                       if self.active_dims is not None and len(self.active_dims) == 1 else "")
                k = self.num_params()
                return [f"{base}{col}_theta"] if k == 1 else [f"{base}{col}_theta_{i}"
                                                               for i in range(k)]
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
        if self.is_categorical():
            n = self.num_params()
            for i in range(n):
                values[offset + i] = cat_default_raw_param(self.kernel_type, i, self.levels or 2)
            return offset + n
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
        """Public layout -> engine layout (kernel.py:494-568): continuous
        parameters in tree order, categorical slots dropped, an isotropic
        polynomial's [degree, offset, os] as [1, degree, offset, os]."""
        p = np.asarray(public_params, dtype=np.float32)
        if p.shape != (self.num_params(),):
            raise ValueError(f"public_params must have shape ({self.num_params()},), got {p.shape}")
        out: List[float] = []
        self._fill_engine(p, 0, out)
        return np.asarray(out, dtype=np.float32)

    def _fill_engine(self, p, off: int, out: list) -> int:
        if self.kernel_type is not None:
            n = self.num_params()
            if self.is_categorical():
                return off + n
            if self.kernel_type == KernelType.POLYNOMIAL and self.ard_dim is None:
                out.extend([1.0, *p[off:off + 3]])
            else:
                out.extend(p[off:off + n])
            return off + n
        mid = self.left._fill_engine(p, off, out)
        if self.operator == "scale":
            out.append(p[mid])
            return mid + 1
        return self.right._fill_engine(p, mid, out)

    def from_engine_params(self, engine_params) -> np.ndarray:
        """Engine layout -> public layout (kernel.py:511-606): categorical
        slots keep their defaults, a polynomial reports its structural degree
        (the hidden variance slot is dropped)."""
        p = np.asarray(engine_params, dtype=np.float32)
        if p.shape != (self.engine_num_params(),):
            raise ValueError(f"engine_params must have shape ({self.engine_num_params()},), "
                             f"got {p.shape}")
        out = self.get_initial_params()
        self._strip_engine(p, 0, out, 0)
        return out

    def _strip_engine(self, p, eoff: int, out, poff: int):
        if self.kernel_type is not None:
            n = self.num_params()
            if self.is_categorical():
                return eoff, poff + n
            if self.kernel_type == KernelType.POLYNOMIAL and self.ard_dim is None:
                out[poff] = float(self.structural_degree())
                out[poff + 1:poff + 3] = p[eoff + 2:eoff + 4]
                return eoff + 4, poff + 3
            out[poff:poff + n] = p[eoff:eoff + n]
            return eoff + n, poff + n
        e, q = self.left._strip_engine(p, eoff, out, poff)
        if self.operator == "scale":
            out[q] = p[e]
            return e + 1, q + 1
        return self.right._strip_engine(p, e, out, q)

    def _public_slots(self) -> List[bool]:
        """Per public parameter: False for categorical slots."""
        if self.kernel_type is not None:
            return [not self.is_categorical()] * self.num_params()
        if self.operator == "scale":
            return self.left._public_slots() + [True]
        return self.left._public_slots() + self.right._public_slots()

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
        if self.levels is not None:
            d["levels"] = int(self.levels)
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
            levels=d.get("levels"),
        )

    # ---------------------------------------------------------- evaluation
    def evaluate(self, X, X2=None, params=None) -> np.ndarray:
        """K(X, X2) in float64 arithmetic, returned as float32 (kernel.py:722-923).

        Leaves follow the engine's expressions (codegen_engine/expressions.py:
        77-326): periodic divides the summed sin^2 terms by the lengthscale
        (not its square) on raw differences, RQ uses (1 + r^2 / (2 alpha))^-alpha,
        and exp is clamped at -20 where the engine's generated code clamps it
        (Matern-3/2, Matern-5/2 and ARD Matern-1/2 leaves; not RBF, isotropic
        Matern-1/2 or periodic leaves, passes/numerical_stability.py:62-85)."""
        X = np.atleast_2d(np.asarray(X, dtype=np.float64))
        X2 = X if X2 is None else np.atleast_2d(np.asarray(X2, dtype=np.float64))
        p = np.ones(self.num_params()) if params is None else np.asarray(params, np.float64)
        K, _ = self._eval(X, X2, p, 0)
        return K.astype(np.float32)

    def _eval(self, X, X2, p, off):
        if self.active_dims is not None:
            cols = list(self.active_dims)
            X, X2 = X[:, cols], X2[:, cols]
        if self.kernel_type is not None:
            return _leaf_matrix(self, X, X2, p[off:off + self.num_params()]), off + self.num_params()
        if self.operator in ("sum", "product"):
            A, mid = self.left._eval(X, X2, p, off)
            B, end = self.right._eval(X, X2, p, mid)
            return (A + B if self.operator == "sum" else A * B), end
        if self.operator == "scale":
            A, mid = self.left._eval(X, X2, p, off)
            return p[mid] * A, mid + 1
        raise ValueError(f"Unknown operator: {self.operator}")

    def __repr__(self) -> str:
        if self.kernel_type is not None:
            tag = "ARD" if (self.ard or self.ard_dim is not None) else ""
            return f"{self.kernel_type.name}{tag}()"
        if self.operator == "scale":
            return f"{self.scale_factor} * {self.left!r}"
        sym = "+" if self.operator == "sum" else "*"
        return f"({self.left!r} {sym} {self.right!r})"


def _leaf_matrix(node: KernelNode, X, X2, p) -> np.ndarray:
    kt = node.kernel_type
    if kt == KernelType.LINEAR:  # kernel.py:822-826
        nls = node.ard_dim if node.ard_dim is not None else 1
        var = p[:nls]
        return p[nls] * ((X * var) @ X2.T if nls > 1 else var[0] * (X @ X2.T))
    if kt == KernelType.POLYNOMIAL:  # kernel.py:828-844 (public [degree, offset, os])
        if node.ard_dim is not None:
            raise NotImplementedError("ARD polynomial evaluation is not supported")
        deg = node.structural_degree()
        return p[2] * np.power(X @ X2.T + p[1], deg)
    q = X.shape[1]
    nls = node.ard_dim if node.ard_dim is not None else 1
    if node.ard_dim is not None and node.ard_dim != q:
        raise ValueError(f"ARD leaf has {node.ard_dim} lengthscales for {q} dimensions")
    ls = p[:nls]
    diff = X[:, None, :] - X2[None, :, :]
    if kt == KernelType.PERIODIC:
        period, os = p[nls], p[nls + 1]
        s2 = np.sin(np.pi * diff / period) ** 2
        S = (s2 / ls).sum(-1) if nls > 1 else s2.sum(-1) / ls[0]
        return os * np.exp(-2.0 * S)
    r2 = ((diff / ls) ** 2).sum(-1)
    if kt == KernelType.RQ:
        alpha, os = p[nls], p[nls + 1]
        return os * (1.0 + r2 / (2.0 * alpha)) ** (-alpha)
    os = p[nls]
    if kt == KernelType.RBF:
        return os * np.exp(-0.5 * r2)
    r = np.sqrt(np.maximum(r2 + 1e-20, 1e-20))
    if kt == KernelType.MATERN12:
        return os * np.exp(np.maximum(-r, -20.0) if node.ard_dim is not None else -r)
    if kt == KernelType.MATERN32:
        return os * (1 + np.sqrt(3.0) * r) * np.exp(np.maximum(-np.sqrt(3.0) * r, -20.0))
    return os * (1 + np.sqrt(5.0) * r + 5.0 / 3.0 * r2) * np.exp(np.maximum(-np.sqrt(5.0) * r, -20.0))


def make_ard_kernel(kernel: KernelNode, dim: int) -> KernelNode:
    """Resolve ARD leaves to per-dimension lengthscales (kernel.py:1520-1583).

    A leaf gets one lengthscale per dimension it sees: its own active_dims,
    else those of its nearest ancestor with active_dims, else ``dim``."""
    if kernel.is_categorical():
        return KernelNode(kernel_type=kernel.kernel_type, levels=kernel.levels,
                          active_dims=kernel.active_dims)
    if kernel.active_dims is not None:
        dim = len(kernel.active_dims)
    if kernel.kernel_type is not None:
        return KernelNode(kernel_type=kernel.kernel_type, ard_dim=dim,
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


def RQ(lengthscale: float = 1.0, alpha: float = 1.0, outputscale: float = 1.0,
       ard: bool = False, active_dims: Optional[List[int]] = None) -> KernelNode:
    return _leaf(KernelType.RQ, ard, active_dims, lengthscale=lengthscale, alpha=alpha,
                 outputscale=outputscale)


def Periodic(lengthscale: float = 1.0, period: float = 1.0, outputscale: float = 1.0,
             ard: bool = False, active_dims: Optional[List[int]] = None) -> KernelNode:
    return _leaf(KernelType.PERIODIC, ard, active_dims, lengthscale=lengthscale, period=period,
                 outputscale=outputscale)


def Linear(variance: float = 1.0, outputscale: float = 1.0, ard: bool = False,
           active_dims: Optional[List[int]] = None) -> KernelNode:
    return _leaf(KernelType.LINEAR, ard, active_dims, variance=variance, outputscale=outputscale)


def Polynomial(degree: float = 3.0, offset: float = 1.0, outputscale: float = 1.0,
               ard: bool = False, active_dims: Optional[List[int]] = None) -> KernelNode:
    return _leaf(KernelType.POLYNOMIAL, ard, active_dims, degree=degree, offset=offset,
                 outputscale=outputscale)


def _cat_leaf(kt: KernelType, levels: int, active_dims) -> KernelNode:
    if active_dims is None or len(active_dims) != 1:
        raise ValueError("categorical kernels take exactly one active dimension")
    if int(levels) < 2:
        raise ValueError("categorical kernels need at least 2 levels")
    return KernelNode(kernel_type=kt, levels=int(levels), active_dims=tuple(active_dims))


def GD(levels: int, active_dims: Optional[List[int]] = None) -> KernelNode:
    """Gower-distance categorical kernel: R_ij = exp(-theta) off the diagonal."""
    return _cat_leaf(KernelType.GD, levels, active_dims)


def CR(levels: int, active_dims: Optional[List[int]] = None) -> KernelNode:
    """Continuous-relaxation kernel: R_ij = exp(-(theta_i + theta_j))."""
    return _cat_leaf(KernelType.CR, levels, active_dims)


def EHH(levels: int, active_dims: Optional[List[int]] = None) -> KernelNode:
    """Exponential homoscedastic hypersphere kernel."""
    return _cat_leaf(KernelType.EHH, levels, active_dims)


def HH(levels: int, active_dims: Optional[List[int]] = None) -> KernelNode:
    """Homoscedastic hypersphere kernel: R = C C^T."""
    return _cat_leaf(KernelType.HH, levels, active_dims)


def FE(levels: int, active_dims: Optional[List[int]] = None) -> KernelNode:
    """Fully exponential kernel (hypersphere angles plus per-level terms)."""
    return _cat_leaf(KernelType.FE, levels, active_dims)
