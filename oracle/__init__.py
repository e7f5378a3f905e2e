"""CPU oracle for the exact-GP hot path — TEST INFRASTRUCTURE ONLY.

This package restates the reference algorithm (caspbian/mojogp) on the CPU so
the gfx950 product path can be checked against it.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import or run anything here, and only as the checker/baseline; the product
(``mojogp_amd``) never routes through it.

Modules
  kernels.py   float64 kernel values, gradients and products
               (reference: mojogp/kernel.py:804-923, codegen_engine/expressions.py,
               codegen_engine/passes/numerical_stability.py)
  cpu_ref/     C restatement of the matvec hot loop for the CPU baseline

Every function states in its docstring what pins it (closed forms, library
routines, invariants); a function with no such check says "parity unpinned".
"""
