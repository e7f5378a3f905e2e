"""mojogp_amd — exact Gaussian-process engine for AMD Instinct MI355X (gfx950).

Python + NumPy host surface over hand-written HIP kernels reached through the
C-ABI library libmojogp_amd.so (ctypes).  No torch in the product path.
"""

__version__ = "0.1.0"
