"""mojogp_amd — exact Gaussian-process engine for AMD Instinct MI355X (gfx950).

Python + NumPy host surface over hand-written HIP kernels reached through the
C-ABI library libmojogp_amd.so (ctypes).  No torch in the product path.

    from mojogp_amd import SingleOutputGP, MultiOutputGP, MultiOutputLMCGP, RBF, Matern52
"""

from .gp import MixedTrainingResult, PredictionResult, SingleOutputGP, TrainingResult
from .kernel import (CR, EHH, FE, GD, HH, RQ, KernelNode, KernelType, Linear, Matern12, Matern32,
                     Matern52, Periodic, Polynomial, RBF, make_ard_kernel)
from .multi_output_gp import (LMCTrainingResult, MultiOutputGP, MultiOutputLMCGP,
                              MultiOutputPredictionResult, MultiOutputTrainingResult)

__version__ = "0.1.0"

__all__ = ["SingleOutputGP", "TrainingResult", "PredictionResult", "KernelNode", "KernelType",
           "RBF", "Matern52", "Matern32", "Matern12", "RQ", "Periodic", "Linear", "Polynomial",
           "GD", "CR", "EHH", "HH", "FE", "MixedTrainingResult", "make_ard_kernel",
           "MultiOutputLMCGP",
           "LMCTrainingResult", "MultiOutputPredictionResult", "MultiOutputGP",
           "MultiOutputTrainingResult"]
