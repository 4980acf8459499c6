"""Qutai's GEMM hot path on AMD Instinct MI355X (gfx950).

``device="amd"`` selects the backend module ``qutai_amd.backends.amd``
(native kernels in ``libqutai_amd.so``, C ABI in ``include/qutai_amd.h``).
Importing the package does not touch the GPU.
"""
from .backends.device import is_available, synchronize
from .core.tensor import Tensor, add, concatenate, divide, gelu, matmul, mean, multiply, relu, softmax, subtract, sum

__all__ = ["Tensor", "add", "concatenate", "divide", "gelu", "matmul", "mean", "multiply", "relu", "softmax",
           "subtract", "sum", "is_available", "synchronize"]
