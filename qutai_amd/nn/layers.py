"""nn.Linear on the amd device (src/qutai/nn/layers.py:133-150).

Weight stored (in, out), ``Y = X @ W + b`` through the Tensor matmul (whose
gradient rule gives dX = G W^T (NT) and dW = X^T G (TN) on the GEMM) and the
trailing-axis bias add; initialisation U(+-in^-1/2) from Random(seed).
"""
from __future__ import annotations

from random import Random

from ..core.tensor import Tensor, matmul


class Linear:
    def __init__(self, in_features, out_features, *, bias=True, seed=None, device="amd", dtype="float32"):
        if in_features <= 0 or out_features <= 0:
            raise ValueError("feature counts must be positive")
        random = Random(seed)
        bound = in_features ** -0.5
        self.weight = Tensor([[random.uniform(-bound, bound) for _ in range(out_features)]
                              for _ in range(in_features)], requires_grad=True, device=device, dtype=dtype)
        self.bias = Tensor([0.0] * out_features, requires_grad=True, device=device, dtype=dtype) if bias else None

    def __call__(self, data):
        tensor = data if isinstance(data, Tensor) else Tensor(data, device=self.weight.device,
                                                              dtype=self.weight.dtype)
        result = matmul(tensor, self.weight)
        return result if self.bias is None else result + self.bias

    def parameters(self):
        return (self.weight,) if self.bias is None else (self.weight, self.bias)
