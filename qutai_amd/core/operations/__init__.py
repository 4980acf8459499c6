from .elementwise import (add, atan, divide, divide_scalar, exp, gelu, log, multiply, negate, relu, scale, square,
                          subtract, tanh)
from .linalg import matmul
from .reductions import mean, softmax, sum
from .transforms import concatenate, reshape, select, transpose

__all__ = ["add", "atan", "concatenate", "divide", "divide_scalar", "exp", "gelu", "log", "matmul", "mean",
           "multiply", "negate", "relu", "reshape", "scale", "select", "softmax", "square", "subtract", "sum",
           "tanh", "transpose"]
