"""Tensor front-end for the GEMM path (src/qutai/core/tensor.py:14-278).

Construction from nested lists or a device storage, ``@`` / ``matmul``
with autograd, broadcasting ``+ - * /`` (a scalar divisor divides in one
kernel), negation, basic indexing, ``sum`` / ``mean`` over everything or
one axis, ``softmax``, the element-wise functions of the reference Tensor,
``to(dtype=)`` casts, ``reshape``, any ``transpose``, ``concatenate``,
``backward`` with leaf gradient accumulation, ``tolist`` / ``item`` reads.
"""
from __future__ import annotations

from functools import partial
from math import prod

from ..backends.device import default_dtype, get_backend, transfer
from ..backends.storage import Storage
from . import grad as autograd
from . import operations
from .shape import flatten, infer_shape, unflatten


class Tensor:
    def __init__(self, data, *, shape=None, requires_grad=False, device=None, dtype=None):
        device = device if device is not None else data.device if isinstance(data, Storage) else "amd"
        dtype = dtype if dtype is not None else data.dtype if isinstance(data, Storage) else default_dtype(device)
        backend = get_backend(device)
        if dtype not in ("float32", "float64", "bfloat16"):
            raise ValueError("real Tensors are float32, float64 or bfloat16")
        if isinstance(data, Storage):
            if data.device != device or data.dtype != dtype:
                raise ValueError("storage device/dtype differ from the Tensor's")
            self.shape = (data.size,) if shape is None else tuple(shape)
            self.storage = data
        else:
            self.shape = infer_shape(data) if shape is None else tuple(shape)
            self.storage = backend.storage(flatten(data), dtype=dtype)
        if any(size < 0 for size in self.shape) or prod(self.shape) != self.storage.size:
            raise ValueError("element count does not match the Tensor shape")
        self.requires_grad = requires_grad
        self.grad = None
        self.parents = ()
        self.backward_rule = None

    @property
    def device(self):
        return self.storage.device

    @property
    def dtype(self):
        return self.storage.dtype

    @property
    def size(self):
        return self.storage.size

    @property
    def ndim(self):
        return len(self.shape)

    def __len__(self):
        if not self.shape:
            raise TypeError("a scalar Tensor has no length")
        return self.shape[0]

    def __matmul__(self, other):
        other = _as_tensor(other, self)
        return _result(operations.matmul(self, other), (self, other))

    def __rmatmul__(self, other):
        other = _as_tensor(other, self)
        return _result(operations.matmul(other, self), (other, self))

    def __add__(self, other):
        other = _as_tensor(other, self)
        return _result(operations.add(self, other), (self, other))

    def __radd__(self, other):
        other = _as_tensor(other, self)
        return _result(operations.add(other, self), (other, self))

    def __sub__(self, other):
        other = _as_tensor(other, self)
        return _result(operations.subtract(self, other), (self, other))

    def __rsub__(self, other):
        other = _as_tensor(other, self)
        return _result(operations.subtract(other, self), (other, self))

    def __mul__(self, other):
        other = _as_tensor(other, self)
        return _result(operations.multiply(self, other), (self, other))

    def __rmul__(self, other):
        other = _as_tensor(other, self)
        return _result(operations.multiply(other, self), (other, self))

    def __truediv__(self, other):
        if isinstance(other, (int, float)) and not isinstance(other, bool):
            # a scalar divisor needs no broadcast tensor (src/qutai/core/tensor.py:119-121)
            return _result(operations.divide_scalar(self, other), (self,))
        other = _as_tensor(other, self)
        return _result(operations.divide(self, other), (self, other))

    def __rtruediv__(self, other):
        other = _as_tensor(other, self)
        return _result(operations.divide(other, self), (other, self))

    def __neg__(self):
        return _result(operations.negate(self), (self,))

    def __getitem__(self, index):
        return _result(operations.select(self, index), (self,))

    def sum(self, axis=None, keepdims=False):
        return _result(operations.sum(self, axis=axis, keepdims=keepdims), (self,))

    def mean(self, axis=None, keepdims=False):
        return _result(operations.mean(self, axis=axis, keepdims=keepdims), (self,))

    def square(self):
        return _result(operations.square(self), (self,))

    def exp(self):
        return _result(operations.exp(self), (self,))

    def log(self):
        return _result(operations.log(self), (self,))

    def tanh(self):
        return _result(operations.tanh(self), (self,))

    def atan(self):
        return _result(operations.atan(self), (self,))

    def reshape(self, shape):
        return _result(operations.reshape(self, shape), (self,))

    def transpose(self, axes=None):
        return _result(operations.transpose(self, axes), (self,))

    @property
    def T(self):
        return self.transpose()

    def tolist(self):
        return unflatten(self.storage.tolist(), self.shape)

    def item(self):
        if self.size != 1:
            raise ValueError("item() needs exactly one element")
        return self.storage.tolist()[0]

    def to(self, device=None, *, dtype=None, copy=False):
        if dtype is not None and dtype not in ("float32", "float64", "bfloat16"):
            raise ValueError("real Tensors are float32, float64 or bfloat16")
        values = transfer(self.storage, device, dtype, copy=copy)
        if values is self.storage:
            return self
        source = self.dtype
        return autograd.record(Tensor(values, shape=self.shape), (self,),
                               lambda g: (transfer(g, None, source),))

    def zero_grad(self):
        self.grad = None

    def backward(self, gradient=None, *, retain_graph=True):
        if not self.requires_grad:
            raise ValueError("this Tensor does not record gradients")
        if gradient is None:
            if self.size != 1:
                raise ValueError("a non-scalar result needs an output gradient of its shape")
            seed = get_backend(self.device).full(self.size, 1.0, dtype=self.dtype)
        else:
            gradient = _as_tensor(gradient, self)
            if gradient.shape != self.shape:
                raise ValueError("output gradient shape differs from the Tensor's")
            if gradient.device != self.device or gradient.dtype != self.dtype:
                raise ValueError("output gradient device and dtype must be the Tensor's")
            seed = gradient.storage

        created = set()  # leaves whose grad storage this pass made: no one else holds it

        def accumulate(tensor, values):
            if isinstance(values, autograd.DeferredGradient):
                if tensor.grad is not None and id(tensor) in created and values.dtype == tensor.dtype:
                    values.add_into(tensor.grad.storage)
                    return
                values = autograd.owned(values.materialize())
            fresh = False
            if values.dtype != tensor.dtype:
                values, fresh = transfer(values, tensor.device, tensor.dtype), True
            if tensor.grad is not None:
                values = get_backend(tensor.device).add(tensor.grad.storage, values)
            elif not (fresh or autograd.take_owned(values)):
                values = values.copy()
            tensor.grad = Tensor(values, shape=tensor.shape)
            created.add(id(tensor))

        autograd.backward(self, seed, retain_graph=retain_graph, leaf_sink=accumulate)

    def __repr__(self):
        return f"Tensor({self.tolist()!r})"


def _as_tensor(data, like=None):
    if isinstance(data, Tensor):
        if like is not None:
            get_backend(like.storage, data.storage)
        return data
    return Tensor(data, device=None if like is None else like.device, dtype=None if like is None else like.dtype)


def _result(computation, parents):
    values, shape, rule = computation
    return autograd.record(Tensor(values, shape=shape, device=values.device, dtype=values.dtype), parents, rule)


def _output(result, *inputs):
    return result if any(isinstance(data, Tensor) for data in inputs) else result.tolist()


def _pair(left, right):
    like = left if isinstance(left, Tensor) else right if isinstance(right, Tensor) else None
    return _as_tensor(left, like), _as_tensor(right, like)


def matmul(left, right):
    """Vector / matrix / batched product (src/qutai/core/tensor.py:275-278)."""
    a, b = _pair(left, right)
    return _output(a @ b, left, right)


def add(left, right):
    a, b = _pair(left, right)
    return _output(a + b, left, right)


def subtract(left, right):
    a, b = _pair(left, right)
    return _output(a - b, left, right)


def multiply(left, right):
    a, b = _pair(left, right)
    return _output(a * b, left, right)


def divide(left, right):
    if isinstance(right, (int, float)) and not isinstance(right, bool):
        return _output(_as_tensor(left) / right, left, right)
    a, b = _pair(left, right)
    return _output(a / b, left, right)


def sum(x, axis=None, keepdims=False):  # noqa: A001 - mirrors qutai.sum
    tensor = _as_tensor(x)
    return _output(tensor.sum(axis, keepdims), x)


def mean(x, axis=None, keepdims=False):
    tensor = _as_tensor(x)
    return _output(tensor.mean(axis, keepdims), x)


def softmax(x, axis=-1):
    tensor = _as_tensor(x)
    return _output(_result(operations.softmax(tensor, axis), (tensor,)), x)


def relu(x):
    tensor = _as_tensor(x)
    return _output(_result(operations.relu(tensor), (tensor,)), x)


def gelu(x):
    tensor = _as_tensor(x)
    return _output(_result(operations.gelu(tensor), (tensor,)), x)


def concatenate(tensors, axis=0):
    items = tuple(_as_tensor(t, tensors[0] if isinstance(tensors[0], Tensor) else None) for t in tensors)
    return _output(_result(operations.concatenate(items, axis), items), *tensors)
