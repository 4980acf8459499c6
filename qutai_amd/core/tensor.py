"""Tensor front-end for the GEMM path (src/qutai/core/tensor.py:14-278).

Only what the contraction path needs: construction from nested lists or a
device storage, ``@`` / ``matmul`` with autograd, same-shape ``+`` and the
broadcast bias add of ``nn.Linear``, ``sum``, ``to(dtype=)`` casts,
``reshape``, last-two-axes ``transpose``, ``backward`` with leaf gradient
accumulation, ``tolist`` / ``item`` reads.
"""
from __future__ import annotations

from functools import partial
from math import isqrt, prod

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
        return _result(_add(self, other), (self, other))

    def __radd__(self, other):
        other = _as_tensor(other, self)
        return _result(_add(other, self), (other, self))

    def sum(self):
        return _result(_sum(self), (self,))

    def reshape(self, shape):
        shape = tuple(shape)
        if -1 in shape:
            known = prod(s for s in shape if s != -1)
            shape = tuple(self.size // known if s == -1 else s for s in shape)
        if prod(shape) != self.size:
            raise ValueError("reshape must keep the element count")
        return _result((self.storage.copy(), shape, lambda g: (g,)), (self,))

    def transpose(self, axes=None):
        rank = self.ndim
        axes = tuple(reversed(range(rank))) if axes is None else tuple(a % rank for a in axes)
        target = tuple(self.shape[a] for a in axes)
        backend = get_backend(self.device)
        values = backend.transpose(self.storage, self.shape, axes=axes)
        inverse = tuple(axes.index(a) for a in range(rank))
        return _result((values, target, lambda g: (backend.transpose(g, target, axes=inverse),)), (self,))

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


def _add(left, right):
    """Same-shape add, or a bias broadcast over the leading axes (last axis equal)."""
    backend = get_backend(left.storage, right.storage)
    if left.shape == right.shape:
        return backend.add(left.storage, right.storage), left.shape, lambda g: (g, g)
    for big, small, swap in ((left, right, False), (right, left, True)):
        if small.ndim == 1 and big.ndim >= 1 and big.shape[-1] == small.shape[0]:
            cols = small.shape[0]
            rows = big.size // cols if cols else 0
            values = backend.add_rows(big.storage, small.storage, rows, cols)

            def rule(g, rows=rows, cols=cols, swap=swap):
                reduced = backend.sum_rows(g, rows, cols)
                return (reduced, g) if swap else (g, reduced)

            return values, big.shape, rule
    raise ValueError(f"add supports equal shapes or a trailing-axis bias, got {left.shape} and {right.shape}")


def _sum(x):
    backend = get_backend(x.storage)
    values = backend.sum_all(x.storage)
    size = x.size
    return values, (), lambda g: (backend.broadcast_scalar(g, size),)


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


def matmul(left, right):
    """Vector / matrix / batched product (src/qutai/core/tensor.py:275-278)."""
    like = left if isinstance(left, Tensor) else right if isinstance(right, Tensor) else None
    a, b = _as_tensor(left, like), _as_tensor(right, like)
    return _output(a @ b, left, right)


def sum(x):  # noqa: A001 - mirrors qutai.sum
    tensor = _as_tensor(x)
    return _output(tensor.sum(), x)
