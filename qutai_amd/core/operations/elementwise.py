"""Broadcasting element-wise arithmetic on operands.

Semantics of src/qutai/core/operations/elementwise.py:10-100: the operands
broadcast to a common shape, the backend's same-named function combines the
broadcast storages, and each gradient is summed back to its operand's shape
(``backend.unbroadcast``).  A trailing-axis vector added to a tensor (the
bias of ``nn.Linear``) takes one fused row-add kernel instead of
materialising the broadcast vector; its gradient is the column sum of G.
"""
from __future__ import annotations

from ...backends.device import get_backend
from ..shape import broadcast_shape


def _operands(left, right):
    backend = get_backend(left.storage, right.storage)
    shape = broadcast_shape(left.shape, right.shape)
    return (backend, shape, backend.broadcast(left.storage, left.shape, shape),
            backend.broadcast(right.storage, right.shape, shape))


def _reduce_to(backend, gradient, shape, target):
    return backend.unbroadcast(gradient, shape, target)


def _bias(big, small):
    """(rows, cols) when ``small`` is a vector along ``big``'s last axis."""
    if len(small.shape) == 1 and big.shape and big.shape[-1] == small.shape[0] and len(big.shape) > 1:
        cols = small.shape[0]
        return (big.storage.size // cols if cols else 0), cols
    return None


def add(left, right):
    backend = get_backend(left.storage, right.storage)
    for big, small, bias_first in ((left, right, False), (right, left, True)):
        layout = _bias(big, small) if hasattr(backend, "add_rows") else None
        if layout is not None:
            rows, cols = layout
            values = backend.add_rows(big.storage, small.storage, rows, cols)

            def bias_rule(g, rows=rows, cols=cols, bias_first=bias_first):
                column_sums = backend.sum_rows(g, rows, cols)
                return (column_sums, g) if bias_first else (g, column_sums)

            return values, big.shape, bias_rule
    backend, shape, a, b = _operands(left, right)

    def rule(g):
        return _reduce_to(backend, g, shape, left.shape), _reduce_to(backend, g, shape, right.shape)

    return backend.add(a, b), shape, rule


def subtract(left, right):
    backend, shape, a, b = _operands(left, right)

    def rule(g):
        return (_reduce_to(backend, g, shape, left.shape),
                backend.negate(_reduce_to(backend, g, shape, right.shape)))

    return backend.subtract(a, b), shape, rule


def multiply(left, right):
    backend, shape, a, b = _operands(left, right)

    def rule(g):
        return (_reduce_to(backend, backend.multiply(g, b), shape, left.shape),
                _reduce_to(backend, backend.multiply(g, a), shape, right.shape))

    return backend.multiply(a, b), shape, rule


def divide(left, right):
    backend, shape, a, b = _operands(left, right)

    def rule(g):
        d_left = backend.divide(g, b)
        d_right = backend.negate(backend.multiply(d_left, backend.divide(a, b)))
        return _reduce_to(backend, d_left, shape, left.shape), _reduce_to(backend, d_right, shape, right.shape)

    return backend.divide(a, b), shape, rule


def divide_scalar(data, value):
    backend = get_backend(data.storage)
    return (backend.divide_scalar(data.storage, value), data.shape,
            lambda g: (get_backend(g).divide_scalar(g, value),))


def scale(data, factor):
    backend = get_backend(data.storage)
    return backend.scale(data.storage, factor), data.shape, lambda g: (get_backend(g).scale(g, factor),)


def negate(data):
    backend = get_backend(data.storage)
    return backend.negate(data.storage), data.shape, lambda g: (get_backend(g).negate(g),)


def square(data):
    backend = get_backend(data.storage)
    return (backend.square(data.storage), data.shape,
            lambda g: (backend.scale(backend.multiply(g, data.storage), 2.0),))


def exp(data):
    backend = get_backend(data.storage)
    values = backend.exp(data.storage)
    return values, data.shape, lambda g: (backend.multiply(g, values),)


def log(data):
    backend = get_backend(data.storage)
    return backend.log(data.storage), data.shape, lambda g: (backend.divide(g, data.storage),)


def _activation(name):
    def operation(data):
        backend = get_backend(data.storage)
        derivative = getattr(backend, name + "_backward")
        return (getattr(backend, name)(data.storage), data.shape, lambda g: (derivative(g, data.storage),))

    operation.__name__ = name
    return operation


relu = _activation("relu")
gelu = _activation("gelu")
tanh = _activation("tanh")
atan = _activation("atan")
