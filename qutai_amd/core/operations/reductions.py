"""Sums and means over all elements or one axis, and softmax.

Semantics of src/qutai/core/operations/reductions.py:9-35 and
src/qutai/core/operations/normalization.py:9-25: the gradient of a sum is
G broadcast back over the reduced axis, of a mean that divided by the
count, and of p = softmax(x) along an axis p * (g - sum(g * p)) along the
same axis.  Softmax along the last axis uses one fused backward kernel;
other axes compose the backend's multiply / sum / broadcast / subtract.
"""
from __future__ import annotations

from ...backends.device import get_backend
from ..shape import normalize_axis, reduced_shape


def sum(data, axis=None, keepdims=False):  # noqa: A001 - the reference's name
    shape = tuple(data.shape)
    target = reduced_shape(shape, axis, keepdims)
    backend = get_backend(data.storage)
    values = backend.sum(data.storage, shape, axis=axis)
    kept = reduced_shape(shape, axis, keepdims=True)
    return values, target, lambda g: (get_backend(g).broadcast(g, kept, shape),)


def mean(data, axis=None, keepdims=False):
    shape = tuple(data.shape)
    count = data.storage.size if axis is None else shape[normalize_axis(axis, len(shape))]
    if count == 0:
        raise ValueError("the mean of no elements is undefined")
    target = reduced_shape(shape, axis, keepdims)
    backend = get_backend(data.storage)
    values = backend.mean(data.storage, shape, axis=axis)
    kept = reduced_shape(shape, axis, keepdims=True)
    return values, target, lambda g: (backend.scale(backend.broadcast(g, kept, shape), 1 / count),)


def softmax(data, axis=-1):
    shape = tuple(data.shape)
    axis = normalize_axis(axis, len(shape))
    if shape[axis] == 0:
        raise ValueError("softmax needs a non-empty axis")
    backend = get_backend(data.storage)
    probabilities = backend.softmax(data.storage, shape, axis)

    def rule(g):
        if axis == len(shape) - 1 and hasattr(backend, "softmax_backward"):
            return (backend.softmax_backward(probabilities, g, shape),)
        weighted = backend.multiply(g, probabilities)
        totals = backend.broadcast(backend.sum(weighted, shape, axis), reduced_shape(shape, axis, True), shape)
        return (backend.multiply(probabilities, backend.subtract(g, totals)),)

    return probabilities, shape, rule
