"""Shape helpers (src/qutai/core/shape.py:8-54)."""
from __future__ import annotations

from itertools import zip_longest
from math import prod


def infer_shape(data) -> tuple[int, ...]:
    """Shape of nested lists/tuples; rejects ragged nesting."""
    if isinstance(data, (int, float)):
        return ()
    if not isinstance(data, (list, tuple)):
        raise TypeError("data must be a number, list or tuple")
    if not data:
        return (0,)
    shapes = [infer_shape(item) for item in data]
    if any(shape != shapes[0] for shape in shapes):
        raise ValueError("ragged data: items of one level must have equal shapes")
    return (len(data), *shapes[0])


def flatten(data) -> list[float]:
    if isinstance(data, (int, float)):
        return [float(data)]
    return [value for item in data for value in flatten(item)]


def unflatten(values: list, shape: tuple[int, ...]):
    if any(size < 0 for size in shape):
        raise ValueError("shape sizes must be non-negative")
    if len(values) != prod(shape):
        raise ValueError("element count does not match the shape")
    if not shape:
        return values[0]
    block = prod(shape[1:])
    return [unflatten(values[i * block:(i + 1) * block], shape[1:]) for i in range(shape[0])]


def broadcast_shape(left: tuple[int, ...], right: tuple[int, ...]) -> tuple[int, ...]:
    """Broadcast result shape (src/qutai/core/shape.py:41-49)."""
    result = []
    for a, b in zip_longest(reversed(left), reversed(right), fillvalue=1):
        if a == b:
            result.append(a)
        elif a == 1:
            result.append(b)
        elif b == 1:
            result.append(a)
        else:
            raise ValueError(f"shapes {left} and {right} cannot be broadcast")
    return tuple(reversed(result))


def strides(shape: tuple[int, ...]) -> tuple[int, ...]:
    """Contiguous strides in elements (src/qutai/core/shape.py:52-54)."""
    return tuple(prod(shape[axis + 1:]) for axis in range(len(shape)))


def normalize_axis(axis: int, rank: int) -> int:
    """Axis in [-rank, rank) as a non-negative index; ValueError otherwise
    (src/qutai/core/shape.py:103-106)."""
    if not -rank <= axis < rank:
        raise ValueError(f"axis {axis} is out of range for {rank} dimensions")
    return axis % rank


def reduced_shape(shape: tuple[int, ...], axis: int | None = None, keepdims: bool = False) -> tuple[int, ...]:
    """Shape after a reduction over ``axis`` (all axes when None)
    (src/qutai/core/shape.py:109-114)."""
    if axis is None:
        return (1,) * len(shape) if keepdims else ()
    axis = normalize_axis(axis, len(shape))
    return shape[:axis] + ((1,) if keepdims else ()) + shape[axis + 1:]


def transpose_axes(rank: int, axes=None) -> tuple[int, ...]:
    """A full permutation of ``rank`` axes (reversed when None); ValueError
    unless every axis appears once (src/qutai/core/shape.py:131-136)."""
    if axes is None:
        return tuple(range(rank - 1, -1, -1))
    order = tuple(normalize_axis(axis, rank) for axis in axes)
    if len(order) != rank or len(set(order)) != rank:
        raise ValueError("a transpose needs every axis exactly once")
    return order
