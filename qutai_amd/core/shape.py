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
