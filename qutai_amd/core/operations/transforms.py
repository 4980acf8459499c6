"""Layout operations: transpose, reshape, concatenate and basic indexing.

Semantics of src/qutai/core/operations/transforms.py:64-123 and the basic
index rules of src/qutai/core/shape.py:57-100 (integers, slices with any
step, ``None`` and one ``Ellipsis``).  An index never expands to a list of
positions: it becomes (shape, element steps, offset), which the backend's
strided copy reads (``gather_slice``) and the gradient writes back
(``scatter_slice``).
"""
from __future__ import annotations

from math import prod

from ...backends.device import get_backend
from ..shape import normalize_axis, strides, transpose_axes


def transpose(data, axes=None):
    shape = tuple(data.shape)
    order = transpose_axes(len(shape), axes)
    target = tuple(shape[a] for a in order)
    inverse = tuple(order.index(a) for a in range(len(order)))
    backend = get_backend(data.storage)
    values = backend.transpose(data.storage, shape, axes=order)
    return values, target, lambda g: (get_backend(g).transpose(g, target, axes=inverse),)


def reshape_target(size: int, shape) -> tuple[int, ...]:
    """``shape`` with at most one -1 resolved so that it holds ``size`` elements."""
    shape = tuple(shape)
    unknown = [i for i, n in enumerate(shape) if n == -1]
    if len(unknown) > 1 or any(n < -1 for n in shape):
        raise ValueError("a reshape takes non-negative sizes and at most one -1")
    if unknown:
        known = prod(n for n in shape if n != -1)
        if known == 0 or size % known:
            raise ValueError(f"cannot reshape {size} elements to {shape}")
        shape = shape[:unknown[0]] + (size // known,) + shape[unknown[0] + 1:]
    if prod(shape) != size:
        raise ValueError(f"cannot reshape {size} elements to {shape}")
    return shape


def reshape(data, shape):
    """A new storage with the same element order; the gradient passes as is."""
    return data.storage.copy(), reshape_target(data.storage.size, shape), lambda g: (g,)


def concatenate(data, axis=0):
    if not data:
        raise ValueError("concatenate needs at least one operand")
    rank = len(data[0].shape)
    axis = normalize_axis(axis, rank)
    first = tuple(data[0].shape)
    for item in data:
        if len(item.shape) != rank or any(a != b for i, (a, b) in enumerate(zip(item.shape, first)) if i != axis):
            raise ValueError("concatenate needs equal shapes outside the joined axis")
    backend = get_backend(*(item.storage for item in data))
    values = backend.concatenate(tuple(item.storage for item in data), tuple(tuple(i.shape) for i in data), axis)
    target = first[:axis] + (sum(item.shape[axis] for item in data),) + first[axis + 1:]
    widths = [item.shape[axis] for item in data]

    def rule(g):
        parts, start = [], 0
        steps = strides(target)
        for width in widths:
            shape = target[:axis] + (width,) + target[axis + 1:]
            parts.append(get_backend(g).gather_slice(g, shape, steps, start * steps[axis]))
            start += width
        return tuple(parts)

    return values, target, rule


def index_view(shape, index) -> tuple[tuple[int, ...], tuple[int, ...], int]:
    """(result shape, element steps, offset) of a basic index into a
    row-major array of ``shape``."""
    parts = index if isinstance(index, tuple) else (index,)
    if sum(part is Ellipsis for part in parts) > 1:
        raise IndexError("an index holds at most one Ellipsis")
    used = sum(part is not None and part is not Ellipsis for part in parts)
    if used > len(shape):
        raise IndexError("too many indices for the tensor")
    expanded = []
    for part in parts:
        if part is Ellipsis:
            expanded.extend([slice(None)] * (len(shape) - used))
        else:
            expanded.append(part)
    if Ellipsis not in parts:
        expanded.extend([slice(None)] * (len(shape) - used))
    result, steps, offset, axis = [], [], 0, 0
    row_steps = strides(shape)
    for part in expanded:
        if part is None:
            result.append(1)
            steps.append(0)
            continue
        length, step = shape[axis], row_steps[axis]
        if isinstance(part, bool) or not isinstance(part, (int, slice)):
            raise TypeError("basic indices are integers, slices, None or Ellipsis")
        if isinstance(part, int):
            position = part + length if part < 0 else part
            if not 0 <= position < length:
                raise IndexError(f"index {part} is out of range for axis {axis} of length {length}")
            offset += position * step
        else:
            start, stop, stride = part.indices(length)
            count = len(range(start, stop, stride))
            result.append(count)
            steps.append(stride * step)
            if count:
                offset += start * step
        axis += 1
    return tuple(result), tuple(steps), offset


def select(data, index):
    shape, steps, offset = index_view(tuple(data.shape), index)
    size = data.storage.size
    values = get_backend(data.storage).gather_slice(data.storage, shape, steps, offset)
    return values, shape, lambda g: (get_backend(g).scatter_slice(g, shape, steps, offset, size),)
