"""TEST INFRASTRUCTURE ONLY — CPU parity oracle for the MI355X GEMM path.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker (or, for the
baseline, as the timed CPU restatement).  The product (``qutai_amd``) never
imports it and has no CPU fallback.

Contents
  * pure-Python restatements of the reference CPU path, each citing the
    reference file:line it follows: ``matmul`` (cpu.py:140-163), ``gemm``
    (cpu_lm.py:11-42), ``softmax`` (cpu.py:250-260 with ``_axis_indices``
    cpu.py:231-237), ``silu`` (cpu_lm.py:107-111), ``routing``
    (cpu_lm.py:204-242), ``route_gather`` (cpu_lm.py:279-283), ``combine``
    (cpu_lm.py:294-303), ``routing_backward`` (cpu_lm.py:245-276),
    ``combine_backward`` (cpu_lm.py:306-320), the decoder glue ``embedding`` /
    ``embedding_backward`` / ``rms_norm`` / ``rms_norm_backward`` /
    ``silu_backward`` / ``rope`` / ``head_rows`` / ``head_rows_backward`` /
    ``head_loss`` / ``head_gradient`` (cpu_lm.py:54-138, 323-371),
    ``attention`` / ``attention_backward``
    (cpu_lm.py:141-201), ``bf16`` (the RNE encoder of cuda.py:98-101 /
    tests/test_bfloat16_storage.py:10-16), and the generic tensor functions
    ``broadcast`` (cpu.py:127-137), ``transpose`` (cpu.py:166-180),
    ``reduce_sum`` (cpu.py:183-203), ``mean`` (cpu.py:206-215),
    ``unbroadcast`` (cpu.py:218-228), ``concatenate`` (cpu.py:514-520),
    ``gather`` / ``scatter`` (cpu.py:104-114), ``binary`` (cpu.py:122-124,
    452-466) and ``unary`` (cpu.py:468-511);
  * ``gemm_f64``: the same float64 sequential-k GEMM compiled from
    ``oracle/gemm_f64.c`` (bit-identical to ``gemm``; used at sizes the
    Python loop cannot finish);
  * ``attention_np`` / ``attention_backward_np``: numpy float64 forms of the
    attention loops for one (batch, head) pair, for the full-size checks;
  * numpy helpers for bf16 rounding of whole arrays.

How each function is pinned (tests/test_oracle.py): reference-test golden
vectors and closed forms, agreement of the two independent GEMM
restatements (Python loop vs C) bit for bit, numpy cross-checks within
tolerance, brute-force routing invariants.  No function is left unpinned.
"""
from __future__ import annotations

import ctypes
import os
import struct
import subprocess
from math import cos, exp, fsum, log, prod, sin, sqrt
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIBRARY = HERE / "_build" / "liboracle.so"


# ---- pure-Python restatements ------------------------------------------------

def bf16(value: float) -> float:
    """fp32 -> bfloat16 -> fp32, round to nearest even (cuda.py:98-101)."""
    bits = struct.unpack("<I", struct.pack("<f", value))[0]
    if bits & 0x7FFFFFFF > 0x7F800000:
        bits = (bits >> 16) | 0x40
    else:
        bits = (bits + 0x7FFF + ((bits >> 16) & 1)) >> 16
    return struct.unpack("<f", struct.pack("<I", bits << 16))[0]


def _broadcast_shape(left, right):
    result = []
    for i in range(max(len(left), len(right))):
        a = left[-1 - i] if i < len(left) else 1
        b = right[-1 - i] if i < len(right) else 1
        if a != b and 1 not in (a, b):
            raise ValueError(f"shapes {left} and {right} cannot be broadcast")
        result.append(max(a, b) if 1 in (a, b) else a)
    return tuple(reversed(result))


def _strides(shape):
    return tuple(prod(shape[axis + 1:]) for axis in range(len(shape)))


def matmul(left, right, left_shape, right_shape) -> list[float]:
    """cpu.matmul (src/qutai/backends/cpu.py:140-163): vectors promoted,
    batch axes broadcast, float64 sum with k = 0..K-1 in order."""
    if len(left_shape) == 1:
        left_shape = (1, *left_shape)
    if len(right_shape) == 1:
        right_shape = (*right_shape, 1)
    batches = _broadcast_shape(left_shape[:-2], right_shape[:-2])
    left_shape = (1,) * (len(batches) + 2 - len(left_shape)) + tuple(left_shape)
    right_shape = (1,) * (len(batches) + 2 - len(right_shape)) + tuple(right_shape)
    left_steps, right_steps = _strides(left_shape), _strides(right_shape)
    rows, inner = left_shape[-2:]
    columns = right_shape[-1]
    result = [0.0] * (prod(batches) * rows * columns)
    from itertools import product as coordinates
    for batch, coordinate in enumerate(coordinates(*(range(size) for size in batches))):
        left_start = right_start = 0
        for axis, position in enumerate(coordinate):
            if left_shape[axis] != 1:
                left_start += position * left_steps[axis]
            if right_shape[axis] != 1:
                right_start += position * right_steps[axis]
        for row in range(rows):
            for column in range(columns):
                total = 0.0
                for k in range(inner):
                    total += left[left_start + row * inner + k] * right[right_start + k * columns + column]
                result[(batch * rows + row) * columns + column] = total
    return result


def gemm(a, b, rows, inner, cols, *, transpose_left=False, transpose_right=False, out=None, accumulate=False):
    """cpu_lm.gemm (src/qutai/backends/cpu_lm.py:11-42)."""
    if accumulate and out is None:
        raise ValueError("accumulate needs out")
    result = list(out) if out is not None else [0.0] * (rows * cols)
    for i in range(rows):
        for j in range(cols):
            value = 0.0
            for k in range(inner):
                value += (a[k * rows + i if transpose_left else i * inner + k]
                          * b[j * inner + k if transpose_right else k * cols + j])
            result[i * cols + j] = value + result[i * cols + j] if accumulate else value
    return result


def _axis_indices(shape, axis):
    """cpu._axis_indices (src/qutai/backends/cpu.py:231-237)."""
    axis %= len(shape)
    step = prod(shape[axis + 1:])
    width = shape[axis] * step
    return (range(outer * width + offset, (outer + 1) * width + offset, step)
            for outer in range(prod(shape[:axis])) for offset in range(step))


def softmax(values, shape, axis) -> list[float]:
    """cpu.softmax (src/qutai/backends/cpu.py:250-260): subtract the group
    maximum, exponentiate, divide by the fsum."""
    result = [0.0] * len(values)
    for indices in _axis_indices(shape, axis):
        items = [values[index] for index in indices]
        peak = max(items)
        weights = [exp(value - peak) for value in items]
        total = fsum(weights)
        for index, weight in zip(indices, weights):
            result[index] = weight / total
    return result


def _coordinates(shape):
    from itertools import product as cartesian
    return cartesian(*(range(size) for size in shape))


def broadcast(values, shape, target) -> list[float]:
    """cpu.broadcast (src/qutai/backends/cpu.py:127-137): every coordinate of
    ``target`` reads the source element whose size-1 axes are pinned to 0."""
    padded = (1,) * (len(target) - len(shape)) + tuple(shape)
    steps = _strides(padded)
    result = []
    for coordinate in _coordinates(target):
        offset = 0
        for position, length, step in zip(coordinate, padded, steps):
            if length != 1:
                offset += position * step
        result.append(values[offset])
    return result


def transpose(values, shape, axes=None) -> list[float]:
    """cpu.transpose (src/qutai/backends/cpu.py:166-180): each source
    element goes to its permuted coordinate."""
    axes = tuple(reversed(range(len(shape)))) if axes is None else tuple(a % len(shape) for a in axes)
    target = tuple(shape[a] for a in axes)
    steps = _strides(target)
    result = [0.0] * len(values)
    for value, coordinate in zip(values, _coordinates(shape)):
        result[sum(coordinate[a] * step for a, step in zip(axes, steps))] = value
    return result


def reduce_sum(values, shape=None, axis=None) -> list[float]:
    """cpu.sum (src/qutai/backends/cpu.py:183-203): everything, or one axis
    with the axis dropped; float64 additions in storage order."""
    if axis is None:
        total = 0.0
        for value in values:
            total += value
        return [total]
    axis %= len(shape)
    target = tuple(shape[:axis]) + tuple(shape[axis + 1:])
    steps = _strides(target)
    result = [0.0] * prod(target)
    for value, coordinate in zip(values, _coordinates(shape)):
        kept = coordinate[:axis] + coordinate[axis + 1:]
        result[sum(c * step for c, step in zip(kept, steps))] += value
    return result


def mean(values, shape=None, axis=None) -> list[float]:
    """cpu.mean (src/qutai/backends/cpu.py:206-215)."""
    count = len(values) if axis is None else shape[axis % len(shape)]
    if not count:
        raise ValueError("the mean of no elements is undefined")
    return [total / count for total in reduce_sum(values, shape, axis)]


def unbroadcast(values, shape, target) -> list[float]:
    """cpu.unbroadcast (src/qutai/backends/cpu.py:218-228): sum every axis
    that the target holds as 1, keeping it as 1."""
    padded = (1,) * (len(shape) - len(target)) + tuple(target)
    current = tuple(shape)
    for axis, (length, original) in enumerate(zip(shape, padded)):
        if original == 1 and length != 1:
            values = reduce_sum(values, current, axis)
            current = current[:axis] + (1,) + current[axis + 1:]
    return list(values)


def concatenate(values, shapes, axis=0) -> list[float]:
    """cpu.concatenate (src/qutai/backends/cpu.py:514-520): for every outer
    index, the pieces' blocks in order."""
    axis %= len(shapes[0])
    sizes = [prod(shape[axis:]) for shape in shapes]
    return [value for outer in range(prod(shapes[0][:axis]))
            for data, size in zip(values, sizes) for value in data[outer * size:(outer + 1) * size]]


def gather(values, positions) -> list[float]:
    """cpu.gather (src/qutai/backends/cpu.py:104-106)."""
    return [values[position] for position in positions]


def scatter(values, positions, size) -> list[float]:
    """cpu.scatter (src/qutai/backends/cpu.py:109-114): additions in input order."""
    result = [0.0] * size
    for position, value in zip(positions, values):
        result[position] += value
    return result


def binary(left, right, operation) -> list[float]:
    """cpu.add / subtract / multiply / divide (src/qutai/backends/cpu.py:122-124,
    452-466) for operation "add", "subtract", "multiply", "divide"."""
    import operator
    function = {"add": operator.add, "subtract": operator.sub, "multiply": operator.mul,
                "divide": operator.truediv}[operation]
    return [function(a, b) for a, b in zip(left, right)]


def unary(values, operation, *, gradient=None, factor=None) -> list[float]:
    """The element-wise functions of src/qutai/backends/cpu.py:468-511 (and
    ``divide_scalar``, x / factor, of the CUDA path, cuda.py:192-195)."""
    from math import atan, erf, pi, tanh
    g = gradient if gradient is not None else [None] * len(values)
    table = {
        "negate": lambda x, _: -x,
        "square": lambda x, _: x * x,
        "scale": lambda x, _: x * factor,
        "divide_scalar": lambda x, _: x / factor,
        "relu": lambda x, _: max(x, 0.0),
        "relu_backward": lambda x, d: d if x > 0 else 0.0,
        "gelu": lambda x, _: x * (1 + erf(x / sqrt(2))) / 2,
        "gelu_backward": lambda x, d: d * ((1 + erf(x / sqrt(2))) / 2 + x * exp(-x * x / 2) / sqrt(2 * pi)),
        "exp": lambda x, _: exp(x),
        "log": lambda x, _: log(x),
        "tanh": lambda x, _: tanh(x),
        "atan": lambda x, _: atan(x),
        "tanh_backward": lambda x, d: d * (1 - tanh(x) ** 2),
        "atan_backward": lambda x, d: d / (1 + x * x),
    }
    function = table[operation]
    return [function(x, d) for x, d in zip(values, g)]


def silu(values) -> list[float]:
    """cpu_lm.silu (src/qutai/backends/cpu_lm.py:107-111)."""
    return [x * (1 / (1 + exp(-x)) if x >= 0 else exp(x) / (1 + exp(x))) for x in values]


def routing(scores, rows, experts, top_k) -> dict:
    """cpu_lm.routing (src/qutai/backends/cpu_lm.py:204-242): float64 softmax
    of the scores, experts sorted by descending probability (stable: lower
    index first on ties), weights renormalised over the top_k, per-expert
    (token, slot) lists in token order, utilization and the aux loss."""
    probs = softmax(scores, (rows, experts), 1)
    weights = [0.0] * (rows * top_k)
    indices = [0] * (rows * top_k)
    token_ids = [[] for _ in range(experts)]
    slot_ids = [[] for _ in range(experts)]
    for row in range(rows):
        selected = sorted(range(experts), key=lambda e: probs[row * experts + e], reverse=True)[:top_k]
        total = sum(probs[row * experts + e] for e in selected)
        for slot, e in enumerate(selected):
            indices[row * top_k + slot] = e
            weights[row * top_k + slot] = probs[row * experts + e] / total
            token_ids[e].append(row)
            slot_ids[e].append(slot)
    counts = tuple(map(len, token_ids))
    utilization = [c / (rows * top_k) for c in counts]
    aux = experts * sum(utilization[e] * sum(probs[row * experts + e] for row in range(rows)) / rows
                        for e in range(experts))
    return dict(probs=probs, weights=weights, indices=indices, counts=counts, ids=token_ids, slots=slot_ids,
                utilization=utilization, aux=aux, rows=rows, experts=experts, top_k=top_k)


def route_gather(values, route, expert, width) -> list[float]:
    """cpu_lm.route_gather (src/qutai/backends/cpu_lm.py:279-283)."""
    return [values[row * width + j] for row in route["ids"][expert] for j in range(width)]


def combine(outputs, weights, route, width) -> list[float]:
    """cpu_lm.combine (src/qutai/backends/cpu_lm.py:294-303): expert-major
    weighted scatter-add."""
    result = [0.0] * (route["rows"] * width)
    for expert, values in outputs:
        for i, (row, slot) in enumerate(zip(route["ids"][expert], route["slots"][expert])):
            factor = weights[row * route["top_k"] + slot]
            for j in range(width):
                result[row * width + j] += factor * values[i * width + j]
    return result


def routing_backward(gradient, route, auxiliary=False) -> list[float]:
    """cpu_lm.routing_backward (src/qutai/backends/cpu_lm.py:245-276): the
    logit gradient of the renormalised top-k weights (gradient [rows*top_k])
    or of the auxiliary loss (gradient [1], utilization held constant)."""
    rows, experts, top_k = route["rows"], route["experts"], route["top_k"]
    probs, weights, indices, util = route["probs"], route["weights"], route["indices"], route["utilization"]
    out = [0.0] * (rows * experts)
    for row in range(rows):
        if auxiliary:
            center = sum(probs[row * experts + e] * util[e] for e in range(experts))
            for e in range(experts):
                out[row * experts + e] = (gradient[0] * experts / rows * probs[row * experts + e]
                                          * (util[e] - center))
        else:
            center = sum(gradient[row * top_k + s] * weights[row * top_k + s] for s in range(top_k))
            for s in range(top_k):
                e = indices[row * top_k + s]
                out[row * experts + e] = weights[row * top_k + s] * (gradient[row * top_k + s] - center)
    return out


def combine_backward(gradient, outputs, weights, route, width):
    """cpu_lm.combine_backward (src/qutai/backends/cpu_lm.py:306-320): per
    expert output the row gradients dy * weight, and the weight gradient
    dy . expert row."""
    grads = []
    dw = [0.0] * len(weights)
    for expert, values in outputs:
        dy = [0.0] * len(values)
        for i, (row, slot) in enumerate(zip(route["ids"][expert], route["slots"][expert])):
            at = row * route["top_k"] + slot
            for j in range(width):
                dy[i * width + j] = gradient[row * width + j] * weights[at]
                dw[at] += gradient[row * width + j] * values[i * width + j]
        grads.append(dy)
    return (*grads, dw)


def attention(q, k, v, batch, time, heads, kv_heads, dim, *, causal=True, scale=None):
    """cpu_lm.attention (src/qutai/backends/cpu_lm.py:141-173): for every
    (b, t, h) in the lm layout ``((b*time + t)*heads + h)*dim``, scores over
    keys s <= t (all keys when ``causal`` is False, the nn path of
    nn/layers.py:334-354) scaled by 1/sqrt(dim) (or ``scale``), max-subtracted
    exponentials, output = sum p v / sum p, lse = peak + log(sum p) at
    ``(b*time + t)*heads + h``.  K/V head = h // (heads // kv_heads)."""
    scale = 1 / dim ** 0.5 if scale is None else scale
    out = [0.0] * (batch * time * heads * dim)
    lse = [0.0] * (batch * time * heads)
    for b in range(batch):
        for t in range(time):
            for h in range(heads):
                qi = ((b * time + t) * heads + h) * dim
                kh = h // (heads // kv_heads)
                keys = range(t + 1) if causal else range(time)
                rows = [((b * time + s) * kv_heads + kh) * dim for s in keys]
                scores = [sum(q[qi + j] * k[r + j] for j in range(dim)) * scale for r in rows]
                peak = max(scores)
                weights = [exp(x - peak) for x in scores]
                total = sum(weights)
                lse[(b * time + t) * heads + h] = peak + log(total)
                for j in range(dim):
                    out[qi + j] = sum(p * v[r + j] for p, r in zip(weights, rows)) / total
    return out, lse


def attention_backward(gradient, q, k, v, out, lse, batch, time, heads, kv_heads, dim):
    """cpu_lm.attention_backward (src/qutai/backends/cpu_lm.py:176-201):
    p = exp(q.k * scale - lse), delta = g.out, ds = p (g.v - delta) scale;
    dq += ds k, dk += ds q, dv += p g over keys s <= t."""
    scale = 1 / dim ** 0.5
    dq, dk, dv = [0.0] * len(q), [0.0] * len(k), [0.0] * len(v)
    for b in range(batch):
        for t in range(time):
            for h in range(heads):
                qi = ((b * time + t) * heads + h) * dim
                kh = h // (heads // kv_heads)
                delta = sum(gradient[qi + j] * out[qi + j] for j in range(dim))
                for s in range(t + 1):
                    ki = ((b * time + s) * kv_heads + kh) * dim
                    p = exp(sum(q[qi + j] * k[ki + j] for j in range(dim)) * scale - lse[(b * time + t) * heads + h])
                    dp = sum(gradient[qi + j] * v[ki + j] for j in range(dim))
                    ds = p * (dp - delta) * scale
                    for j in range(dim):
                        dq[qi + j] += ds * k[ki + j]
                        dk[ki + j] += ds * q[qi + j]
                        dv[ki + j] += p * gradient[qi + j]
    return dq, dk, dv


def attention_np(q, k, v, *, causal=True, scale=None):
    """numpy float64 form of ``attention`` for one (batch, head) pair at
    sizes the loop cannot finish: q [T, D], k/v [T, D] -> (out [T, D], lse [T])."""
    q, k, v = (np.asarray(a, dtype=np.float64) for a in (q, k, v))
    scale = 1 / q.shape[1] ** 0.5 if scale is None else scale
    s = (q @ k.T) * scale
    if causal:
        s = np.where(np.tril(np.ones(s.shape, dtype=bool)), s, -np.inf)
    peak = s.max(axis=1, keepdims=True)
    w = np.exp(s - peak)
    total = w.sum(axis=1, keepdims=True)
    return (w @ v) / total, (peak + np.log(total))[:, 0]


def attention_backward_np(g, q, k, v, out, lse, *, scale=None, causal=True):
    """numpy float64 form of ``attention_backward`` for one (batch, head) pair
    (causal, or every key with ``causal=False`` as for nn attention): returns
    dq, dk, dv of that pair."""
    g, q, k, v, out = (np.asarray(a, dtype=np.float64) for a in (g, q, k, v, out))
    scale = 1 / q.shape[1] ** 0.5 if scale is None else scale
    p = np.exp((q @ k.T) * scale - np.asarray(lse, dtype=np.float64)[:, None])
    if causal:
        p = np.where(np.tril(np.ones(p.shape, dtype=bool)), p, 0.0)
    delta = (g * out).sum(axis=1, keepdims=True)
    ds = p * (g @ v.T - delta) * scale
    return ds @ k, ds.T @ q, p.T @ g


# ---- decoder glue (cpu_lm.py) --------------------------------------------------

def embedding(weight, ids, width) -> list[float]:
    """cpu_lm.embedding (src/qutai/backends/cpu_lm.py:54-58)."""
    return [weight[token * width + j] for token in ids for j in range(width)]


def embedding_backward(gradient, ids, count, width) -> list[float]:
    """cpu_lm.embedding_backward (cpu_lm.py:61-66)."""
    result = [0.0] * (count * width)
    for i, token in enumerate(ids):
        for j in range(width):
            result[token * width + j] += gradient[i * width + j]
    return result


def rms_norm(values, weight, width, eps):
    """cpu_lm.rms_norm (cpu_lm.py:69-81): (out, inverse)."""
    rows = len(values) // width
    out, inverse = [0.0] * len(values), [0.0] * rows
    for row in range(rows):
        inv = 1 / sqrt(sum(values[row * width + j] ** 2 for j in range(width)) / width + eps)
        inverse[row] = inv
        for j in range(width):
            out[row * width + j] = values[row * width + j] * inv * weight[j]
    return out, inverse


def rms_norm_backward(gradient, values, weight, inverse, width):
    """cpu_lm.rms_norm_backward (cpu_lm.py:84-104): (dx, dw)."""
    dx, dw = [0.0] * len(values), [0.0] * width
    for row in range(len(inverse)):
        inv = inverse[row]
        projected = sum(gradient[row * width + j] * weight[j] * values[row * width + j] for j in range(width)) / width
        for j in range(width):
            i = row * width + j
            dx[i] = inv * (gradient[i] * weight[j] - values[i] * inv * inv * projected)
            dw[j] += gradient[i] * values[i] * inv
    return dx, dw


def silu_backward(gradient, values) -> list[float]:
    """cpu_lm.silu_backward (cpu_lm.py:114-122)."""
    out = []
    for g, x in zip(gradient, values):
        s = 1 / (1 + exp(-x)) if x >= 0 else exp(x) / (1 + exp(x))
        out.append(g * s * (1 + x * (1 - s)))
    return out


def rope(values, batch, time, heads, dim, theta, offset=0, inverse=False) -> list[float]:
    """cpu_lm.rope (cpu_lm.py:125-138)."""
    out = [0.0] * len(values)
    for b in range(batch):
        for t in range(time):
            for h in range(heads):
                for j in range(0, dim, 2):
                    angle = (offset + t) * theta ** (-j / dim) * (-1 if inverse else 1)
                    c, s = cos(angle), sin(angle)
                    i = ((b * time + t) * heads + h) * dim + j
                    out[i], out[i + 1] = values[i] * c - values[i + 1] * s, values[i] * s + values[i + 1] * c
    return out


def head_rows(values, start, count, width, time) -> list[float]:
    """cpu_lm.head_rows (cpu_lm.py:323-331)."""
    return [values[(row // (time - 1) * time + row % (time - 1)) * width + j]
            for row in range(start, start + count) for j in range(width)]


def head_rows_backward(target, gradient, start, count, width, time):
    """cpu_lm.head_rows_backward (cpu_lm.py:334-338), in place on the list."""
    for row in range(count):
        at = (start + row) // (time - 1) * time + (start + row) % (time - 1)
        for j in range(width):
            target[at * width + j] += gradient[row * width + j]


def head_loss(logits, labels, rows, vocab, *, start=0) -> float:
    """cpu_lm.head_loss (cpu_lm.py:345-355): summed cross entropy, -100 ignored."""
    result = 0.0
    for row in range(rows):
        label = labels[start + row]
        if label == -100:
            continue
        peak = max(logits[row * vocab + j] for j in range(vocab))
        result += log(sum(exp(logits[row * vocab + j] - peak) for j in range(vocab))) - (
            logits[row * vocab + label] - peak)
    return result


def head_gradient(logits, labels, rows, vocab, gradient, count, *, start=0) -> list[float]:
    """cpu_lm.head_gradient (cpu_lm.py:358-371), returned as a new list."""
    out = list(logits)
    for row in range(rows):
        label = labels[start + row]
        peak = max(logits[row * vocab + j] for j in range(vocab))
        total = sum(exp(logits[row * vocab + j] - peak) for j in range(vocab))
        for j in range(vocab):
            out[row * vocab + j] = (0 if label == -100 else
                                    gradient[0] / count * (exp(logits[row * vocab + j] - peak) / total - (j == label)))
    return out


# ---- compiled float64 GEMM -----------------------------------------------------

_lib = None


def build() -> Path:
    """Compile oracle/gemm_f64.c (gcc, -ffp-contract=off) into oracle/_build."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIBRARY


def _library():
    global _lib
    if _lib is None:
        if not LIBRARY.exists():
            build()
        lib = ctypes.CDLL(str(LIBRARY))
        lib.oracle_gemm_f64.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int64] * 3 + [ctypes.c_int] * 3 + [
            ctypes.c_void_p, ctypes.c_int64, ctypes.c_int]
        lib.oracle_gemm_f64.restype = ctypes.c_int
        lib.oracle_bf16_round.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        lib.oracle_bf16_round.restype = None
        _lib = lib
    return _lib


def gemm_f64(a, b, rows, inner, cols, *, transpose_left=False, transpose_right=False, row_list=None, out=None,
             accumulate=False, threads=None) -> np.ndarray:
    """Compiled restatement of ``gemm`` (bit-identical).  ``a``/``b`` are
    float64 arrays in the reference layouts; ``row_list`` restricts the
    output to those rows (result shape [len(row_list), cols])."""
    a = np.ascontiguousarray(a, dtype=np.float64).ravel()
    b = np.ascontiguousarray(b, dtype=np.float64).ravel()
    if a.size < rows * inner or b.size < inner * cols:
        raise ValueError("operand too small")
    selected = None if row_list is None else np.ascontiguousarray(row_list, dtype=np.int64)
    n = rows if selected is None else selected.size
    result = np.zeros((n, cols)) if out is None else np.array(out, dtype=np.float64).reshape(n, cols)
    threads = threads or min(16, os.cpu_count() or 1)
    status = _library().oracle_gemm_f64(
        a.ctypes.data, b.ctypes.data, result.ctypes.data, rows, inner, cols, int(transpose_left),
        int(transpose_right), int(accumulate), None if selected is None else selected.ctypes.data, n, threads)
    if status:
        raise MemoryError("oracle allocation failed")
    return result


def bf16_round_c(x: np.ndarray) -> np.ndarray:
    """C restatement of the RNE encoder; returns the bf16 words."""
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    y = np.empty(x.size, dtype=np.uint16)
    _library().oracle_bf16_round(x.ctypes.data, y.ctypes.data, x.size)
    return y


def bf16_words(x: np.ndarray) -> np.ndarray:
    """numpy restatement of the RNE encoder (fp32 -> bf16 words)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return np.where(nan, (u >> 16) | 0x40, rounded).astype(np.uint16)


def bf16_values(words: np.ndarray) -> np.ndarray:
    """bf16 words -> fp32 values (exact)."""
    return (np.asarray(words, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_round_array(x: np.ndarray) -> np.ndarray:
    return bf16_values(bf16_words(x)).reshape(np.shape(x))


def rel_frobenius(got, ref) -> float:
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    denominator = np.linalg.norm(ref)
    return float(np.linalg.norm(got - ref) / denominator) if denominator else float(np.linalg.norm(got - ref))
