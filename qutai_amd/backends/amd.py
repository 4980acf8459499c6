"""MI355X backend module (device string ``"amd"``).

A drop-in sibling of the reference CUDA backend module
(src/qutai/backends/cuda.py): the same function names, argument meaning,
dtype rules and exception types for the operations on the GEMM path, so the
reference's callers (``operations.matmul`` and its gradient, ``nn.Linear``,
the ``lm`` projections) can select it through ``device=``.  Every function
enqueues libqutai_amd kernels on the default stream; ``tolist`` is the
explicit synchronising read.  There is no CPU fallback: when the native
library or the GPU is missing, the first device touch raises.
"""
from __future__ import annotations

import struct
from array import array
from collections.abc import Iterable
from itertools import product
from math import isqrt, prod

from .amd_runtime import get_runtime
from .precision import matmul_precision
from .storage import Storage
from ..core.shape import broadcast_shape, strides

# dtype -> (array typecode, item size); the order gives the C-ABI dtype codes
# (same table as src/qutai/backends/cuda.py:17).
_TYPES = {"float32": ("f", 4), "float64": ("d", 8), "complex64": ("f", 8), "complex128": ("d", 16),
          "int64": ("q", 8), "bfloat16": ("H", 2)}
_CODES = {name: index for index, name in enumerate(_TYPES)}
_SUPPORTED = ("float32", "float64", "int64", "bfloat16")


def code(dtype: str) -> int:
    return _CODES[dtype]


class AMDStorage(Storage):
    """Owns one device allocation; ``tolist`` is the synchronising read."""
    device = "amd"

    def __init__(self, size: int, dtype: str = "float32") -> None:
        if dtype not in _SUPPORTED:
            raise ValueError(f"the amd device does not support dtype {dtype}")
        if size < 0:
            raise ValueError("storage size must be non-negative")
        self.dtype, self._size = dtype, size
        self.runtime = get_runtime()
        self.ptr = self.runtime.allocate(self.nbytes)

    @property
    def size(self) -> int:
        return self._size

    @property
    def nbytes(self) -> int:
        return self._size * _TYPES[self.dtype][1]

    def __len__(self) -> int:
        return self._size

    def __del__(self) -> None:
        if getattr(self, "ptr", 0):
            self.runtime.free(self.ptr)
            self.ptr = 0

    def copy(self) -> AMDStorage:
        result = AMDStorage(self.size, self.dtype)
        self.runtime.copy(result.ptr, self.ptr, self.nbytes)
        return result

    def to_array(self) -> array:
        """Raw host copy (bfloat16 as 16-bit words)."""
        buffer = array(_TYPES[self.dtype][0], bytes(self.nbytes))
        self.runtime.download(self.ptr, buffer)
        return buffer

    def tolist(self):
        buffer = self.to_array()
        if self.dtype == "bfloat16":
            widened = array("I", (value << 16 for value in buffer))
            return array("f", widened.tobytes()).tolist()
        return buffer.tolist()


class AMDView(AMDStorage):
    """Elements [offset, offset + size) of another amd storage, sharing its
    memory: it holds the parent alive and never frees anything itself."""

    def __init__(self, base: AMDStorage, offset: int, size: int) -> None:
        if not isinstance(base, AMDStorage) or offset < 0 or size < 0 or offset + size > base.size:
            raise ValueError("view outside its storage")
        self.dtype, self._size, self.runtime, self.base = base.dtype, size, base.runtime, base
        self.ptr = base.ptr + offset * _TYPES[base.dtype][1]

    def __del__(self) -> None:
        pass


def view(base: AMDStorage, offset: int, size: int) -> AMDView:
    return AMDView(base, offset, size)


def _p(value) -> int:
    return value.ptr if value is not None else 0


def is_available() -> bool:
    try:
        get_runtime()
        return True
    except (OSError, RuntimeError):
        return False


def synchronize() -> None:
    get_runtime().synchronize()


def memory_stats():
    return get_runtime().memory_stats()


def reset_peak_memory_stats():
    get_runtime().reset_peak_memory_stats()


def empty_cache():
    get_runtime().empty_cache()


def _bf16_bits(value: float) -> int:
    """Host bfloat16 encoder: round to nearest even, NaN kept quiet
    (src/qutai/backends/cuda.py:98-101)."""
    bits = struct.unpack("<I", struct.pack("<f", value))[0]
    if bits & 0x7FFFFFFF > 0x7F800000:
        return (bits >> 16) | 0x40
    return (bits + 0x7FFF + ((bits >> 16) & 1)) >> 16


def storage(values: Iterable = (), *, dtype: str = "float64") -> AMDStorage:
    """Upload host values (an iterable, or an ``array``/buffer of the
    dtype's item type) into a new device storage.  bfloat16 input is
    uploaded as float32 and rounded on the device with the same RNE rule."""
    if isinstance(values, Storage):
        return from_storage(values, dtype=dtype)
    if dtype not in _SUPPORTED:
        raise ValueError(f"the amd device does not support dtype {dtype}")
    if dtype == "bfloat16":
        wide = values if isinstance(values, array) and values.typecode == "f" else array("f", values)
        staged = AMDStorage(len(wide), "float32")
        staged.runtime.upload(staged.ptr, wide)
        return from_storage(staged, dtype="bfloat16")
    typecode = _TYPES[dtype][0]
    buffer = values if isinstance(values, array) and values.typecode == typecode else array(typecode, values)
    result = AMDStorage(len(buffer), dtype)
    result.runtime.upload(result.ptr, buffer)
    return result


def full(size: int, value: float = 0.0, *, dtype: str = "float64") -> AMDStorage:
    result = AMDStorage(size, dtype)
    if size:
        result.runtime.call("qutai_amd_fill", result.ptr, size, float(value), code(dtype))
    return result


def from_storage(values: Storage, *, dtype: str) -> AMDStorage:
    if values.device != "amd":
        return storage(values.tolist(), dtype=dtype)
    if values.dtype == dtype:
        return values.copy()
    result = AMDStorage(values.size, dtype)
    if values.size:
        result.runtime.call("qutai_amd_cast", values.ptr, result.ptr, values.size, code(values.dtype), code(dtype))
    return result


def copy_into(target: AMDStorage, source: AMDStorage) -> None:
    if (target.device, target.dtype, target.size) != (source.device, source.dtype, source.size):
        raise ValueError("copy needs the same device, dtype and element count")
    target.runtime.copy(target.ptr, source.ptr, target.nbytes)


def take(values: AMDStorage, start: int, size: int) -> AMDStorage:
    """Contiguous slice copy (src/qutai/backends/cuda_lm.py:58-62)."""
    if start < 0 or size < 0 or start + size > values.size:
        raise ValueError("slice out of range")
    result = AMDStorage(size, values.dtype)
    item = _TYPES[values.dtype][1]
    result.runtime.copy(result.ptr, values.ptr + start * item, size * item)
    return result


def gemm(left, right, rows, inner, cols, *, batch=1, transpose_left=False, transpose_right=False,
         left_stride=None, right_stride=None, out_dtype=None, out=None, accumulate=False):
    """Batched GEMM; bf16 inputs accumulate in fp32; ``out`` receives or accumulates the result.

    Argument meaning, dtype resolution and validation are those of the
    reference boundary ``cuda.gemm`` (src/qutai/backends/cuda.py:305-337):
    A is rows x inner (inner x rows when transpose_left), B is inner x cols
    (cols x inner when transpose_right), per-batch strides default to the
    dense sizes and 0 broadcasts; the result is [batch][rows][cols].
    """
    if not isinstance(left, AMDStorage) or not isinstance(right, AMDStorage):
        raise ValueError("GEMM inputs must be amd storages")
    allowed = ("float32", "bfloat16", "float64")
    if left.dtype not in allowed or right.dtype not in allowed:
        raise ValueError("GEMM supports float32, bfloat16 and float64 only")
    double = left.dtype == "float64" or right.dtype == "float64"
    if double and left.dtype != right.dtype:
        raise ValueError("float64 GEMM needs both inputs in float64")
    dtype = ("float64" if double else "float32") if out_dtype is None else out_dtype
    if dtype not in (("float64",) if double else ("float32", "bfloat16")):
        raise ValueError("GEMM output dtype is incompatible with the inputs")
    if any(type(x) is not int or x < 0 for x in (rows, inner, cols, batch)):
        raise ValueError("GEMM dimensions must be non-negative integers")
    sa = rows * inner if left_stride is None else left_stride
    sb = inner * cols if right_stride is None else right_stride
    if any(type(x) is not int or x < 0 for x in (sa, sb)):
        raise ValueError("GEMM batch strides must be non-negative integers")
    if batch and (left.size < (batch - 1) * sa + rows * inner or right.size < (batch - 1) * sb + inner * cols):
        raise ValueError("GEMM input storage is too small")
    if accumulate and out is None:
        raise ValueError("GEMM accumulation needs out")
    size = batch * rows * cols
    if out is not None:
        if not isinstance(out, AMDStorage) or out.dtype != dtype or out.size != size:
            raise ValueError("GEMM out has the wrong device, dtype or size")
        for value in (left, right):
            if out.nbytes and value.nbytes and out.ptr < value.ptr + value.nbytes and value.ptr < out.ptr + out.nbytes:
                raise ValueError("GEMM out must not share memory with an input")
    result = out if out is not None else AMDStorage(size, dtype)
    if not size:
        return result
    mixed = not double and (left.dtype == "bfloat16" or right.dtype == "bfloat16" or matmul_precision() == "bfloat16")
    runtime = get_runtime()
    workspace = None
    if not double:
        need = runtime.lib.qutai_amd_gemm_workspace_size(rows, inner, cols, batch, sa, sb, int(bool(transpose_left)),
                                                         int(bool(transpose_right)), code(left.dtype),
                                                         code(right.dtype), int(mixed))
        if need:
            workspace = AMDStorage((need + 1) // 2, "bfloat16")
    runtime.call("qutai_amd_gemm", left.ptr, right.ptr, result.ptr, rows, inner, cols, batch, sa, sb,
                 int(bool(transpose_left)), int(bool(transpose_right)), code(left.dtype), code(right.dtype),
                 code(dtype), int(bool(accumulate)), int(mixed), _p(workspace),
                 workspace.nbytes if workspace is not None else 0, mfma=not double)
    return result


def matmul(left, right, left_shape, right_shape):
    """Broadcast-batched matmul with the batching rules of
    src/qutai/backends/cuda.py:365-380: one strided-batched GEMM when each
    side is either unbatched or fully batched; otherwise one GEMM per
    broadcast batch coordinate."""
    if left.dtype not in ("float32", "float64", "bfloat16"):
        raise ValueError("amd matmul supports real floating storages only")
    if len(left_shape) == 1:
        left_shape = (1, *left_shape)
    if len(right_shape) == 1:
        right_shape = (*right_shape, 1)
    batches = broadcast_shape(left_shape[:-2], right_shape[:-2])
    a = (1,) * (len(batches) + 2 - len(left_shape)) + tuple(left_shape)
    b = (1,) * (len(batches) + 2 - len(right_shape)) + tuple(right_shape)
    count = prod(batches)
    rows, inner, columns = a[-2], a[-1], b[-1]
    if prod(a[:-2]) in (1, count) and prod(b[:-2]) in (1, count):
        return gemm(left, right, rows, inner, columns, batch=count,
                    left_stride=0 if prod(a[:-2]) == 1 else None,
                    right_stride=0 if prod(b[:-2]) == 1 else None, out_dtype=left.dtype)
    result = AMDStorage(count * rows * columns, left.dtype)
    steps_a, steps_b = strides(a), strides(b)
    item = _TYPES[left.dtype][1]
    for index, coordinate in enumerate(product(*(range(n) for n in batches))):
        offset_a = sum(p * steps_a[d] for d, p in enumerate(coordinate) if a[d] != 1)
        offset_b = sum(p * steps_b[d] for d, p in enumerate(coordinate) if b[d] != 1)
        view_a = _View(left, offset_a, rows * inner)
        view_b = _View(right, offset_b, inner * columns)
        view_c = _View(result, index * rows * columns, rows * columns)
        _gemm_views(view_a, view_b, view_c, rows, inner, columns, item)
    return result


class _View:
    """Sub-range of a storage used as a GEMM operand (no copy)."""

    def __init__(self, base: AMDStorage, offset: int, size: int):
        self.base, self.offset, self.size = base, offset, size


def _gemm_views(a: _View, b: _View, c: _View, rows, inner, cols, item):
    runtime = get_runtime()
    dtype = a.base.dtype
    mixed = dtype == "bfloat16" or (dtype == "float32" and matmul_precision() == "bfloat16")
    workspace = None
    if dtype != "float64":
        need = runtime.lib.qutai_amd_gemm_workspace_size(rows, inner, cols, 1, 0, 0, 0, 0, code(dtype), code(dtype),
                                                         int(mixed))
        if need:
            workspace = AMDStorage((need + 1) // 2, "bfloat16")
    runtime.call("qutai_amd_gemm", a.base.ptr + a.offset * item, b.base.ptr + b.offset * item,
                 c.base.ptr + c.offset * item, rows, inner, cols, 1, 0, 0, 0, 0, code(dtype), code(dtype),
                 code(dtype), 0, int(mixed), _p(workspace), workspace.nbytes if workspace is not None else 0,
                 mfma=dtype != "float64")


def add_widen(left: AMDStorage, right: AMDStorage) -> AMDStorage:
    """fp32 left + bf16 right (exactly widened), fp32 result."""
    if left.dtype != "float32" or right.dtype != "bfloat16" or left.size != right.size:
        raise ValueError("add_widen takes float32 + bfloat16 storages of one size")
    result = AMDStorage(left.size, "float32")
    if left.size:
        result.runtime.call("qutai_amd_add_widen", left.ptr, right.ptr, result.ptr, left.size)
    return result


def add(left: AMDStorage, right: AMDStorage) -> AMDStorage:
    if (left.dtype, left.size) != (right.dtype, right.size):
        raise ValueError("add needs equal dtype and size")
    result = AMDStorage(left.size, left.dtype)
    if left.size:
        result.runtime.call("qutai_amd_add", left.ptr, right.ptr, result.ptr, left.size, code(left.dtype))
    return result


def scale(values: AMDStorage, factor: float) -> AMDStorage:
    """values * factor (cuda.py:198)."""
    result = AMDStorage(values.size, values.dtype)
    if values.size:
        result.runtime.call("qutai_amd_scale", values.ptr, result.ptr, values.size, float(factor), code(values.dtype))
    return result


def concatenate(values, shapes, axis=0) -> AMDStorage:
    """Concatenation along ``axis`` (cuda.py:383-394): the pieces of every
    outer index copied device to device, in order."""
    rank = len(shapes[0])
    axis = axis % rank
    if len({v.dtype for v in values}) != 1 or any(len(s) != rank for s in shapes):
        raise ValueError("concatenate needs storages of one dtype and shapes of one rank")
    outer = prod(shapes[0][:axis])
    sizes = [prod(shape[axis:]) for shape in shapes]
    total = sum(sizes)
    result = AMDStorage(outer * total, values[0].dtype)
    item = _TYPES[values[0].dtype][1]
    start = 0
    for data, size in zip(values, sizes):
        for o in range(outer):
            if size:
                result.runtime.copy(result.ptr + (o * total + start) * item, data.ptr + o * size * item, size * item)
        start += size
    return result


def transpose(values: AMDStorage, shape, axes=None) -> AMDStorage:
    """Axis permutation that swaps two adjacent axes: the last two (the form
    the matmul gradient uses, src/qutai/core/operations/linalg.py:37-38) or
    any other pair (the head split and merge of nn.MultiHeadAttention,
    src/qutai/nn/layers.py:322-325, 354)."""
    rank = len(shape)
    axes = tuple(reversed(range(rank))) if axes is None else tuple(a % rank for a in axes)
    if axes == tuple(range(rank)):
        return values.copy()
    swapped = [i for i in range(rank - 1) if axes[i] == i + 1 and axes[i + 1] == i]
    if len(swapped) != 1 or any(axes[j] != j for j in range(rank) if j not in (swapped[0], swapped[0] + 1)):
        raise NotImplementedError("amd transpose swaps two adjacent axes")
    i = swapped[0]
    if i < rank - 2:
        result = AMDStorage(values.size, values.dtype)
        if values.size:
            result.runtime.call("qutai_amd_swap_axes", values.ptr, result.ptr, prod(shape[:i]), shape[i],
                                shape[i + 1], prod(shape[i + 2:]), code(values.dtype))
        return result
    rows, cols = shape[-2], shape[-1]
    batch = prod(shape[:-2])
    result = AMDStorage(values.size, values.dtype)
    if values.size:
        result.runtime.call("qutai_amd_transpose_last2", values.ptr, result.ptr, batch, rows, cols,
                            code(values.dtype))
    return result


def unbroadcast(values: AMDStorage, shape, target) -> AMDStorage:
    """Sum a gradient of ``shape`` down to the broadcast source ``target``."""
    shape, target = tuple(shape), tuple(target)
    padded = (1,) * (len(shape) - len(target)) + target
    current, current_shape = values, shape
    for axis in range(len(shape)):
        if padded[axis] == 1 and current_shape[axis] != 1:
            outer = prod(current_shape[:axis])
            inner = prod(current_shape[axis + 1:])
            reduced = AMDStorage(outer * inner, values.dtype)
            if reduced.size:
                reduced.runtime.call("qutai_amd_sum_middle", current.ptr, reduced.ptr, outer, current_shape[axis],
                                     inner, code(values.dtype))
            current = reduced
            current_shape = current_shape[:axis] + (1,) + current_shape[axis + 1:]
    return current if current is not values else values.copy()


def softmax(values: AMDStorage, shape, axis, *, scale: float = 1.0) -> AMDStorage:
    """Stable softmax along the last axis (src/qutai/backends/cuda.py:464-472);
    ``scale`` multiplies the input first (the 1/sqrt(D) of attention scores)."""
    axis %= len(shape)
    if axis != len(shape) - 1:
        raise NotImplementedError("amd softmax runs along the last axis")
    width = shape[axis]
    rows = values.size // width if width else 0
    result = AMDStorage(values.size, values.dtype)
    if values.size:
        result.runtime.call("qutai_amd_softmax_rows", values.ptr, result.ptr, rows, width, float(scale),
                            code(values.dtype))
    return result


def softmax_backward(probs: AMDStorage, gradient: AMDStorage, shape, *, scale: float = 1.0) -> AMDStorage:
    """Input gradient of ``softmax(values, shape, -1, scale=scale)`` from its
    output and output gradient: scale * p * (g - rowsum(g * p))."""
    if probs.dtype != gradient.dtype or probs.size != gradient.size:
        raise ValueError("softmax_backward needs probabilities and gradient of one dtype and size")
    width = shape[-1]
    rows = probs.size // width if width else 0
    result = AMDStorage(probs.size, probs.dtype)
    if probs.size:
        result.runtime.call("qutai_amd_softmax_backward", probs.ptr, gradient.ptr, result.ptr, rows, width,
                            float(scale), code(probs.dtype))
    return result


def causal_mask(values: AMDStorage, rows: int, width: int, length: int, offset: int = 0) -> AMDStorage:
    """Scores [rows][width] with keys after each query (row r is query
    r % length; it sees keys <= offset + r % length) set to -inf."""
    if values.size != rows * width:
        raise ValueError("causal_mask size does not match rows x width")
    result = AMDStorage(values.size, values.dtype)
    if values.size:
        result.runtime.call("qutai_amd_causal_mask", values.ptr, result.ptr, rows, width, length, offset,
                            code(values.dtype))
    return result


def add_rows(values: AMDStorage, bias: AMDStorage, rows: int, cols: int) -> AMDStorage:
    """values [rows][cols] + bias [cols] (the bias add of nn.Linear)."""
    if values.dtype != bias.dtype or values.size != rows * cols or bias.size != cols:
        raise ValueError("add_rows needs [rows][cols] values and a [cols] bias of one dtype")
    result = AMDStorage(values.size, values.dtype)
    if values.size:
        result.runtime.call("qutai_amd_add_rows", values.ptr, bias.ptr, result.ptr, rows, cols, code(values.dtype))
    return result


def sum_rows(values: AMDStorage, rows: int, cols: int) -> AMDStorage:
    """Column sums of a [rows][cols] storage (gradient of a broadcast bias)."""
    result = AMDStorage(cols, values.dtype)
    if cols:
        result.runtime.call("qutai_amd_sum_middle", values.ptr, result.ptr, 1, rows, cols, code(values.dtype))
    return result


def sum_all(values: AMDStorage) -> AMDStorage:
    """Sum of all elements, in two parallel passes of about sqrt(n) each."""
    n = values.size
    if n == 0:
        return full(1, 0.0, dtype=values.dtype)
    width = max(1, isqrt(n))
    while n % width:
        width -= 1
    partial = sum_rows(values, n // width, width)
    return sum_rows(partial, width, 1) if width > 1 else partial


def broadcast_scalar(value: AMDStorage, size: int) -> AMDStorage:
    """A [size] storage holding the single element of ``value``."""
    zeros = full(size, 0.0, dtype=value.dtype)
    return add_rows(zeros, value, size, 1)
