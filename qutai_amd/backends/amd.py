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

import ctypes
import struct
from array import array
from collections.abc import Iterable
from itertools import product
from builtins import sum as _add_up  # the module defines the reference's `sum`
from math import prod

from .amd_runtime import get_runtime
from .precision import matmul_precision
from .storage import Storage
from ..core.shape import broadcast_shape, normalize_axis, strides, transpose_axes

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


# The storage class under the name the reference's serialization and
# checkpoint code spells `cuda.CUDAStorage` (core/serialization.py:69,
# lm/checkpoint.py:89): constructor (size, dtype), `ptr`, `nbytes`, `runtime`.
storage_class = AMDStorage


def normal(size: int, mean: float = 0.0, std: float = 1.0, *, seed=None, dtype: str = "float32") -> AMDStorage:
    """N(mean, std) values (cuda.normal, src/qutai/backends/cuda.py:297-302,
    called by nn Dropout, nn/layers.py:87): drawn on the host with
    Random(seed).gauss, as the CPU path draws them (cpu_lm.py:6-8), and
    uploaded once."""
    if dtype not in ("float32", "float64"):
        raise ValueError("normal draws float32 or float64 values")
    from random import Random

    draw = Random(seed)
    return storage(array("d", (draw.gauss(mean, std) for _ in range(size))), dtype=dtype)


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


def cast_into(target: AMDStorage, source: AMDStorage) -> None:
    """``target`` (e.g. a view into a larger block) receives ``source``'s values
    in its own dtype: the conversion of ``from_storage`` without a new
    allocation."""
    if target.device != "amd" or source.device != "amd" or target.size != source.size:
        raise ValueError("cast_into needs two amd storages of one element count")
    if target.dtype == source.dtype:
        copy_into(target, source)
    elif source.size:
        target.runtime.call("qutai_amd_cast", source.ptr, target.ptr, source.size, code(source.dtype),
                            code(target.dtype))


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
        offset_a = _add_up(p * steps_a[d] for d, p in enumerate(coordinate) if a[d] != 1)
        offset_b = _add_up(p * steps_b[d] for d, p in enumerate(coordinate) if b[d] != 1)
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


_FLOATS = ("float32", "float64", "bfloat16")
_MAX_RANK = 8


def _item(dtype: str) -> int:
    return _TYPES[dtype][1]


def _copy_strided(source: AMDStorage, target: AMDStorage, dims, source_steps, target_steps, *, source_offset=0,
                  target_offset=0) -> None:
    """target[offset + c . target_steps] = source[offset + c . source_steps]
    for every coordinate c of ``dims`` (one strided-copy launch)."""
    dims = tuple(dims) or (1,)
    source_steps = tuple(source_steps) or (1,)
    target_steps = tuple(target_steps) or (1,)
    if not prod(dims):
        return
    if len(dims) > _MAX_RANK:
        raise ValueError(f"the amd device copies tensors of at most {_MAX_RANK} dimensions")
    rank = len(dims)
    array_type = ctypes.c_int64 * rank
    item = _item(source.dtype)
    get_runtime().call("qutai_amd_strided_copy", source.ptr + source_offset * item, target.ptr + target_offset * item,
                       rank, array_type(*dims), array_type(*source_steps), array_type(*target_steps), item)


def _span(shape, steps, offset) -> tuple[int, int]:
    """Lowest and highest element a strided view of ``shape`` touches."""
    low = high = offset
    for size, step in zip(shape, steps):
        if size > 1:
            low += min(0, (size - 1) * step)
            high += max(0, (size - 1) * step)
    return low, high


def broadcast(values: AMDStorage, shape, target) -> AMDStorage:
    """``values`` of ``shape`` repeated to ``target`` (src/qutai/backends/cuda.py:245-252):
    the same storage when the shapes agree, else a new one; size-1 axes
    (and missing leading axes) are read with stride 0."""
    shape, target = tuple(shape), tuple(target)
    if shape == target:
        return values
    if len(shape) > len(target):
        raise ValueError(f"shape {shape} cannot broadcast to {target}")
    padded = (1,) * (len(target) - len(shape)) + shape
    if any(n != 1 and n != t for n, t in zip(padded, target)):
        raise ValueError(f"shape {shape} cannot broadcast to {target}")
    if values.size != prod(shape):
        raise ValueError("storage size does not match the broadcast source shape")
    steps = tuple(0 if n == 1 else step for n, step in zip(padded, strides(padded)))
    result = AMDStorage(prod(target), values.dtype)
    _copy_strided(values, result, target, steps, strides(target))
    return result


def transpose(values: AMDStorage, shape, axes=None) -> AMDStorage:
    """Any axis permutation (src/qutai/backends/cuda.py:255-262), reversed
    axes when ``axes`` is None.  A swap of the last two axes runs through
    32x32 LDS tiles (both sides coalesced); every other permutation is one
    strided copy whose innermost runs stay 16-byte vectors when the last
    axis does not move."""
    shape = tuple(shape)
    rank = len(shape)
    order = transpose_axes(rank, axes)
    if values.size != prod(shape):
        raise ValueError("storage size does not match the shape")
    target = tuple(shape[a] for a in order)
    result = AMDStorage(values.size, values.dtype)
    if not values.size:
        return result
    if rank >= 2 and order == tuple(range(rank - 2)) + (rank - 1, rank - 2):
        result.runtime.call("qutai_amd_transpose_last2", values.ptr, result.ptr, prod(shape[:-2]), shape[-2],
                            shape[-1], code(values.dtype))
        return result
    source_steps = strides(shape)
    _copy_strided(values, result, target, tuple(source_steps[a] for a in order), strides(target))
    return result


def concatenate(values, shapes, axis=0) -> AMDStorage:
    """Pieces joined along ``axis`` (src/qutai/backends/cuda.py:383-394): one
    strided copy per piece into its column range of the [outer][total]
    result."""
    shapes = [tuple(shape) for shape in shapes]
    if not values or len(values) != len(shapes):
        raise ValueError("concatenate needs one shape per storage")
    rank = len(shapes[0])
    axis = normalize_axis(axis, rank)
    if len({v.dtype for v in values}) != 1 or any(len(s) != rank for s in shapes):
        raise ValueError("concatenate needs storages of one dtype and shapes of one rank")
    if any(s[:axis] != shapes[0][:axis] or s[axis + 1:] != shapes[0][axis + 1:] for s in shapes):
        raise ValueError("concatenate needs equal shapes outside the joined axis")
    outer = prod(shapes[0][:axis])
    sizes = [prod(shape[axis:]) for shape in shapes]
    total = _add_up(sizes)
    result = AMDStorage(outer * total, values[0].dtype)
    start = 0
    for data, size in zip(values, sizes):
        if data.size != outer * size:
            raise ValueError("storage size does not match its shape")
        _copy_strided(data, result, (outer, size), (size, 1), (total, 1), target_offset=start)
        start += size
    return result


def gather_slice(values: AMDStorage, shape, steps, offset) -> AMDStorage:
    """Strided view read (src/qutai/backends/cuda.py:237-238): element c of
    the result is values[offset + c . steps]."""
    shape, steps = tuple(shape), tuple(steps)
    low, high = _span(shape, steps, offset)
    if prod(shape) and (low < 0 or high >= values.size):
        raise IndexError("slice outside the storage")
    result = AMDStorage(prod(shape), values.dtype)
    _copy_strided(values, result, shape, steps, strides(shape), source_offset=offset)
    return result


def scatter_slice(values: AMDStorage, shape, steps, offset, size) -> AMDStorage:
    """Inverse of ``gather_slice`` (src/qutai/backends/cuda.py:241-242): a
    zero storage of ``size`` with ``values`` written at offset + c . steps."""
    shape, steps = tuple(shape), tuple(steps)
    if values.size != prod(shape):
        raise ValueError("storage size does not match the slice shape")
    low, high = _span(shape, steps, offset)
    if prod(shape) and (low < 0 or high >= size):
        raise IndexError("slice outside the storage")
    result = full(size, 0.0, dtype=values.dtype)
    _copy_strided(values, result, shape, strides(shape), steps, target_offset=offset)
    return result


def _positions(positions, limit: int):
    index = positions if isinstance(positions, array) and positions.typecode == "q" else array("q", positions)
    if index and (min(index) < 0 or max(index) >= limit):
        raise IndexError("position outside the storage")
    return storage(index, dtype="int64"), index


def gather(values: AMDStorage, positions) -> AMDStorage:
    """values[positions[i]] for each i (src/qutai/backends/cuda.py:211-215)."""
    device_index, index = _positions(positions, values.size)
    result = AMDStorage(len(index), values.dtype)
    if len(index):
        result.runtime.call("qutai_amd_gather", values.ptr, device_index.ptr, result.ptr, len(index),
                            _item(values.dtype))
    return result


def _group_by_target(index, size: int):
    """CSR grouping of source positions by target, in one counting pass:
    ``start`` (size + 1 offsets) and ``order`` (the source indices of each
    target in input order, target by target).  O(n + size); stable, so
    repeated positions add up in input order."""
    start = array("q", bytes(8 * (size + 1)))
    for position in index:
        start[position + 1] += 1
    for t in range(size):
        start[t + 1] += start[t]
    cursor = start[:size]
    order = array("q", bytes(8 * len(index)))
    for i, position in enumerate(index):
        order[cursor[position]] = i
        cursor[position] += 1
    return start, order


def scatter(values: AMDStorage, positions, size: int) -> AMDStorage:
    """Zeros of ``size`` with values[i] added at positions[i]
    (src/qutai/backends/cuda.py:218-226).  Repeated positions add up in
    input order: the sources of every target are grouped on the host and
    summed by one lane, so the result is deterministic."""
    if values.dtype not in _FLOATS:
        raise ValueError("scatter accumulates floating storages only")
    index = positions if isinstance(positions, array) and positions.typecode == "q" else array("q", positions)
    if len(index) != values.size:
        raise ValueError("scatter needs one position per value")
    if index and (min(index) < 0 or max(index) >= size):
        raise IndexError("position outside the storage")
    counts, order = _group_by_target(index, size)
    start = storage(counts, dtype="int64")
    sources = storage(order, dtype="int64") if order else None
    result = AMDStorage(size, values.dtype)
    if size:
        result.runtime.call("qutai_amd_scatter", values.ptr, start.ptr, _p(sources), result.ptr, size,
                            code(values.dtype))
    return result


# element-wise arithmetic (binary and unary op codes of qutai_amd_binary / qutai_amd_unary)
_ADD, _SUBTRACT, _MULTIPLY, _DIVIDE = 0, 1, 2, 3
(_NEGATE, _SQUARE, _SCALE, _RELU, _RELU_BACKWARD, _GELU, _GELU_BACKWARD, _EXP, _LOG, _TANH, _ATAN, _TANH_BACKWARD,
 _ATAN_BACKWARD, _DIVIDE_SCALAR) = range(14)


class _Flag:
    """A device int32 that a kernel sets when it meets an invalid operand."""

    def __init__(self):
        self.runtime = get_runtime()
        self.ptr = self.runtime.allocate(4)

    def __del__(self):
        if getattr(self, "ptr", 0):
            self.runtime.free(self.ptr)
            self.ptr = 0

    def raised(self) -> bool:
        value = array("i", [0])
        self.runtime.download(self.ptr, value)
        return bool(value[0])


def _binary(left: AMDStorage, right: AMDStorage, operation: int, out: AMDStorage | None = None) -> AMDStorage:
    if left.dtype == "int64":
        raise ValueError("int64 index storages take no arithmetic")
    if (left.size, left.dtype) != (right.size, right.dtype):
        raise ValueError("element-wise operations need equal element counts and dtypes")
    result = out if out is not None else AMDStorage(left.size, left.dtype)
    flag = _Flag() if operation == _DIVIDE and left.size else None
    if left.size:
        result.runtime.call("qutai_amd_binary", left.ptr, right.ptr, result.ptr, left.size, operation,
                            code(left.dtype), _p(flag))
    if flag is not None and flag.raised():
        raise ZeroDivisionError("division by zero")
    return result


def _unary(values: AMDStorage, operation: int, factor: float = 0.0, gradient: AMDStorage | None = None,
           out: AMDStorage | None = None) -> AMDStorage:
    if values.dtype not in _FLOATS:
        raise ValueError("element-wise functions take real floating storages")
    if gradient is not None and (gradient.size, gradient.dtype) != (values.size, values.dtype):
        raise ValueError("gradient and values need equal element counts and dtypes")
    result = out if out is not None else AMDStorage(values.size, values.dtype)
    flag = _Flag() if operation == _LOG and values.size else None
    if values.size:
        result.runtime.call("qutai_amd_unary", values.ptr, _p(gradient), result.ptr, values.size, operation,
                            float(factor), code(values.dtype), _p(flag))
    if flag is not None and flag.raised():
        raise ValueError("the natural logarithm needs positive inputs")
    return result


def add(left: AMDStorage, right: AMDStorage) -> AMDStorage:
    """left + right (src/qutai/backends/cuda.py:186)."""
    return _binary(left, right, _ADD)


def subtract(left: AMDStorage, right: AMDStorage) -> AMDStorage:
    """left - right (src/qutai/backends/cuda.py:187)."""
    return _binary(left, right, _SUBTRACT)


def multiply(left: AMDStorage, right: AMDStorage) -> AMDStorage:
    """left * right (src/qutai/backends/cuda.py:188)."""
    return _binary(left, right, _MULTIPLY)


def divide(left: AMDStorage, right: AMDStorage) -> AMDStorage:
    """left / right; ZeroDivisionError when a divisor is zero, found on the
    device and read back as the reference does (src/qutai/backends/cuda.py:189,
    171-183)."""
    return _binary(left, right, _DIVIDE)


def add_into(target: AMDStorage, source: AMDStorage) -> None:
    """target += source in place (src/qutai/backends/cuda.py:141-147)."""
    if (target.device, target.dtype, target.size) != (source.device, source.dtype, source.size):
        raise ValueError("add_into needs storages of one device, dtype and size")
    if target.dtype == "int64":
        raise ValueError("index storages take no gradient accumulation")
    _binary(target, source, _ADD, out=target)


def scale_into(values: AMDStorage, factor: float) -> None:
    """values *= factor in place (src/qutai/backends/cuda.py:150-154)."""
    if values.dtype == "int64":
        raise ValueError("index storages take no scaling")
    _unary(values, _SCALE, factor, out=values)


def _real(value: float, dtype: str) -> float:
    """``value`` as the kernel's arithmetic type sees it (fp32 for fp32/bf16)."""
    return value if dtype == "float64" else struct.unpack("<f", struct.pack("<f", value))[0]


def divide_scalar(values: AMDStorage, value: float) -> AMDStorage:
    """values / value (src/qutai/backends/cuda.py:192-195); the divisor is
    rounded to the arithmetic type first and a zero one raises
    ZeroDivisionError on the host."""
    divisor = _real(float(value), values.dtype)
    if divisor == 0 and values.size:
        raise ZeroDivisionError("division by zero")
    return _unary(values, _DIVIDE_SCALAR, divisor)


def negate(values):
    return _unary(values, _NEGATE)


def square(values):
    return _unary(values, _SQUARE)


def relu(values):
    return _unary(values, _RELU)


def relu_backward(gradient, values):
    return _unary(values, _RELU_BACKWARD, gradient=gradient)


def gelu(values):
    return _unary(values, _GELU)


def gelu_backward(gradient, values):
    return _unary(values, _GELU_BACKWARD, gradient=gradient)


def exp(values):
    return _unary(values, _EXP)


def log(values):
    """Natural log; ValueError when some input is not positive
    (src/qutai/backends/cuda.py:204, 157-168)."""
    return _unary(values, _LOG)


def tanh(values):
    return _unary(values, _TANH)


def atan(values):
    return _unary(values, _ATAN)


def tanh_backward(gradient, values):
    return _unary(values, _TANH_BACKWARD, gradient=gradient)


def atan_backward(gradient, values):
    return _unary(values, _ATAN_BACKWARD, gradient=gradient)


def add_widen(left: AMDStorage, right: AMDStorage) -> AMDStorage:
    """fp32 left + bf16 right (exactly widened), fp32 result."""
    if left.dtype != "float32" or right.dtype != "bfloat16" or left.size != right.size:
        raise ValueError("add_widen takes float32 + bfloat16 storages of one size")
    result = AMDStorage(left.size, "float32")
    if left.size:
        result.runtime.call("qutai_amd_add_widen", left.ptr, right.ptr, result.ptr, left.size)
    return result


def scale(values: AMDStorage, factor: float) -> AMDStorage:
    """values * factor (src/qutai/backends/cuda.py:198)."""
    result = AMDStorage(values.size, values.dtype)
    if values.size:
        result.runtime.call("qutai_amd_scale", values.ptr, result.ptr, values.size, float(factor), code(values.dtype))
    return result


# reductions over one axis
def _reduce(values: AMDStorage, outer: int, width: int, inner: int) -> AMDStorage:
    result = AMDStorage(outer * inner, values.dtype)
    if not result.size:
        return result
    runtime = get_runtime()
    need = runtime.lib.qutai_amd_reduce_sum_workspace_size(outer, width, inner, code(values.dtype))
    workspace = AMDStorage((need + 3) // 4, "float32") if need else None
    runtime.call("qutai_amd_reduce_sum", values.ptr, result.ptr, outer, width, inner, code(values.dtype),
                 _p(workspace), workspace.nbytes if workspace is not None else 0)
    return result


def _axis_split(size: int, shape, axis) -> tuple[int, int, int]:
    if axis is None:
        return 1, size, 1
    if shape is None:
        raise ValueError("a sum over an axis needs the shape")
    shape = tuple(shape)
    axis = normalize_axis(axis, len(shape))
    return prod(shape[:axis]), shape[axis], prod(shape[axis + 1:])


def sum(values: AMDStorage, shape=None, axis=None) -> AMDStorage:  # noqa: A001 - the reference's name
    """Sum of everything (axis None) or over one axis
    (src/qutai/backends/cuda.py:265-274), fp32 accumulation (fp64 for fp64)."""
    if values.dtype not in _FLOATS:
        raise ValueError("sum takes real floating storages")
    return _reduce(values, *_axis_split(values.size, shape, axis))


def mean(values: AMDStorage, shape=None, axis=None) -> AMDStorage:
    """Average over everything or one axis (src/qutai/backends/cuda.py:277-280)."""
    count = _axis_split(values.size, shape, axis)[1]
    if not count:
        raise ValueError("the mean of no elements is undefined")
    return scale(sum(values, shape, axis), 1 / count)


def unbroadcast(values: AMDStorage, shape, target) -> AMDStorage:
    """Sum a gradient of ``shape`` down to the broadcast source ``target``
    (src/qutai/backends/cuda.py:283-289): every axis that ``target`` holds
    as 1 (or lacks) is summed, keeping its place."""
    shape, target = tuple(shape), tuple(target)
    padded = (1,) * (len(shape) - len(target)) + target
    current, current_shape = values, shape
    for axis, (length, original) in enumerate(zip(shape, padded)):
        if original == 1 and length != 1:
            current = sum(current, current_shape, axis)
            current_shape = current_shape[:axis] + (1,) + current_shape[axis + 1:]
    return current


def softmax(values: AMDStorage, shape, axis, *, scale: float = 1.0) -> AMDStorage:
    """Stable softmax along any axis (src/qutai/backends/cuda.py:464-472);
    ``scale`` multiplies the input first (the 1/sqrt(D) of attention scores)."""
    shape = tuple(shape)
    axis = normalize_axis(axis, len(shape))
    outer, width, inner = prod(shape[:axis]), shape[axis], prod(shape[axis + 1:])
    result = AMDStorage(values.size, values.dtype)
    if values.size:
        result.runtime.call("qutai_amd_softmax", values.ptr, result.ptr, outer, width, inner, float(scale),
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
    return _reduce(values, 1, rows, cols)


def sum_all(values: AMDStorage) -> AMDStorage:
    """Sum of all elements as a one-element storage."""
    return _reduce(values, 1, values.size, 1)


def broadcast_scalar(value: AMDStorage, size: int) -> AMDStorage:
    """A [size] storage holding the single element of ``value``."""
    return broadcast(value, (1,), (size,))
