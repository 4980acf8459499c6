"""Matrix products of operands, with the gradient rule of a product.

Operands are anything with ``storage`` / ``shape`` / ``requires_grad``; the
result is ``(values, shape, rule)`` and nothing here touches ``Tensor``.
The semantics are those of the reference operation
(src/qutai/core/operations/linalg.py:11-56): a 1-D left operand is a row
(1, n) and a 1-D right operand a column (n, 1), those axes are dropped from
the result, batch axes broadcast, and the gradients are dA = G B^T and
dB = A^T G computed under the matmul precision of the forward pass, in the
dtype of the operand they belong to.

How the gradients are computed is this build's own plan, chosen to keep
every gradient inside the GEMM:

* equal batch axes (or none): one strided-batched GEMM per gradient with a
  transposed operand (NT for dA, TN for dB) -- no transpose pass;
* one side unbatched (its batch axes all 1): the unbatched operand's
  gradient sums over the batch, which is folded into the GEMM's reduction
  (A^T G over batch x rows at once, one TN product), and the batched
  operand's gradient is a strided-batched GEMM that reads the unbatched
  operand with batch stride 0;
* any other broadcast: the per-batch products at the broadcast batch shape
  (``backend.matmul``), summed back over the broadcast axes.
"""
from __future__ import annotations

from math import prod

from ...backends.device import get_backend
from ...backends.precision import matmul_precision, set_matmul_precision
from ..shape import broadcast_shape


def _matrix_shapes(left_shape, right_shape):
    """(left as matrix, right as matrix, result shape) of a product."""
    if not left_shape or not right_shape:
        raise ValueError("matmul operands need at least one dimension")
    a = (1, *left_shape) if len(left_shape) == 1 else tuple(left_shape)
    b = (*right_shape, 1) if len(right_shape) == 1 else tuple(right_shape)
    if a[-1] != b[-2]:
        raise ValueError(f"matrix shapes {tuple(left_shape)} and {tuple(right_shape)} are incompatible")
    batch = broadcast_shape(a[:-2], b[:-2])
    rows = () if len(left_shape) == 1 else (a[-2],)
    cols = () if len(right_shape) == 1 else (b[-1],)
    return a, b, batch + rows + cols


def matmul(left, right):
    """Vector, matrix or batch-broadcast product of two operands."""
    a, b, shape = _matrix_shapes(left.shape, right.shape)
    backend = get_backend(left.storage, right.storage)
    values = backend.matmul(left.storage, right.storage, a, b)
    return values, shape, ProductGradient(left, right, a, b, matmul_precision())


def _last_two_swapped(rank: int) -> tuple[int, ...]:
    return (*range(rank - 2), rank - 1, rank - 2)


class ProductGradient:
    """Backward rule of C = A @ B for operands of matrix shapes ``a`` and
    ``b``; returns (dA, dB), None for an operand that needs no gradient."""

    def __init__(self, left, right, a, b, precision):
        self.left, self.right, self.a, self.b, self.precision = left, right, a, b, precision
        self.batch = broadcast_shape(a[:-2], b[:-2])

    def __call__(self, gradient):
        with set_matmul_precision(self.precision):
            backend = get_backend(gradient.device)
            d_left = self._left(backend, gradient) if self.left.requires_grad else None
            d_right = self._right(backend, gradient) if self.right.requires_grad else None
        return d_left, d_right

    def _layout(self):
        """'same', 'right-shared', 'left-shared' or 'mixed' batch layout."""
        count = prod(self.batch)
        left_count, right_count = prod(self.a[:-2]), prod(self.b[:-2])
        if self.a[:-2] == self.b[:-2]:
            return "same"
        if right_count == 1 and left_count == count:
            return "right-shared"
        if left_count == 1 and right_count == count:
            return "left-shared"
        return "mixed"

    def _left(self, backend, gradient):
        """dA = G B^T (rows x inner per batch)."""
        rows, inner, cols = self.a[-2], self.a[-1], self.b[-1]
        count, dtype, right = prod(self.batch), self.left.storage.dtype, self.right.storage
        layout = self._layout() if hasattr(backend, "gemm") else "mixed"
        if layout in ("same", "right-shared"):
            return backend.gemm(gradient, right, rows, cols, inner, batch=count, transpose_right=True,
                                right_stride=0 if layout == "right-shared" else None, out_dtype=dtype)
        if layout == "left-shared":
            # one G_p B_p^T per batch, then the sum over the batch
            per_batch = backend.gemm(gradient, right, rows, cols, inner, batch=count, transpose_right=True,
                                     out_dtype=dtype)
            return backend.unbroadcast(per_batch, self.batch + (rows, inner), self.a)
        flipped = backend.transpose(right, self.b, axes=_last_two_swapped(len(self.b)))
        per_batch = backend.matmul(gradient, flipped, self.batch + (rows, cols), self.b[:-2] + (cols, inner))
        return backend.unbroadcast(per_batch, self.batch + (rows, inner), self.a)

    def _right(self, backend, gradient):
        """dB = A^T G (inner x cols per batch)."""
        rows, inner, cols = self.a[-2], self.a[-1], self.b[-1]
        count, dtype, left = prod(self.batch), self.right.storage.dtype, self.left.storage
        layout = self._layout() if hasattr(backend, "gemm") else "mixed"
        if layout in ("same", "left-shared"):
            return backend.gemm(left, gradient, inner, rows, cols, batch=count, transpose_left=True,
                                left_stride=0 if layout == "left-shared" else None, out_dtype=dtype)
        if layout == "right-shared":
            # the batch sum is part of the reduction: A as (batch * rows) x inner
            return backend.gemm(left, gradient, inner, count * rows, cols, transpose_left=True, out_dtype=dtype)
        flipped = backend.transpose(left, self.a, axes=_last_two_swapped(len(self.a)))
        per_batch = backend.matmul(flipped, gradient, self.a[:-2] + (inner, rows), self.batch + (rows, cols))
        return backend.unbroadcast(per_batch, self.batch + (inner, cols), self.b)
