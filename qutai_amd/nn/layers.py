"""nn layers on the amd device (src/qutai/nn/layers.py:133-150, 288-357).

``Linear``: weight stored (in, out), ``Y = X @ W + b`` through the Tensor
matmul (whose gradient rule gives dX = G W^T (NT) and dW = X^T G (TN) on the
GEMM) and the trailing-axis bias add; initialisation U(+-in^-1/2) from
Random(seed).

``Attention`` / ``MultiHeadAttention``: query/key/value Linear projections
(seeds seed, seed+1, seed+2; the output projection seed+3), softmax(Q K^T /
sqrt(D)) V per head, optional causal mask.  The forward runs the fused
attention kernels on the projections as they are ((batch, length, heads *
dim) is the lm layout), so the length x length scores are never stored;
``weights`` materialises them (batched NT GEMM, mask, row softmax) like the
reference.  ``MultiHeadAttention(..., cache=KVCache())`` runs causal
inference over new positions only: their projections, the cached keys and
values appended, the score product against every cached key with the
causal mask shifted by the cached length, softmax and the value product, all
with graph recording off (src/qutai/nn/layers.py:334-355).
"""
from __future__ import annotations

from math import sqrt
from random import Random

from ..backends import amd, amd_lm
from ..core import operations
from ..core.context import set_recording
from ..core.grad import record
from ..core.tensor import Tensor, _result, matmul
from .cache import KVCache  # noqa: F401 - the reference exposes it beside the layers


def _tensor(data, like):
    return data if isinstance(data, Tensor) else Tensor(data, device=like.device, dtype=like.dtype)


def softmax(x, axis=-1, *, scale=1.0):
    """softmax(scale * x) along ``axis``, recorded (qutai.softmax,
    src/qutai/core/operations/normalization.py:9-25); along the last axis
    the scale is folded into the kernel and the backward is one fused pass."""
    if axis % x.ndim != x.ndim - 1:
        return _result(operations.softmax(x if scale == 1.0 else x * scale, axis), (x,))
    if x.shape[-1] == 0:
        raise ValueError("softmax needs a non-empty axis")
    values = amd.softmax(x.storage, x.shape, -1, scale=scale)
    return record(Tensor(values, shape=x.shape), (x,),
                  lambda g: (amd.softmax_backward(values, g, x.shape, scale=scale),))


def causal_mask(scores, offset=0):
    """Scores (..., length, total) with keys after each query set to -inf
    (the mask of src/qutai/nn/layers.py:337-341); the gradient passes through."""
    length, total = scores.shape[-2], scores.shape[-1]
    values = amd.causal_mask(scores.storage, scores.size // total, total, length, offset)
    return record(Tensor(values, shape=scores.shape), (scores,), lambda g: (g,))


class Linear:
    def __init__(self, in_features, out_features, *, bias=True, seed=None, device="amd", dtype="float32"):
        if in_features <= 0 or out_features <= 0:
            raise ValueError("feature counts must be positive")
        random = Random(seed)
        bound = in_features ** -0.5
        self.weight = Tensor([[random.uniform(-bound, bound) for _ in range(out_features)]
                              for _ in range(in_features)], requires_grad=True, device=device, dtype=dtype)
        self.bias = Tensor([0.0] * out_features, requires_grad=True, device=device, dtype=dtype) if bias else None

    def __call__(self, data):
        tensor = _tensor(data, self.weight)
        result = matmul(tensor, self.weight)
        return result if self.bias is None else result + self.bias

    def parameters(self):
        return (self.weight,) if self.bias is None else (self.weight, self.bias)


def _attend(q, k, v, heads, causal):
    """softmax(Q K^T / sqrt(D)) V for (batch, length, heads * D) projections,
    recorded: the fused attention kernels of amd_lm (D <= 256)."""
    batch, length, features = q.shape
    dims = (batch, length, heads, heads, features // heads)
    out, lse = amd_lm.attention(q.storage, k.storage, v.storage, *dims, causal=causal, layout=1)
    return record(Tensor(out, shape=q.shape), (q, k, v),
                  lambda g: amd_lm.attention_backward(g, q.storage, k.storage, v.storage, out, lse, *dims,
                                                      causal=causal, layout=1))


class Attention:
    """Single-head self-attention over (batch, length, features) inputs
    (src/qutai/nn/layers.py:288-310)."""

    heads, causal = 1, False

    def __init__(self, in_features, out_features=None, *, seed=None, device="amd", dtype="float32"):
        out_features = in_features if out_features is None else out_features
        seeds = (None, None, None) if seed is None else (seed, seed + 1, seed + 2)
        self.query = Linear(in_features, out_features, seed=seeds[0], device=device, dtype=dtype)
        self.key = Linear(in_features, out_features, seed=seeds[1], device=device, dtype=dtype)
        self.value = Linear(in_features, out_features, seed=seeds[2], device=device, dtype=dtype)

    def _input(self, data):
        tensor = _tensor(data, self.query.weight)
        if tensor.ndim != 3:
            raise ValueError("attention input must be (batch, length, features)")
        return tensor

    def _split(self, tensor):
        """(batch, length, features) -> (batch, heads, length, features / heads)."""
        batch, length, features = tensor.shape
        return tensor.reshape((batch, length, self.heads, features // self.heads)).transpose((0, 2, 1, 3))

    def _probabilities(self, queries, keys):
        """softmax(Q K^T / sqrt(D)) of projected (batch, length, features)
        queries and keys: (batch, [heads,] queries, keys)."""
        if self.heads > 1:
            queries, keys = self._split(queries), self._split(keys)
        scores = matmul(queries, keys.transpose((*range(keys.ndim - 2), keys.ndim - 1, keys.ndim - 2)))
        if self.causal:
            scores = causal_mask(scores)
        return softmax(scores, -1, scale=1 / sqrt(queries.shape[-1]))

    def weights(self, data):
        """Attention probabilities (batch, [heads,] queries, keys); rows sum to 1."""
        tensor = self._input(data)
        return self._probabilities(self.query(tensor), self.key(tensor))

    def _mix(self, q, k, v):
        """Per-head softmax(Q K^T / sqrt(D)) V, merged back to (batch, length,
        features): the fused kernels for bf16/fp32 up to 256 per head,
        otherwise (fp64, larger heads) the score and value products."""
        if q.shape[-1] // self.heads <= 256 and q.dtype in ("bfloat16", "float32"):
            return _attend(q, k, v, self.heads, self.causal)
        weights = self._probabilities(q, k)
        if self.heads == 1:
            return matmul(weights, v)
        batch, length, features = v.shape
        return matmul(weights, self._split(v)).transpose((0, 2, 1, 3)).reshape((batch, length, features))

    def __call__(self, data):
        tensor = self._input(data)
        return self._mix(*(layer(tensor) for layer in (self.query, self.key, self.value)))

    def parameters(self):
        return tuple(dict.fromkeys(p for layer in (self.query, self.key, self.value) for p in layer.parameters()))


class MultiHeadAttention(Attention):
    """Heads over a split of the features, then an output projection
    (src/qutai/nn/layers.py:313-357)."""

    def __init__(self, features, heads=1, *, causal=False, seed=None, device="amd", dtype="float32"):
        if heads <= 0 or features % heads:
            raise ValueError("heads must be positive and divide the feature count")
        super().__init__(features, seed=seed, device=device, dtype=dtype)
        self.heads, self.causal = heads, causal
        self.output = Linear(features, features, seed=None if seed is None else seed + 3, device=device, dtype=dtype)

    def __call__(self, data, *, cache=None):
        """Training/full forward through the fused kernels; with ``cache``
        (causal only) inference over the new positions, recording off."""
        if cache is not None and not self.causal:
            raise ValueError("a KV cache serves causal attention inference only")
        if cache is None:
            tensor = self._input(data)
            return self.output(self._mix(*(layer(tensor) for layer in (self.query, self.key, self.value))))
        with set_recording(False):
            tensor = self._input(data)
            queries, keys, values = (self._split(layer(tensor)) for layer in (self.query, self.key, self.value))
            keys, values = cache.update(keys, values)
            length, total = queries.shape[2], keys.shape[2]
            scores = matmul(queries, keys.transpose((0, 1, 3, 2)))
            probabilities = softmax(causal_mask(scores, offset=total - length), -1,
                                    scale=1 / sqrt(queries.shape[-1]))
            mixed = matmul(probabilities, values)
            batch, _, features = tensor.shape
            return self.output(mixed.transpose((0, 2, 1, 3)).reshape((batch, length, features)))

    def parameters(self):
        return tuple(dict.fromkeys((*super().parameters(), *self.output.parameters())))
