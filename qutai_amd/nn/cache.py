"""Keys and values of earlier positions for causal attention inference
(src/qutai/nn/cache.py:5-29).

The cache holds (batch, heads, length, head_dim) tensors with no graph:
``update`` appends the new positions along the length axis (one strided
copy per piece through ``backend.concatenate``) and returns everything
cached so far.
"""
from __future__ import annotations

from ..backends.device import get_backend
from ..core.tensor import Tensor


def _joined(previous, current):
    if previous is None:
        return Tensor(current.storage.copy(), shape=current.shape)
    batch, heads, length, features = current.shape
    values = get_backend(previous.storage, current.storage).concatenate(
        (previous.storage, current.storage), (previous.shape, current.shape), axis=2)
    return Tensor(values, shape=(batch, heads, previous.shape[2] + length, features))


class KVCache:
    def __init__(self):
        self.keys = None
        self.values = None

    @property
    def length(self) -> int:
        return 0 if self.keys is None else self.keys.shape[2]

    def update(self, keys, values):
        """Append keys and values of shape (batch, heads, new, head_dim);
        returns the cached keys and values of every position."""
        if keys.ndim != 4 or keys.shape != values.shape:
            raise ValueError("cached keys and values need one 4-D shape")
        if self.keys is not None and (self.keys.shape[:2] + self.keys.shape[3:]
                                      != keys.shape[:2] + keys.shape[3:]):
            raise ValueError("new keys and values must match the cache in batch, heads and head size")
        self.keys, self.values = _joined(self.keys, keys), _joined(self.values, values)
        return self.keys, self.values
