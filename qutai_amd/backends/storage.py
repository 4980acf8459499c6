"""Storage protocol shared by the backends (src/qutai/backends/storage.py:4-21)."""
from __future__ import annotations


class Storage:
    """Flat numeric buffer; independent of Tensor and of any device."""
    device: str
    dtype: str

    @property
    def size(self) -> int:
        raise NotImplementedError

    @property
    def nbytes(self) -> int:
        raise NotImplementedError

    def copy(self):
        raise NotImplementedError

    def tolist(self):
        raise NotImplementedError
