"""Matmul precision switch (src/qutai/backends/precision.py:1-11).

``set_matmul_precision("bfloat16")`` makes fp32 GEMMs run on the bf16 MFMA
path (autocast); the token it returns restores the previous value, and it
also works as a context manager, as the reference relies on
(src/qutai/core/operations/linalg.py:27, src/qutai/lm/layers.py:51).
"""
from __future__ import annotations

from contextvars import ContextVar

_matmul_precision: ContextVar[str | None] = ContextVar("qutai_amd_matmul_precision", default=None)


class _Token:
    def __init__(self, token):
        self._token = token

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        _matmul_precision.reset(self._token)
        return False


def matmul_precision() -> str | None:
    return _matmul_precision.get()


def set_matmul_precision(dtype: str | None) -> _Token:
    if dtype not in (None, "bfloat16"):
        raise ValueError("matmul precision must be None or 'bfloat16'")
    return _Token(_matmul_precision.set(dtype))
