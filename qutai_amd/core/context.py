"""Graph-recording switch (src/qutai/core/context.py:4-25)."""
from __future__ import annotations

from contextlib import contextmanager
from contextvars import ContextVar

_recording: ContextVar[bool] = ContextVar("qutai_amd_recording", default=True)


def is_recording() -> bool:
    return _recording.get()


@contextmanager
def set_recording(enabled: bool):
    token = _recording.set(bool(enabled))
    try:
        yield
    finally:
        _recording.reset(token)
