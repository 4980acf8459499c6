"""Backend registry for the MI355X build (src/qutai/backends/device.py:5-47).

The reference registers ``{"cpu": cpu, "cuda": cuda, "apple": apple}``; this
package registers its own device module under the new device string
``"amd"``.  Registering it next to the reference's modules is the one-line
change described in INTEGRATION.md.
"""
from __future__ import annotations

from . import amd
from .storage import Storage

_BACKENDS = {"amd": amd}


def get_backend(device="amd", *others):
    """Backend for a device string or storage; several storages must share device and dtype."""
    if isinstance(device, Storage):
        if any((item.device, item.dtype) != (device.device, device.dtype) for item in others):
            raise ValueError("operands must share device and dtype")
        device = device.device
    if device not in _BACKENDS:
        raise ValueError(f"unsupported device: {device}")
    return _BACKENDS[device]


def default_dtype(device: str) -> str:
    """GPU devices default to float32 (src/qutai/backends/device.py:18-22)."""
    get_backend(device)
    return "float32"


def is_available(device: str) -> bool:
    return device in _BACKENDS and _BACKENDS[device].is_available()


def synchronize(device: str = "amd") -> None:
    get_backend(device).synchronize()


def transfer(values, device=None, dtype=None, *, copy=False):
    """Same-device dtype change (src/qutai/backends/device.py:35-47)."""
    device = values.device if device is None else device
    dtype = values.dtype if dtype is None else dtype
    backend = get_backend(device)
    if (device, dtype) == (values.device, values.dtype) and not copy:
        return values
    return backend.from_storage(values, dtype=dtype)
