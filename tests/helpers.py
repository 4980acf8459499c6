"""Shared helpers of the GPU tests: numpy <-> amd storage and input draws."""
from array import array

import numpy as np

from oracle import reference as ora


def upload(x, dtype):
    """numpy -> amd storage of ``dtype`` (bf16 rounded on the device, RNE)."""
    from qutai_amd.backends import amd

    x = np.ascontiguousarray(x)
    if dtype == "float64":
        return amd.storage(array("d", x.astype(np.float64).tobytes()), dtype="float64")
    return amd.storage(array("f", x.astype(np.float32).tobytes()), dtype=dtype)


def download(storage):
    raw = storage.to_array()
    if storage.dtype == "bfloat16":
        return ora.bf16_values(np.frombuffer(raw, dtype=np.uint16))
    if storage.dtype == "int64":
        return np.frombuffer(raw, dtype=np.int64).copy()
    return np.frombuffer(raw, dtype=np.float32 if storage.dtype == "float32" else np.float64).copy()


def stored(x, dtype):
    """The float64 values the device holds for ``x`` stored as ``dtype``."""
    x = np.asarray(x)
    if dtype == "bfloat16":
        return ora.bf16_round_array(x.astype(np.float32)).astype(np.float64)
    if dtype == "float32":
        return x.astype(np.float32).astype(np.float64)
    return x.astype(np.float64)


def normal(seed, shape, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(np.float32)
