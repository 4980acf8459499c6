"""safetensors files for device tensors (src/qutai/core/serialization.py:14-112).

``SafeTensors(path, device="amd")`` is a read-only mapping name -> Tensor:
the header is parsed and validated when the file is opened (the same checks
and ``ValueError`` cases as the reference: header length, JSON object,
string metadata, known dtypes F32 / F64 / BF16, integer shapes and offsets,
data length = element count x width, no overlapping spans); a tensor's bytes
are uploaded to HBM on first access straight from a memory map of the file,
with no host-side copy.  BF16 files load as bf16 device storage.

``save_safetensors(path, tensors, metadata=None)`` writes the same format
(8-byte little-endian header length, JSON header padded with spaces to a
multiple of 8, tensor bytes in header order), streaming each device tensor
through one reusable host buffer of ``chunk_bytes``, to a temporary file
that replaces ``path`` when complete.
"""
from __future__ import annotations

import json
import mmap
import struct
from collections.abc import Mapping
from math import prod
from pathlib import Path

from .core.tensor import Tensor

DTYPES = {"F32": ("float32", 4), "F64": ("float64", 8), "BF16": ("bfloat16", 2)}
_HEADER_LIMIT = 16 * 1024 * 1024


def _device_backend(device):
    if device != "amd":
        raise ValueError("this package reads safetensors into the amd device")
    from .backends import amd

    return amd


class SafeTensors(Mapping):
    def __init__(self, path, device="amd"):
        self.path, self.device, self._cache = Path(path), device, {}
        _device_backend(device)
        file_size = self.path.stat().st_size
        with self.path.open("rb") as stream:
            raw = stream.read(8)
            if len(raw) != 8:
                raise ValueError("not a safetensors file: shorter than its header length")
            size = struct.unpack("<Q", raw)[0]
            if size > _HEADER_LIMIT or size > file_size - 8:
                raise ValueError("invalid safetensors header length")
            try:
                header = json.loads(stream.read(size))
            except (UnicodeDecodeError, json.JSONDecodeError) as error:
                raise ValueError(f"safetensors header is not JSON: {error}") from None
        if not isinstance(header, dict):
            raise ValueError("the safetensors header must be a JSON object")
        self.metadata = header.pop("__metadata__", {})
        if not isinstance(self.metadata, dict) or not all(
                isinstance(k, str) and isinstance(v, str) for k, v in self.metadata.items()):
            raise ValueError("safetensors metadata must map strings to strings")
        self._header, self._start = header, size + 8
        data_size = file_size - self._start
        spans = []
        for name, item in header.items():
            if not isinstance(item, dict) or item.get("dtype") not in DTYPES:
                raise ValueError(f"unsupported safetensors tensor: {name}")
            shape, offsets = item.get("shape"), item.get("data_offsets")
            if not isinstance(shape, list) or any(type(n) is not int or n < 0 for n in shape):
                raise ValueError(f"invalid tensor shape: {name}")
            if not isinstance(offsets, list) or len(offsets) != 2 or any(type(n) is not int for n in offsets):
                raise ValueError(f"invalid tensor offsets: {name}")
            start, end = offsets
            if not 0 <= start <= end <= data_size or end - start != prod(shape) * DTYPES[item["dtype"]][1]:
                raise ValueError(f"invalid tensor data length: {name}")
            if start != end:
                spans.append((start, end))
        spans.sort()
        if any(a[1] > b[0] for a, b in zip(spans, spans[1:])):
            raise ValueError("safetensors tensor data overlaps")

    def __iter__(self):
        return iter(self._header)

    def __len__(self):
        return len(self._header)

    def __contains__(self, name):
        return name in self._header

    def dtype_of(self, name):
        return DTYPES[self._header[name]["dtype"]][0]

    def shape_of(self, name):
        return tuple(self._header[name]["shape"])

    def __getitem__(self, name):
        if name not in self._cache:
            amd = _device_backend(self.device)
            item = self._header[name]
            dtype = DTYPES[item["dtype"]][0]
            start, end = item["data_offsets"]
            storage = amd.AMDStorage(prod(item["shape"]), dtype)
            if end > start:
                with self.path.open("rb") as stream, \
                        mmap.mmap(stream.fileno(), 0, access=mmap.ACCESS_COPY) as data, \
                        memoryview(data)[self._start + start:self._start + end] as view:
                    storage.runtime.upload(storage.ptr, view)
            self._cache[name] = Tensor(storage, shape=tuple(item["shape"]))
        return self._cache[name]


def device_chunks(storage, chunk_bytes=4 << 20, *, offset=0, nbytes=None):
    """The bytes of a device storage (or of its byte range offset .. offset +
    nbytes), read back in pieces of at most chunk_bytes through one reused
    host buffer (src/qutai/lm/checkpoint.py:120-146)."""
    nbytes = storage.nbytes - offset if nbytes is None else nbytes
    if offset < 0 or nbytes < 0 or offset + nbytes > storage.nbytes:
        raise ValueError("byte range outside the storage")
    chunk_bytes = max(8, chunk_bytes // 8 * 8)
    buffer = bytearray(min(chunk_bytes, nbytes))
    view = memoryview(buffer)
    done = 0
    while done < nbytes:
        take = min(chunk_bytes, nbytes - done)
        piece = view[:take]
        storage.runtime.download(storage.ptr + offset + done, piece)
        yield piece
        done += take


def save_safetensors(path, tensors, *, metadata=None, chunk_bytes=4 << 20):
    """Write name -> Tensor (amd device) to a safetensors file (serialization.py:80-112)."""
    tensors = dict(tensors)
    header, offset = {}, 0
    names = {dtype: code for code, (dtype, _) in DTYPES.items()}
    for name, tensor in tensors.items():
        if not isinstance(name, str) or name == "__metadata__":
            raise ValueError("invalid tensor name")
        if tensor.dtype not in names:
            raise ValueError(f"unsupported tensor dtype: {tensor.dtype}")
        if tensor.device != "amd":
            raise ValueError("save_safetensors writes amd device tensors")
        size = tensor.storage.nbytes
        header[name] = dict(dtype=names[tensor.dtype], shape=list(tensor.shape), data_offsets=[offset, offset + size])
        offset += size
    if metadata is not None:
        if not isinstance(metadata, dict) or not all(isinstance(k, str) and isinstance(v, str)
                                                     for k, v in metadata.items()):
            raise ValueError("metadata must map strings to strings")
        header["__metadata__"] = metadata
    encoded = json.dumps(header, separators=(",", ":")).encode("utf-8")
    encoded += b" " * (-len(encoded) % 8)
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    temporary = path.with_suffix(path.suffix + ".tmp")
    try:
        with temporary.open("wb") as stream:
            stream.write(struct.pack("<Q", len(encoded)))
            stream.write(encoded)
            for tensor in tensors.values():
                for piece in device_chunks(tensor.storage, chunk_bytes):
                    stream.write(piece)
        temporary.replace(path)
    finally:
        temporary.unlink(missing_ok=True)
    return path
