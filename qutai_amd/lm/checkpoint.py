"""Training checkpoints of device models in the reference's format
(src/qutai/lm/checkpoint.py: ``qutai-training`` version 1).

A checkpoint is a directory holding ``manifest.json`` and binary shards
``data-<generation>-<index>.bin`` (at most ``shard_bytes`` each, their
sha256 and size in the manifest).  Each tensor record gives its dtype, size,
byte count and the shard segments holding its bytes.  Tensors move between
HBM and the shards in pieces of ``chunk_bytes`` through one host buffer, so
a checkpoint of any size needs only that much host memory
(checkpoint.py:120-146, 386-411).

Parameter names are the reference model's: this package's MoE blocks keep
each projection of all experts in one (experts, out, in) tensor, which is
written as the reference's per-expert tensors ``ffn.experts.{e}.gate.weight``
(row block e, a byte range of the stacked storage) and read back the same
way, so a reference-written MoE checkpoint loads into the stacked layout.

What is saved: parameters (with their gradients), the model configuration,
the step / token counters, a free ``state`` dict and Python's global random
state.  Optimizer state, data-loader position and tokenizer hashes are not
part of this path and are written as ``null``.
"""
from __future__ import annotations

import hashlib
import json
import os
import random
import uuid
from dataclasses import asdict, is_dataclass
from pathlib import Path

from ..core.tensor import Tensor
from ..serialization import device_chunks

WIDTHS = {"float32": 4, "float64": 8, "bfloat16": 2}
FORMAT, VERSION = "qutai-training", 1


def _manifest_path(path):
    path = Path(path)
    return path if path.suffix == ".json" else path / "manifest.json"


def _file_hash(path):
    digest = hashlib.sha256()
    with Path(path).open("rb") as stream:
        for block in iter(lambda: stream.read(1 << 20), b""):
            digest.update(block)
    return digest.hexdigest()


def _config(model):
    config = getattr(model, "config", None)
    return asdict(config) if is_dataclass(config) else config


def _tuples(value):
    return tuple(_tuples(v) for v in value) if isinstance(value, (list, tuple)) else value


class _View:
    """A byte range of a device storage that is saved or loaded as one
    reference tensor (an expert's block of a stacked weight)."""

    def __init__(self, storage, offset, size, shape):
        self.storage, self.offset, self.size, self.shape = storage, offset, size, tuple(shape)
        self.dtype = storage.dtype
        self.nbytes = size * WIDTHS[storage.dtype]


def _reference_views(model):
    """[(reference name, parameter, view of its value, view-or-None of its
    gradient)] in the reference's named_parameters order
    (src/qutai/lm/decoder.py:39-81): a stacked (experts, out, in) weight
    contributes one entry per expert, expert-major over gate, up, down."""
    named = list(model.named_parameters())
    lookup = dict(named)
    result, done = [], set()

    def view(parameter, name, e=None):
        if e is None:
            shape, offset, size = parameter.shape, 0, parameter.size
        else:
            size = parameter.size // parameter.shape[0]
            shape, offset = parameter.shape[1:], e * size * WIDTHS[parameter.dtype]
        grad = parameter.grad
        return (name, parameter, _View(parameter.storage, offset, size, shape),
                _View(grad.storage, offset, size, shape) if grad is not None else None)

    for name, parameter in named:
        if name in done:
            continue
        prefix, stacked, kind = name.rpartition(".experts.")
        if stacked and kind in ("gate.weight", "up.weight", "down.weight") and parameter.ndim == 3:
            group = [(k, lookup[f"{prefix}.experts.{k}.weight"]) for k in ("gate", "up", "down")]
            done.update(f"{prefix}.experts.{k}.weight" for k, _ in group)
            for e in range(parameter.shape[0]):
                result.extend(view(p, f"{prefix}.experts.{e}.{k}.weight", e) for k, p in group)
        else:
            result.append(view(parameter, name))
    if len({name for name, *_ in result}) != len(result):
        raise ValueError("parameter names must be unique")
    return result


class _ShardWriter:
    def __init__(self, directory, shard_bytes, chunk_bytes):
        self.directory, self.shard_bytes, self.chunk_bytes = directory, shard_bytes, chunk_bytes
        self.generation = uuid.uuid4().hex
        self.shards, self.created, self.file, self.size = [], [], None, 0

    def _open(self):
        self.name = f"data-{self.generation}-{len(self.shards):05d}.bin"
        self.temporary = self.directory / (self.name + ".part")
        self.created += [self.temporary, self.directory / self.name]
        self.file = self.temporary.open("xb")
        self.size, self.digest = 0, hashlib.sha256()

    def finish(self):
        if self.file is None:
            return
        self.file.flush()
        os.fsync(self.file.fileno())
        self.file.close()
        self.file = None
        os.replace(self.temporary, self.directory / self.name)
        self.shards.append({"file": self.name, "nbytes": self.size, "sha256": self.digest.hexdigest()})

    def write(self, view):
        segments = []
        for chunk in device_chunks(view.storage, self.chunk_bytes, offset=view.offset, nbytes=view.nbytes):
            remaining = chunk
            while len(remaining):
                if self.file is None:
                    self._open()
                take = min(len(remaining), self.shard_bytes - self.size)
                part = remaining[:take]
                segments.append({"file": self.name, "offset": self.size, "nbytes": take})
                self.file.write(part)
                self.digest.update(part)
                self.size += take
                remaining = remaining[take:]
                if self.size == self.shard_bytes:
                    self.finish()
        return {"dtype": view.dtype, "size": view.size, "nbytes": view.nbytes, "segments": segments}

    def discard(self):
        if self.file is not None:
            self.file.close()
            self.file = None
        for path in self.created:
            path.unlink(missing_ok=True)


def checkpoint_metadata(path, *, verify=False):
    """The manifest; with ``verify`` the shards' sizes and hashes are checked too."""
    manifest = _manifest_path(path)
    metadata = json.loads(manifest.read_text(encoding="utf8"))
    if verify:
        _validate_files(manifest, metadata)
    return metadata


def save_checkpoint(path, model, optimizer=None, *, global_step=0, tokens=0, learning_rate=None, state=None,
                    shard_bytes=256 << 20, chunk_bytes=4 << 20):
    """Write the model's parameters and gradients (checkpoint.py:205-342);
    the manifest replaces the previous one only when every shard is on disk,
    and the previous generation's shards are removed after that."""
    if optimizer is not None:
        raise ValueError("optimizer state is not part of this checkpoint path")
    if shard_bytes < 1 or chunk_bytes < 1 or global_step < 0 or tokens < 0:
        raise ValueError("shard and buffer sizes must be positive, counters non-negative")
    manifest = _manifest_path(path)
    manifest.parent.mkdir(parents=True, exist_ok=True)
    previous = checkpoint_metadata(manifest) if manifest.exists() else None
    writer = _ShardWriter(manifest.parent, shard_bytes, chunk_bytes)
    temporary = manifest.parent / f"manifest-{writer.generation}.tmp"
    published = False
    try:
        parameters, aliases, tensors = [], {}, {}
        for name, parameter, value, grad in _reference_views(model):
            reference = f"parameter.{len(parameters)}"
            tensors[reference] = writer.write(value)
            gradient = None
            if grad is not None:
                gradient = reference + ".gradient"
                tensors[gradient] = writer.write(grad)
            parameters.append({"name": name, "tensor": reference, "shape": list(value.shape),
                               "requires_grad": parameter.requires_grad, "gradient": gradient})
            aliases[name] = reference
        writer.finish()
        metadata = {
            "format": FORMAT, "version": VERSION, "model_type": type(model).__name__,
            "model_config": _config(model), "parameters": parameters, "aliases": aliases, "tensors": tensors,
            "buffers": {}, "optimizer": None, "shards": writer.shards, "tokenizer_sha256": None,
            "training": {"global_step": global_step, "tokens": tokens, "learning_rate": learning_rate, "data": None,
                         "extra": state or {}},
            "rng": {"python": random.getstate(), "named": {}},
        }
        with temporary.open("x", encoding="utf8") as file:
            json.dump(metadata, file, ensure_ascii=False, indent=2, allow_nan=False)
            file.flush()
            os.fsync(file.fileno())
        os.replace(temporary, manifest)
        published = True
        for shard in previous.get("shards", []) if previous else ():
            old = Path(shard["file"])
            if old.name == str(old) and old.name.startswith("data-"):
                try:
                    (manifest.parent / old).unlink(missing_ok=True)
                except OSError:
                    pass
        return manifest
    finally:
        temporary.unlink(missing_ok=True)
        if not published:
            writer.discard()


def _validate_files(manifest, metadata):
    """Shard names, sizes and hashes, tensor records and their segments
    (checkpoint.py:345-383); raises ValueError before anything is loaded."""
    if metadata.get("format") != FORMAT or metadata.get("version") != VERSION:
        raise ValueError("not a supported qutai training checkpoint")
    shards = {}
    for shard in metadata["shards"]:
        relative = Path(shard["file"])
        if relative.name != str(relative) or relative.is_absolute():
            raise ValueError("checkpoint shards must be file names in the manifest's directory")
        path = manifest.parent / relative
        if not path.exists() or path.stat().st_size != shard["nbytes"] or _file_hash(path) != shard["sha256"]:
            raise ValueError(f"checkpoint shard size or hash mismatch: {relative}")
        shards[shard["file"]] = shard["nbytes"]
    for record in metadata["tensors"].values():
        if record["dtype"] not in WIDTHS or record["size"] < 0 or record["nbytes"] != record["size"] * \
                WIDTHS[record["dtype"]]:
            raise ValueError("checkpoint tensor dtype or size is invalid")
        if sum(s["nbytes"] for s in record["segments"]) != record["nbytes"]:
            raise ValueError("checkpoint tensor segments do not add up to its size")
        for s in record["segments"]:
            if s["file"] not in shards or s["offset"] < 0 or s["nbytes"] < 0 or \
                    s["offset"] + s["nbytes"] > shards[s["file"]]:
                raise ValueError("checkpoint tensor segment outside its shard")


def _read_into(directory, record, view, chunk_bytes):
    if view.dtype != record["dtype"] or view.size != record["size"]:
        raise ValueError("target storage dtype or size differs from the checkpoint")
    offset = view.offset
    for segment in record["segments"]:
        with (directory / segment["file"]).open("rb") as file:
            file.seek(segment["offset"])
            remaining = segment["nbytes"]
            while remaining:
                content = bytearray(file.read(min(chunk_bytes, remaining)))
                if not content:
                    raise ValueError("checkpoint data is truncated")
                view.storage.runtime.upload(view.storage.ptr + offset, content)
                offset += len(content)
                remaining -= len(content)


def load_checkpoint(path, model, optimizer=None, *, restore_rng=True, strict=True, chunk_bytes=4 << 20):
    """Restore into the existing model, keeping its Tensor and storage
    objects (checkpoint.py:411-595): every file and record is validated
    before device memory is touched.  Returns the training counters."""
    from ..backends import amd

    if optimizer is not None:
        raise ValueError("optimizer state is not part of this checkpoint path")
    if chunk_bytes < 1:
        raise ValueError("the read buffer must be positive")
    manifest = _manifest_path(path)
    metadata = checkpoint_metadata(manifest)
    _validate_files(manifest, metadata)
    if strict and metadata["model_config"] != json.loads(json.dumps(_config(model))):
        raise ValueError("checkpoint model configuration differs from the model's")
    views = _reference_views(model)
    if {name for name, *_ in views} != set(metadata["aliases"]):
        raise ValueError("checkpoint parameter names differ from the model's")
    if len(set(metadata["aliases"].values())) != len(metadata["aliases"]):
        raise ValueError("the model does not share parameters the way the checkpoint does")
    records = {r["name"]: r for r in metadata["parameters"]}
    tensors = metadata["tensors"]
    for name, parameter, value, _ in views:
        record = records.get(name)
        if record is None or record["tensor"] != metadata["aliases"][name]:
            raise ValueError(f"checkpoint has no parameter record for {name}")
        saved = tensors[record["tensor"]]
        if list(value.shape) != record["shape"] or value.dtype != saved["dtype"] or value.size != saved["size"]:
            raise ValueError(f"checkpoint parameter shape or dtype differs: {name}")
        if record["gradient"] is not None and (tensors[record["gradient"]]["size"],
                                               tensors[record["gradient"]]["dtype"]) != (value.size, value.dtype):
            raise ValueError(f"checkpoint gradient dtype or size differs: {name}")
    if metadata.get("buffers"):
        raise ValueError("checkpoint holds model buffers this model does not have")
    if restore_rng and metadata["rng"]["named"]:
        raise ValueError("checkpoint holds named random generators that were not given")
    gradient_state = {}
    for name, parameter, value, _ in views:
        record = records[name]
        _read_into(manifest.parent, tensors[record["tensor"]], value, chunk_bytes)
        parameter.requires_grad = record["requires_grad"]
        gradient_state.setdefault(parameter, []).append((value, record["gradient"]))
    for parameter, parts in gradient_state.items():
        if all(gradient is None for _, gradient in parts):
            parameter.grad = None
            continue
        # an expert that received no tokens has no gradient in the reference:
        # its block of the stacked gradient stays zero
        parameter.grad = Tensor(amd.full(parameter.size, 0.0, dtype=parameter.dtype), shape=parameter.shape)
        for value, gradient in parts:
            if gradient is not None:
                target = _View(parameter.grad.storage, value.offset, value.size, value.shape)
                _read_into(manifest.parent, tensors[gradient], target, chunk_bytes)
    if restore_rng:
        random.setstate(_tuples(metadata["rng"]["python"]))
    return {**metadata["training"], "tokenizer_sha256": metadata["tokenizer_sha256"],
            "model_config": metadata["model_config"]}


def load_weights(model, source, *, strict=True):
    """Copy a safetensors file (a path or an open ``SafeTensors``) into the
    model's parameters by the reference's names; file tensors of another
    dtype (bf16 weights into fp32 parameters, or the reverse) are converted
    on the device with round-to-nearest-even.  With ``strict`` the file must
    hold exactly the model's parameters."""
    from ..backends import amd
    from ..serialization import SafeTensors

    tensors = source if isinstance(source, SafeTensors) else SafeTensors(source)
    views = _reference_views(model)
    names = {name for name, *_ in views}
    if strict and set(tensors) != names:
        missing, extra = sorted(names - set(tensors)), sorted(set(tensors) - names)
        raise ValueError(f"safetensors names differ from the model's (missing {missing[:3]}, extra {extra[:3]})")
    for name, _, value, _ in views:
        if name not in tensors:
            continue
        if tensors.shape_of(name) != value.shape:
            raise ValueError(f"{name}: file shape {tensors.shape_of(name)} differs from {value.shape}")
    loaded = []
    for name, _, value, _ in views:
        if name not in tensors:
            continue
        stored = tensors[name].storage
        if stored.dtype != value.dtype:
            stored = amd.from_storage(stored, dtype=value.dtype)
        value.storage.runtime.copy(value.storage.ptr + value.offset, stored.ptr, value.nbytes)
        loaded.append(name)
    return loaded


def save_weights(model, path, *, dtype=None, metadata=None):
    """Write the model's parameters under the reference's names (stacked
    expert weights split per expert), in their own dtype or converted to
    ``dtype`` (e.g. "bfloat16" for a half-size export)."""
    from ..backends import amd
    from ..serialization import save_safetensors

    out = {}
    for name, _, value, _ in _reference_views(model):
        item = WIDTHS[value.dtype]
        part = amd.take(value.storage, value.offset // item, value.size)
        if dtype is not None and dtype != part.dtype:
            part = amd.from_storage(part, dtype=dtype)
        out[name] = Tensor(part, shape=value.shape)
    return save_safetensors(path, out, metadata=metadata)
