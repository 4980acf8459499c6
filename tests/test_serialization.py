"""Host-side checks of the safetensors reader and the checkpoint validator
(no device memory is touched): the reference's invalid-file cases
(tests/test_public_tensor_io.py:123-136), header compatibility with the
independent ``safetensors`` library's writer, and tampered checkpoint
shards (src/qutai/lm/checkpoint.py:345-383)."""
import hashlib
import json
import struct

import numpy as np
import pytest

import qutai_amd.lm.checkpoint as checkpoint
from qutai_amd.serialization import SafeTensors, save_safetensors


@pytest.mark.parametrize("header,payload", [
    ({"x": {"dtype": "F32", "shape": [2], "data_offsets": [0, 4]}}, b"1234"),
    ({"x": {"dtype": "F32", "shape": [-1], "data_offsets": [0, 4]}}, b"1234"),
    ({"x": {"dtype": "F32", "shape": [1], "data_offsets": [-1, 3]}}, b"1234"),
    ({"x": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]},
      "y": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]}}, b"1234"),
    ({"__metadata__": {"key": 4}}, b""),
    ({"x": {"dtype": "I8", "shape": [4], "data_offsets": [0, 4]}}, b"1234"),
    ([1, 2], b""),
])
def test_invalid_files_raise_value_error(tmp_path, header, payload):
    path = tmp_path / "bad.safetensors"
    encoded = json.dumps(header).encode()
    path.write_bytes(struct.pack("<Q", len(encoded)) + encoded + payload)
    with pytest.raises(ValueError):
        SafeTensors(path)


def test_header_length_and_metadata_checks(tmp_path):
    path = tmp_path / "bad.safetensors"
    path.write_bytes(struct.pack("<Q", 1000000000))
    with pytest.raises(ValueError):
        SafeTensors(path)
    path.write_bytes(b"1234")
    with pytest.raises(ValueError):
        SafeTensors(path)
    with pytest.raises(ValueError):
        save_safetensors(path, {}, metadata={"key": 4})
    with pytest.raises(ValueError):
        SafeTensors(path, device="cpu")


def test_header_of_the_safetensors_library_is_read(tmp_path):
    """Names, dtypes, shapes and metadata of a file written by the
    ``safetensors`` package parse identically (no tensor is loaded)."""
    from safetensors.numpy import save_file

    path = tmp_path / "lib.safetensors"
    tensors = {"a": np.arange(6, dtype=np.float32).reshape(2, 3), "b": np.zeros((0, 4), np.float64),
               "c": np.array(2.5, dtype=np.float32)}
    save_file(tensors, str(path), metadata={"k": "v"})
    loaded = SafeTensors(path)
    assert set(loaded) == {"a", "b", "c"} and len(loaded) == 3
    assert loaded.metadata == {"k": "v"}
    assert (loaded.dtype_of("a"), loaded.shape_of("a")) == ("float32", (2, 3))
    assert (loaded.dtype_of("b"), loaded.shape_of("b")) == ("float64", (0, 4))
    assert loaded.shape_of("c") == ()


def _write_checkpoint(directory, payload=b"\x00" * 16, *, tamper=False, segment=None):
    shard = directory / "data-x-00000.bin"
    shard.write_bytes(payload)
    digest = hashlib.sha256(payload).hexdigest()
    if tamper:
        shard.write_bytes(payload[:-1] + b"\x01")
    record = {"dtype": "float32", "size": 4, "nbytes": 16,
              "segments": [segment or {"file": shard.name, "offset": 0, "nbytes": 16}]}
    metadata = {"format": "qutai-training", "version": 1, "shards": [
        {"file": shard.name, "nbytes": len(payload), "sha256": digest}], "tensors": {"parameter.0": record}}
    manifest = directory / "manifest.json"
    manifest.write_text(json.dumps(metadata))
    return manifest


def test_checkpoint_validation(tmp_path):
    manifest = _write_checkpoint(tmp_path)
    checkpoint.checkpoint_metadata(manifest, verify=True)
    for kwargs in ({"tamper": True}, {"segment": {"file": "data-x-00000.bin", "offset": 8, "nbytes": 16}},
                   {"segment": {"file": "other.bin", "offset": 0, "nbytes": 16}}):
        manifest = _write_checkpoint(tmp_path, **kwargs)
        with pytest.raises(ValueError):
            checkpoint.checkpoint_metadata(manifest, verify=True)
    metadata = json.loads(manifest.read_text())
    metadata["version"] = 2
    manifest.write_text(json.dumps(metadata))
    with pytest.raises(ValueError):
        checkpoint.checkpoint_metadata(tmp_path, verify=True)
