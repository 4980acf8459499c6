"""safetensors and training checkpoints of device tensors and models:
the reference's round-trip test (tests/test_public_tensor_io.py:102-121)
on the amd device for F32, F64 and BF16; byte-for-byte interchange with the
independent ``safetensors`` library in both directions; Decoder checkpoints
(dense and MoE) restored exactly into a differently initialised model, in
the reference's parameter names, through small shards and chunks; bf16
weight export and import; a tampered shard rejected before any parameter
changes."""
import json

import numpy as np
import pytest

import qutai_amd.lm.checkpoint as ckpt
from oracle import decoder as od
from tests.helpers import download

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def amd():
    from qutai_amd.backends import amd

    amd.get_runtime()
    return amd


def _raw(storage):
    return bytes(storage.to_array())


@pytest.mark.parametrize("dtype", ["float32", "float64", "bfloat16"])
def test_roundtrip_and_lazy_cache(amd, tmp_path, dtype):
    from qutai_amd import Tensor
    from qutai_amd.serialization import SafeTensors, save_safetensors

    path = tmp_path / "model.safetensors"
    source = Tensor([[.25, -3.5], [2., 7.]], requires_grad=True, device="amd", dtype=dtype)
    save_safetensors(path, {"weight": source, "empty": Tensor([], shape=(0, 2), device="amd", dtype=dtype),
                            "scalar": Tensor(2., device="amd", dtype=dtype)}, metadata={"test": "中文"})
    data = path.read_bytes()
    loaded = SafeTensors(path)
    assert list(loaded) == ["weight", "empty", "scalar"]
    assert loaded.metadata == {"test": "中文"}
    assert not loaded["weight"].requires_grad
    assert loaded["weight"] is loaded["weight"]
    assert loaded["weight"].tolist() == source.tolist()
    assert loaded["weight"].dtype == dtype
    assert loaded["empty"].shape == (0, 2)
    assert loaded["scalar"].item() == 2.
    assert path.read_bytes() == data


def test_interchange_with_the_safetensors_library(amd, tmp_path):
    import torch
    from safetensors.torch import load_file, save_file

    from qutai_amd.serialization import SafeTensors, save_safetensors

    g = torch.Generator().manual_seed(0)
    tensors = {"w_bf16": torch.randn(37, 24, generator=g).to(torch.bfloat16),
               "w_f32": torch.randn(5, 7, 3, generator=g), "w_f64": torch.randn(11, generator=g, dtype=torch.float64)}
    path = tmp_path / "lib.safetensors"
    save_file(tensors, str(path), metadata={"format": "pt"})
    ours = SafeTensors(path)
    for name, t in tensors.items():
        assert ours[name].shape == tuple(t.shape)
        assert _raw(ours[name].storage) == t.contiguous().view(torch.uint8).numpy().tobytes(), name
    back = tmp_path / "ours.safetensors"
    save_safetensors(back, {name: ours[name] for name in tensors}, chunk_bytes=24)
    reread = load_file(str(back))
    for name, t in tensors.items():
        assert reread[name].dtype == t.dtype and torch.equal(reread[name], t), name


def _decoder(ffn_type, seed):
    from qutai_amd.lm import Config, Decoder

    values = od.dense_config(ffn_type=ffn_type)
    values["max_seq_len"] = 16
    return Decoder(Config(**values), seed=seed), values


def _state(model):
    return {name: (_raw(p.storage), None if p.grad is None else _raw(p.grad.storage))
            for name, p in model.named_parameters()}


@pytest.mark.parametrize("ffn_type", ["dense", "moe"])
def test_decoder_checkpoint_restores_parameters_and_gradients(amd, tmp_path, ffn_type):
    model, values = _decoder(ffn_type, 7)
    tokens = [[1, 2, 3, 4], [2, 3, 4, 5]]
    model.loss(tokens, chunk_size=3).backward()
    expected = model.loss(tokens, chunk_size=3, train=False).item()
    manifest = ckpt.save_checkpoint(tmp_path / "run", model, global_step=3, tokens=8, state={"note": "x"},
                                    shard_bytes=1000, chunk_bytes=64)
    metadata = json.loads(manifest.read_text())
    # the reference's parameter names and order (src/qutai/lm/decoder.py:39-81)
    assert [p["name"] for p in metadata["parameters"]] == list(od.parameter_shapes(values))
    assert [p["shape"] for p in metadata["parameters"]] == [list(s) for s in od.parameter_shapes(values).values()]
    assert len(metadata["shards"]) > 1
    restored, _ = _decoder(ffn_type, 99)
    assert _state(restored) != _state(model)
    info = ckpt.load_checkpoint(manifest, restored, chunk_bytes=40)
    assert (info["global_step"], info["tokens"], info["extra"]) == (3, 8, {"note": "x"})
    assert _state(restored) == _state(model)
    assert restored.loss(tokens, chunk_size=3, train=False).item() == expected
    # a second save replaces the first generation's shards
    old = {s["file"] for s in metadata["shards"]}
    ckpt.save_checkpoint(tmp_path / "run", model, shard_bytes=1000)
    assert not any((tmp_path / "run" / name).exists() for name in old)


def test_tampered_shard_is_rejected_before_loading(amd, tmp_path):
    model, _ = _decoder("dense", 7)
    manifest = ckpt.save_checkpoint(tmp_path / "run", model, shard_bytes=1 << 20)
    shard = tmp_path / "run" / json.loads(manifest.read_text())["shards"][0]["file"]
    data = bytearray(shard.read_bytes())
    data[100] ^= 1
    shard.write_bytes(bytes(data))
    target, _ = _decoder("dense", 99)
    before = _state(target)
    with pytest.raises(ValueError):
        ckpt.load_checkpoint(manifest, target)
    assert _state(target) == before
    from qutai_amd.lm import Config, Decoder

    other = Decoder(Config(**{**od.dense_config(d_ff=16), "max_seq_len": 16}), seed=1)
    with pytest.raises(ValueError):
        ckpt.load_checkpoint(manifest, other)  # the configuration differs


@pytest.mark.parametrize("ffn_type", ["dense", "moe"])
def test_bf16_weight_export_and_import(amd, tmp_path, ffn_type):
    from qutai_amd.serialization import SafeTensors

    model, values = _decoder(ffn_type, 7)
    path = ckpt.save_weights(model, tmp_path / "w.safetensors", dtype="bfloat16", metadata={"dtype": "bf16"})
    file = SafeTensors(path)
    assert set(file) == set(od.parameter_shapes(values))
    assert {file.dtype_of(n) for n in file} == {"bfloat16"}
    restored, _ = _decoder(ffn_type, 99)
    loaded = ckpt.load_weights(restored, path)
    assert len(loaded) == len(file)
    from tests.helpers import stored

    for (name, p), (_, q) in zip(model.named_parameters(), restored.named_parameters()):
        assert np.array_equal(download(q.storage), stored(download(p.storage), "bfloat16")), name
    with pytest.raises(ValueError):
        ckpt.load_weights(_decoder("moe" if ffn_type == "dense" else "dense", 1)[0], path)
