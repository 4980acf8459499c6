"""A whole Decoder.loss step on the MI355X against the float64 decoder
restatement (oracle/decoder.py), after tests/test_lm_decoder.py:136-165:
same parameters on both sides, loss within 1e-5 and every parameter
gradient within 2e-5 (1 + |g|) of the float64 value (the reference's own
bar for its GPU decoder against its CPU one), dense and MoE blocks, with and
without activation recomputation, chunked heads with ignored labels, and no
device-to-host read inside the step.  The bf16 case (autocast, head width
64: the fused attention kernels) is held to the bf16 bar on the loss and to
3e-2 relative Frobenius error on each gradient."""
from unittest.mock import patch

import numpy as np
import pytest

from oracle import decoder as od
from oracle import reference as ora
from tests.helpers import download, stored

pytestmark = pytest.mark.gpu

TOKENS = [[1, 2, 3, 4], [2, 3, 4, 5]]
LABELS = [[1, -100, 3, 4], [2, 3, 4, 5]]


@pytest.fixture(scope="module")
def amd():
    from qutai_amd.backends import amd

    amd.get_runtime()
    return amd


def _model(amd, config_values, seed):
    from qutai_amd.lm import Config, Decoder

    config = Config(**{k: v for k, v in config_values.items()})
    model = Decoder(config, seed=3)
    params = {k: stored(np.array(v), "float32").tolist() for k, v in od.random_parameters(config_values, seed).items()}
    named = dict(model.named_parameters())
    for name, tensor in named.items():
        if ".ffn.experts." in name:  # stacked (experts, out, in) block of the per-expert weights
            prefix, _, kind = name.rpartition(".experts.")
            values = [v for e in range(config.n_experts) for v in params[f"{prefix}.experts.{e}.{kind}"]]
        else:
            values = params[name]
        amd.copy_into(tensor.storage, amd.storage(values, dtype="float32"))
    return model, params


def _device_gradients(model, config):
    grads = {}
    for name, tensor in model.named_parameters():
        g = download(tensor.grad.storage)
        if ".ffn.experts." in name:
            prefix, _, kind = name.rpartition(".experts.")
            for e, block in enumerate(g.reshape(config["n_experts"], -1)):
                grads[f"{prefix}.experts.{e}.{kind}"] = block
        else:
            grads[name] = g
    return grads


def _config(**changes):
    values = od.dense_config(**changes)
    values.pop("max_seq_len")
    values["max_seq_len"] = 64
    return values


@pytest.mark.parametrize("ffn_type", ["dense", "moe"])
@pytest.mark.parametrize("recompute", [False, True])
def test_fp32_loss_step_matches_float64(amd, ffn_type, recompute):
    from qutai_amd.backends.amd import AMDStorage

    config = _config(ffn_type=ffn_type, aux_loss_coef=0.5, activation_checkpointing=recompute)
    model, params = _model(amd, config, 11)
    expected, ref_grads = od.loss_and_gradients(config, params, TOKENS, LABELS, chunk_size=3)
    with patch.object(AMDStorage, "to_array", side_effect=AssertionError("the step read device memory")):
        loss = model.loss(TOKENS, LABELS, chunk_size=3)
        loss.backward()
    assert loss.item() == pytest.approx(expected, abs=1e-5)
    got = _device_gradients(model, config)
    assert set(got) == set(ref_grads)
    for name, reference in ref_grads.items():
        reference = np.array(reference)
        assert np.all(np.abs(got[name] - reference) <= 2e-5 * (1 + np.abs(reference))), name
    # the logits of the tied head, and the cached lm loss
    logits = download(model(TOKENS, train=False).storage)
    assert np.allclose(logits, od.logits(config, params, TOKENS), rtol=0, atol=2e-5)


def test_two_steps_with_an_update_between(amd):
    """Gradients of a second step after a plain SGD update made on both sides."""
    config = _config(ffn_type="moe", top_k=1)
    model, params = _model(amd, config, 12)
    for step in range(2):
        for p in model.parameters():
            p.zero_grad()
        expected, ref_grads = od.loss_and_gradients(config, params, TOKENS, chunk_size=5)
        loss = model.loss(TOKENS, chunk_size=5)
        loss.backward()
        assert loss.item() == pytest.approx(expected, abs=1e-5), step
        got = _device_gradients(model, config)
        for name, reference in ref_grads.items():
            assert np.all(np.abs(got[name] - reference) <= 2e-5 * (1 + np.abs(reference))), (step, name)
        # w -= 0.5 g, in float32 on the host for both sides
        for name, tensor in model.named_parameters():
            new = download(tensor.storage) - np.float32(0.5) * download(tensor.grad.storage)
            amd.copy_into(tensor.storage, amd.storage(new.astype(np.float32).tolist(), dtype="float32"))
        params = {}
        for name, tensor in model.named_parameters():
            values = download(tensor.storage).astype(np.float64)
            if ".ffn.experts." in name:
                prefix, _, kind = name.rpartition(".experts.")
                for e, block in enumerate(values.reshape(config["n_experts"], -1)):
                    params[f"{prefix}.experts.{e}.{kind}"] = block.tolist()
            else:
                params[name] = values.tolist()


def test_masked_targets_give_zero_loss_and_gradients(amd):
    from qutai_amd.lm import Config, Decoder

    model = Decoder(Config(**{**_config(n_layers=1)}), seed=2)
    loss = model.loss([[1, 2, 3]], labels=[[-100, -100, -100]])
    assert loss.item() == 0
    loss.backward()
    for p in model.parameters():
        assert not download(p.grad.storage).any()


def test_rejections(amd):
    from qutai_amd.lm import Config, Decoder

    model = Decoder(Config(**_config(n_layers=1)), seed=2)
    for call in (lambda: model.loss([[1]]), lambda: model.loss([[1, 2]], chunk_size=0),
                 lambda: model.loss([[1, 17]]), lambda: model.loss([[1, 2]], labels=[[1, 99]]),
                 lambda: model.loss([[1, 2]], labels=[[1, 2, 3]])):
        with pytest.raises(ValueError):
            call()
    with pytest.raises(ValueError):
        Decoder(Config(**_config()), dtype="float64")


@pytest.mark.parametrize("ffn_type", ["dense", "moe"])
def test_bf16_autocast_step_on_the_fused_attention(amd, ffn_type):
    """Head width 64 with bf16 activations: the fused attention forward and
    backward, bf16 GEMMs with fp32 accumulation, fp32 residual stream."""
    from qutai_amd.lm.precision import autocast

    config = _config(vocab_size=96, n_layers=2, d_model=128, n_heads=2, n_kv_heads=1, d_ff=192, n_experts=4,
                     top_k=2, d_expert=64, ffn_type=ffn_type, aux_loss_coef=0.1, activation_checkpointing=True)
    rng = np.random.default_rng(5)
    tokens = rng.integers(0, 96, size=(2, 24)).tolist()
    model, params = _model(amd, config, 13)
    params = {k: (np.array(v) * (0.1 / 0.3) if not k.endswith("norm.weight") else np.array(v)).tolist()
              for k, v in params.items()}
    for name, tensor in model.named_parameters():  # rescale the device copies the same way
        if not name.endswith("norm.weight"):
            values = download(tensor.storage).astype(np.float64) * (0.1 / 0.3)
            amd.copy_into(tensor.storage, amd.storage(values.astype(np.float32).tolist(), dtype="float32"))
    params = {k: stored(np.array(v), "float32").tolist() for k, v in params.items()}
    expected, ref_grads = od.loss_and_gradients(config, params, tokens, chunk_size=16)
    with autocast():
        loss = model.loss(tokens, chunk_size=16)
    loss.backward()
    assert abs(loss.item() - expected) <= 1e-2 * abs(expected)
    got = _device_gradients(model, config)
    worst = max(ora.rel_frobenius(got[name], np.array(reference)) for name, reference in ref_grads.items()
                if np.any(reference))
    assert worst <= 3e-2
