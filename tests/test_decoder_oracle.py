"""Pins of the float64 decoder restatement (oracle/decoder.py): its chained
backward against central differences of its own loss (the reference's own
check, tests/test_lm_decoder.py:73-99), for the dense and the MoE block and
for chunked heads with ignored labels; the masked-target closed form
(tests/test_lm_decoder.py:113-120) and causality of the logits
(tests/test_lm_decoder.py:101-111)."""
import pytest

from oracle import decoder as od

TOKENS = [[1, 2, 3, 4], [2, 3, 4, 5]]
LABELS = [[1, -100, 3, 4], [2, 3, 4, 5]]


@pytest.mark.parametrize("ffn_type,seed,chunk", [("dense", 1, 2), ("moe", 2, 3), ("moe", 5, 20)])
def test_gradients_match_central_differences(ffn_type, seed, chunk):
    config = od.dense_config(ffn_type=ffn_type, aux_loss_coef=0.5)
    params = od.random_parameters(config, seed)
    loss, grads = od.loss_and_gradients(config, params, TOKENS, LABELS, chunk_size=chunk)
    assert loss == pytest.approx(od.loss(config, params, TOKENS, LABELS, chunk_size=7), abs=1e-12)
    h = 1e-6
    worst = 0.0
    for name, values in params.items():
        for i in range(0, len(values), 3):  # every third entry of every parameter
            original = values[i]
            values[i] = original + h
            upper = od.loss(config, params, TOKENS, LABELS, chunk_size=chunk)
            values[i] = original - h
            lower = od.loss(config, params, TOKENS, LABELS, chunk_size=chunk)
            values[i] = original
            numeric = (upper - lower) / (2 * h)
            worst = max(worst, abs(numeric - grads[name][i]) / (1 + abs(numeric)))
    assert worst < 1e-7


def test_masked_targets_give_zero_loss_and_gradients():
    config = od.dense_config(n_layers=1)
    params = od.random_parameters(config, 3)
    loss, grads = od.loss_and_gradients(config, params, [[1, 2, 3]], [[-100, -100, -100]])
    assert loss == 0
    assert all(v == 0 for values in grads.values() for v in values)


def test_logits_are_causal_and_match_the_head():
    config = od.dense_config()
    params = od.random_parameters(config, 4)
    first = od.logits(config, params, [[1, 2, 3, 4]])
    second = od.logits(config, params, [[1, 2, 9, 8]])
    vocab = config["vocab_size"]
    assert first[:2 * vocab] == pytest.approx(second[:2 * vocab], abs=1e-12)
    assert first[2 * vocab:] != pytest.approx(second[2 * vocab:], abs=1e-6)
    # the loss over one sequence is the mean cross entropy of these logits
    from math import exp, log

    ce = [log(sum(exp(v) for v in first[t * vocab:(t + 1) * vocab])) - first[t * vocab + label]
          for t, label in enumerate([2, 3, 4])]
    assert od.loss(config, params, [[1, 2, 3, 4]]) == pytest.approx(sum(ce) / 3, rel=1e-12)


def test_parameter_count_matches_the_reference_formula():
    """Config.parameter_counts (src/qutai/lm/config.py:58-71) for the tiny dense and MoE models."""
    for ffn_type in ("dense", "moe"):
        config = od.dense_config(ffn_type=ffn_type)
        d, k = config["d_model"], config["n_kv_heads"] * (config["d_model"] // config["n_heads"])
        shared = config["vocab_size"] * d + d
        attention = 2 * d * d + 2 * d * k + 2 * d
        if ffn_type == "dense":
            expected = shared + config["n_layers"] * (attention + 3 * d * config["d_ff"])
        else:
            expected = shared + config["n_layers"] * (attention + d * config["n_experts"]
                                                      + config["n_experts"] * 3 * d * config["d_expert"])
        shapes = od.parameter_shapes(config).values()
        total = 0
        for shape in shapes:
            size = 1
            for s in shape:
                size *= s
            total += size
        assert total == expected
