"""nn.Attention / nn.MultiHeadAttention on the MI355X (src/qutai/nn/layers.py:
288-357), after the reference's tests/test_attention.py:10-90: the
hand-computed identity-projection value, probabilities that sum to one, the
3-D input check, the shared-weight Linear golden values, and every input
and parameter gradient against a float64 composition of the oracle's
attention forms (oracle/reference.py attention_np / attention_backward_np)
and the Linear rules, for the fused (bf16, 64 per head), general (fp32, any
head width <= 256) and product (head width > 256) paths, causal and not.
fp32 within 1e-5 relative Frobenius error; bf16 within 1e-2 of a float64
reference that rounds to bf16 wherever the layer stores a tensor (the
reference's own bf16 semantics: every stored result is a bf16 tensor)."""
import math

import numpy as np
import pytest

from oracle import reference as ora
from tests.helpers import download, stored, upload

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def amd():
    from qutai_amd.backends import amd

    amd.get_runtime()
    return amd


def _set(amd, tensor, values):
    amd.copy_into(tensor.storage, amd.storage(list(np.asarray(values, dtype=np.float64).ravel()), dtype=tensor.dtype))


def test_identity_projections_match_hand_computed_attention(amd):
    from qutai_amd import Tensor, nn

    layer = nn.Attention(2, seed=42)
    for projection in (layer.query, layer.key, layer.value):
        _set(amd, projection.weight, [1.0, 0.0, 0.0, 1.0])
        _set(amd, projection.bias, [0.0, 0.0])
    inputs = Tensor([[[1, 0], [0, 1]]], device="amd", dtype="float32")
    probability = math.exp(1 / math.sqrt(2)) / (math.exp(1 / math.sqrt(2)) + 1)
    result = layer(inputs)
    assert result.shape == (1, 2, 2)
    expected = [probability, 1 - probability, 1 - probability, probability]
    assert np.allclose(download(result.storage), expected, rtol=0, atol=1e-6)
    assert np.allclose(download(layer.weights(inputs).storage), download(result.storage), rtol=0, atol=1e-6)


def test_rows_are_probabilities_and_input_must_be_3d(amd):
    from qutai_amd import Tensor, nn

    layer = nn.Attention(2, 4, seed=42)
    weights = layer.weights(Tensor([[[1, 0], [0, 1], [2, 1]]], device="amd", dtype="float32"))
    assert weights.shape == (1, 3, 3)
    w = download(weights.storage).reshape(3, 3)
    assert np.allclose(w.sum(axis=1), 1, atol=1e-6) and (w >= 0).all() and (w <= 1).all()
    with pytest.raises(ValueError):
        layer([[1, 2]])
    mha = nn.MultiHeadAttention(8, heads=2, causal=True, seed=1)
    probs = download(mha.weights(Tensor(np.random.default_rng(0).standard_normal((2, 5, 8)).tolist(), device="amd",
                                        dtype="float32")).storage).reshape(2, 2, 5, 5)
    assert np.allclose(probs.sum(axis=-1), 1, atol=1e-6)
    assert (probs[..., np.triu_indices(5, 1)[0], np.triu_indices(5, 1)[1]] == 0).all()
    with pytest.raises(ValueError):  # a cache serves causal attention only (nn/layers.py:346)
        nn.MultiHeadAttention(8, heads=2, seed=1)(Tensor([[[0.0] * 8]], device="amd", dtype="float32"),
                                                   cache=nn.KVCache())
    with pytest.raises(ValueError):
        nn.MultiHeadAttention(8, heads=3)


def test_sequence_linear_shared_weight_gradients(amd):
    """tests/test_attention.py:80-90."""
    from qutai_amd import Tensor, nn

    layer = nn.Linear(2, 1, seed=42)
    _set(amd, layer.weight, [2.0, 3.0])
    inputs = Tensor([[[1, 2], [3, 4]], [[5, 6], [7, 8]]], requires_grad=True, device="amd", dtype="float32")
    output = layer(inputs)
    assert output.shape == (2, 2, 1)
    assert output.tolist() == [[[8.0], [18.0]], [[28.0], [38.0]]]
    output.sum().backward()
    assert layer.weight.grad.tolist() == [[16.0], [20.0]]
    assert layer.bias.grad.tolist() == [4.0]
    assert inputs.grad.storage.tolist() == [2.0, 3.0] * 4


def _reference(x, params, heads, causal, with_output, rnd=lambda a: a):
    """float64 forward and gradients of loss = sum(y * dy) for the layer.
    ``rnd`` is applied wherever the device stores a tensor (every product,
    bias add, attention output and gradient), so that for bf16 storage the
    reference carries the same roundings as the layer and only the fp32
    accumulation inside each kernel differs."""
    wq, bq, wk, bk, wv, bv = params[:6]
    batch, time, _ = x.shape
    q, k, v = (rnd(rnd(x @ w) + b) for w, b in ((wq, bq), (wk, bk), (wv, bv)))
    features = q.shape[-1]
    dim = features // heads
    split = lambda t: t.reshape(batch, time, heads, dim)
    qs, ks, vs = split(q), split(k), split(v)
    mixed = np.zeros((batch, time, heads, dim))
    lses = {}
    for b in range(batch):
        for h in range(heads):
            mixed[b, :, h], lses[b, h] = ora.attention_np(qs[b, :, h], ks[b, :, h], vs[b, :, h], causal=causal)
    mixed = rnd(mixed.reshape(batch, time, features))
    y = rnd(rnd(mixed @ params[6]) + params[7]) if with_output else mixed

    def grads(dy):
        out = {}
        dmixed = dy
        if with_output:
            out["wo"] = rnd(mixed.reshape(-1, features).T @ dy.reshape(-1, features))
            out["bo"] = rnd(dy.sum(axis=(0, 1)))
            dmixed = rnd(dy @ params[6].T)
        dm = dmixed.reshape(batch, time, heads, dim)
        dq, dk, dv = (np.zeros((batch, time, heads, dim)) for _ in range(3))
        for b in range(batch):
            for h in range(heads):
                dq[b, :, h], dk[b, :, h], dv[b, :, h] = ora.attention_backward_np(
                    dm[b, :, h], qs[b, :, h], ks[b, :, h], vs[b, :, h], mixed.reshape(batch, time, heads, dim)[b, :, h],
                    lses[b, h], causal=causal)
        flat = x.reshape(-1, x.shape[-1])
        dx = None
        for name, d, w in (("q", dq, wq), ("k", dk, wk), ("v", dv, wv)):
            d = rnd(d.reshape(-1, features))
            out["w" + name], out["b" + name] = rnd(flat.T @ d), rnd(d.sum(axis=0))
            part = rnd(d @ w.T)
            dx = part if dx is None else rnd(dx + part)
        out["x"] = dx.reshape(x.shape)
        return out

    return y, grads


@pytest.mark.parametrize("features,heads,causal,dtype", [
    (3, 1, False, "float32"),          # single head, general kernel (nn.Attention(2, 3))
    (128, 2, True, "bfloat16"),        # fused MFMA kernels, causal
    (128, 2, False, "bfloat16"),       # fused MFMA kernels
    (96, 3, True, "float32"),          # general kernel, 32 per head
    (300, 1, False, "float32"),        # head width > 256: score and value products
])
def test_forward_and_all_gradients_match_float64(amd, features, heads, causal, dtype):
    from qutai_amd import Tensor, nn

    in_features = 2 if features == 3 else features
    if heads == 1 and features == 3:
        layer = nn.Attention(in_features, features, seed=7, dtype=dtype)
        with_output = False
    else:
        layer = nn.MultiHeadAttention(features, heads=heads, causal=causal, seed=7, dtype=dtype)
        with_output = True
    rng = np.random.default_rng(features)
    batch, time = 2, 70 if features > 3 else 2
    x = rng.standard_normal((batch, time, in_features)) * 0.5
    # weights 5x the default init so the scores are not all close to zero
    params_dev = [p for lin in ([layer.query, layer.key, layer.value] + ([layer.output] if with_output else []))
                  for p in (lin.weight, lin.bias)]
    host = []
    for i, p in enumerate(params_dev):
        values = download(p.storage).astype(np.float64) * 5 if i % 2 == 0 else rng.standard_normal(p.size) * 0.1
        _set(amd, p, values)
        host.append(stored(values, dtype).reshape(p.shape))
    xs = stored(x, dtype)
    inputs = Tensor(upload(x, dtype), shape=x.shape, requires_grad=True)
    y = layer(inputs)
    rnd = (lambda a: stored(a, "bfloat16")) if dtype == "bfloat16" else (lambda a: a)
    y_ref, grads = _reference(xs, host, heads, causal, with_output, rnd)
    tol = 1e-5 if dtype == "float32" else 1e-2
    errors = {}
    errors["y"] = ora.rel_frobenius(download(y.storage), y_ref.ravel())
    dy = rng.standard_normal(y_ref.shape)
    y.backward(Tensor(upload(dy, dtype), shape=y.shape))
    ref = grads(stored(dy, dtype))
    names = ["wq", "bq", "wk", "bk", "wv", "bv"] + (["wo", "bo"] if with_output else [])
    for name, p in zip(names, params_dev):
        got = download(p.grad.storage)
        if name == "bk":
            # exactly zero: a key bias shifts all of a query's scores alike and
            # softmax ignores it; the device value is rounding noise
            assert np.linalg.norm(got) <= tol * np.linalg.norm(ref["wk"]), name
            continue
        errors[name] = ora.rel_frobenius(got, ref[name].ravel())
    errors["x"] = ora.rel_frobenius(download(inputs.grad.storage), ref["x"].ravel())
    print({k: f"{v:.2e}" for k, v in errors.items()})
    assert max(errors.values()) <= tol, errors
