"""Parity at the full BASELINE sizes of the calls that bench.py times:
bf16 4096^3 through Tensor @ (bf16 result), the config-3 bmm-form attention
products, all three config-4 projections forward and backward, and one
decoder_train-shape loss step with the loss head's gradients.  Full
outputs are checked through properties (bit equality with the host-rounded
fp32 product, finiteness) and sampled rows against the float64 oracle."""
import numpy as np
import pytest

from oracle import reference as ora
from tests.helpers import download, normal, stored, upload

pytestmark = pytest.mark.gpu

BF16_TOL = 1e-2
FP32_TOL = 1e-5


@pytest.fixture(scope="module")
def amd():
    from qutai_amd.backends import amd as backend

    backend.get_runtime()
    return backend


def sampled(n, count=24, seed=0):
    picks = {0, 1, n // 2, n - 1}
    picks.update(np.random.default_rng(seed).choice(n, size=count, replace=False).tolist())
    return sorted(picks)


def test_config2_bf16_result_through_tensor_matmul(amd):
    """The headline call (Tensor @ on bf16 storage returns bf16, the dtype
    rule of src/qutai/backends/cuda.py:374) at 4096^3: every element equals
    the RNE rounding of the same product's fp32 output (one rounding of the
    same fp32 accumulators), and sampled rows are within the bf16 bar of the
    float64 product of the unrounded inputs."""
    from qutai_amd import Tensor

    n = 4096
    rng = np.random.default_rng(1)
    a = (rng.standard_normal(n * n) * n ** -0.5).astype(np.float32)
    b = (rng.standard_normal(n * n) * n ** -0.5).astype(np.float32)
    left, right = upload(a, "bfloat16"), upload(b, "bfloat16")
    product = Tensor(left, shape=(n, n)) @ Tensor(right, shape=(n, n))
    assert product.dtype == "bfloat16" and product.shape == (n, n)
    words = np.frombuffer(product.storage.to_array(), dtype=np.uint16)
    wide = download(amd.gemm(left, right, n, n, n, out_dtype="float32"))
    assert np.array_equal(words, ora.bf16_words(wide)), "bf16 result differs from the rounded fp32 result"
    result = ora.bf16_values(words).astype(np.float64).reshape(n, n)
    rows = sampled(n)
    unrounded = ora.gemm_f64(a.astype(np.float64), b.astype(np.float64), n, n, n, row_list=rows)
    assert ora.rel_frobenius(result[rows], unrounded) <= BF16_TOL
    exact = ora.gemm_f64(stored(a, "bfloat16"), stored(b, "bfloat16"), n, n, n, row_list=rows)
    assert ora.rel_frobenius(result[rows], exact) <= 4e-3  # one bf16 rounding of the result
    assert np.isfinite(result).all()


def test_config3_bmm_form_against_float64_attention(amd):
    """S = Q K^T (bf16), P = softmax(S / 8), O = P V for B8 x H16, T 2048,
    D 64: O of 8 heads (first and last included) against the float64
    attention of the stored inputs, with no device rounding copied into the
    reference; P rows against the float64 probabilities."""
    from qutai_amd import Tensor
    from qutai_amd.lm.layers import attention_products

    groups, time, dim = 128, 2048, 64
    q, k, v = (normal(2 + i, groups * time * dim) for i in range(3))
    tensors = [Tensor(upload(x, "bfloat16"), shape=(groups, time, dim)) for x in (q, k, v)]
    out, probs = attention_products(*tensors)
    o = download(out.storage).reshape(groups, time, dim)
    p = download(probs.storage).reshape(groups, time, time)
    assert np.isfinite(o).all()
    for h in (0, 1, 31, 57, 64, 90, 126, 127):
        qr, kr, vr = (stored(x, "bfloat16").reshape(groups, time, dim)[h] for x in (q, k, v))
        expected, lse = ora.attention_np(qr, kr, vr, causal=False)
        assert ora.rel_frobenius(o[h], expected) <= BF16_TOL, h
        rows = sampled(time, 8, seed=h)
        exact_p = np.exp((qr[rows] @ kr.T) * dim ** -0.5 - lse[rows, None])
        assert ora.rel_frobenius(p[h][rows], exact_p) <= BF16_TOL, h


@pytest.mark.parametrize("projection", ["gate", "up", "down"])
def test_config4_projection_forward_backward(amd, projection):
    """One SwiGLU projection of config 4 through lm.linear under the bf16
    storage of the benchmark: Y = X W^T (NT), dX = dY W (NN), dW = dY^T X
    (TN) at 4096 tokens, sampled rows against float64.  The down projection
    (2048 x 5632, K = 5632 forward, dW over K = 4096 on 192-wide tiles) is
    the one that differs in shape from gate/up."""
    from qutai_amd import Tensor
    from qutai_amd.lm.layers import linear

    tokens, width, hidden = 4096, 2048, 5632
    fan_in, fan_out = (width, hidden) if projection != "down" else (hidden, width)
    seed = {"gate": 3, "up": 4, "down": 5}[projection]
    x = normal(seed, tokens * fan_in)
    w = normal(seed + 30, fan_out * fan_in, 0.02)
    g = normal(seed + 60, tokens * fan_out)
    xt = Tensor(upload(x, "bfloat16"), shape=(8, 512, fan_in), requires_grad=True)
    wt = Tensor(upload(w, "bfloat16"), shape=(fan_out, fan_in), requires_grad=True)
    y = linear(xt, wt)
    assert y.shape == (8, 512, fan_out) and y.dtype == "bfloat16"
    y.backward(Tensor(upload(g, "bfloat16"), shape=y.shape))
    xr = stored(x, "bfloat16").reshape(tokens, fan_in)
    wr = stored(w, "bfloat16").reshape(fan_out, fan_in)
    gr = stored(g, "bfloat16").reshape(tokens, fan_out)
    rows = sampled(tokens, 12, seed=seed)
    got_y = download(y.storage).reshape(tokens, fan_out)
    assert np.isfinite(got_y).all()
    assert ora.rel_frobenius(got_y[rows], ora.gemm_f64(xr[rows], wr, len(rows), fan_in, fan_out,
                                                       transpose_right=True)) <= BF16_TOL
    got_dx = download(xt.grad.storage).reshape(tokens, fan_in)
    assert ora.rel_frobenius(got_dx[rows], ora.gemm_f64(gr[rows], wr, len(rows), fan_out, fan_in)) <= BF16_TOL
    w_rows = sampled(fan_out, 12, seed=seed + 1)
    got_dw = download(wt.grad.storage).reshape(fan_out, fan_in)
    exact_dw = ora.gemm_f64(gr, xr, fan_out, tokens, fan_in, transpose_left=True, row_list=w_rows)
    assert ora.rel_frobenius(got_dw[w_rows], exact_dw) <= BF16_TOL
    assert np.isfinite(got_dx).all() and np.isfinite(got_dw).all()


def _decoder(seed):
    """bench.py's decoder_train model: config-4 shapes, 2 layers, vocab 32768."""
    from qutai_amd.backends import amd_lm
    from qutai_amd.lm import Config, Decoder

    config = Config(vocab_size=32768, n_layers=2, d_model=2048, n_heads=32, n_kv_heads=8, d_ff=5632,
                    max_seq_len=2048, activation_checkpointing=False)
    rng = np.random.default_rng(seed)
    host_normal = amd_lm.normal
    amd_lm.normal = lambda size, mean=0.0, std=1.0, *, seed=None, dtype="float32": upload(
        rng.normal(mean, std, size), dtype)
    try:
        model = Decoder(config, seed=seed)
    finally:
        amd_lm.normal = host_normal
    return model, rng.integers(0, config.vocab_size, size=(2, 2048)).tolist()


def _head_float64(h, w, labels, chunk=512):
    """Per-row cross entropy and log-sum-exp of bf16 hidden rows against the
    bf16 tied weight, in float64."""
    losses, lses = np.empty(len(h)), np.empty(len(h))
    for r0 in range(0, len(h), chunk):
        logits = h[r0:r0 + chunk] @ w.T
        peak = logits.max(axis=1, keepdims=True)
        lse = (peak + np.log(np.exp(logits - peak).sum(axis=1, keepdims=True)))[:, 0]
        lses[r0:r0 + chunk] = lse
        losses[r0:r0 + chunk] = lse - logits[np.arange(len(logits)), labels[r0:r0 + chunk]]
    return losses, lses


def test_decoder_train_shape_loss_and_head_gradients(amd):
    """One Decoder.loss step at bench.py's decoder_train shapes under
    autocast: the device loss equals the float64 cross entropy of the
    device's own final hidden states against the tied weight (all 4094
    prediction rows), every parameter gradient is finite, and the loss
    head's gradients (dX rows and dW vocabulary rows) match float64."""
    from qutai_amd import Tensor
    from qutai_amd.lm import autocast
    from qutai_amd.lm.layers import projection_loss

    model, tokens = _decoder(5)
    with autocast():
        hidden = model.hidden(tokens, train=False)
        loss = model.loss(tokens, chunk_size=1024)
    loss.backward()
    value = model.last_lm_loss.item()
    assert np.isfinite(loss.item()) and np.isfinite(value)
    for name, parameter in model.named_parameters():
        grad = download(parameter.grad.storage)
        assert np.isfinite(grad).all() and np.abs(grad).max() > 0, name

    batch, time, width = hidden.shape
    h = stored(download(hidden.storage), "bfloat16").reshape(batch, time, width)
    w = stored(download(model.embedding.weight.storage), "bfloat16").reshape(-1, width)
    rows = h[:, :-1].reshape(-1, width)  # position t predicts token t + 1
    labels = np.array([row[1:] for row in tokens]).ravel()
    losses, lse = _head_float64(rows, w, labels)
    assert abs(value - losses.mean()) <= 1e-3 * losses.mean()

    # the loss head alone with leaf inputs: dX and dW against float64
    hleaf = Tensor(hidden.storage.copy(), shape=hidden.shape, requires_grad=True)
    wleaf = Tensor(model.embedding.weight.storage.copy(), shape=model.embedding.weight.shape, requires_grad=True)
    with autocast():
        head = projection_loss(hleaf, wleaf, tokens, 1024)
    head.backward()
    assert abs(head.item() - losses.mean()) <= 1e-3 * losses.mean()
    count = len(labels)
    dx = download(hleaf.grad.storage).reshape(batch, time, width)
    assert np.all(dx[:, -1] == 0)  # the last position predicts nothing
    picks = sampled(count, 12)
    for r in picks:
        p = np.exp(rows[r] @ w.T - lse[r])
        p[labels[r]] -= 1
        expected = (p @ w) / count
        got = dx.reshape(-1, width)[(r // (time - 1)) * time + r % (time - 1)]
        assert ora.rel_frobenius(got, expected) <= BF16_TOL, r
    dw = download(wleaf.grad.storage).reshape(-1, width)
    for v in sampled(w.shape[0], 8, seed=3):
        column = np.exp(rows @ w[v] - lse)
        column -= labels == v
        assert ora.rel_frobenius(dw[v], (column @ rows) / count) <= BF16_TOL, v


def test_decoder_train_shape_layer_weight_gradients(amd, monkeypatch):
    """One Decoder.loss step at decoder_train shapes under autocast, with
    every projection of the first block observed: pass-through graph nodes
    keep each projection's bf16 input and the gradient that reaches its
    output.  Sampled rows of the q, k, v, out and down weight gradients
    (fp32 masters) equal the float64 G^T X of those device tensors within
    1e-5; rows of the gate and up weight gradients equal float64
    dGate^T X / dUp^T X, with dGate / dUp formed from the device's bf16 gate
    and up products and activation gradient (the silu_mul backward, rounded to
    bf16 as the device stores them), within the bf16 bar.  The three
    projections run separately here; a second model of the same seed with
    the stacked q/k/v GEMM gives the same loss bit for bit, bit-identical
    q and out weight gradients in the last block, its k and v weight
    gradients within fp32 rounding (split K when computed alone), and every
    earlier gradient within bf16 rounding (src/qutai/lm/layers.py:35-74,
    291-350)."""
    from qutai_amd.core.grad import record
    from qutai_amd.core.tensor import Tensor
    from qutai_amd.backends import amd_lm
    from qutai_amd.lm import autocast
    from qutai_amd.lm import layers

    seen = []
    plain_linear, plain_swiglu = layers.linear, layers.swiglu

    def observed(result, entry):
        def rule(g):
            entry["g"] = g
            return (g,)
        return record(Tensor(result.storage, shape=result.shape), (result,), rule)

    def spy_linear(x, weight):
        entry = dict(kind="linear", weight=weight, x=layers._bf16_input(x))
        seen.append(entry)
        return observed(plain_linear(x, weight), entry)

    def spy_swiglu(x, w_gate, w_up):
        entry = dict(kind="swiglu", weight=w_gate, up_weight=w_up, x=layers._bf16_input(x))
        seen.append(entry)
        return observed(plain_swiglu(x, w_gate, w_up), entry)

    monkeypatch.setattr(layers, "linear", spy_linear)
    monkeypatch.setattr(layers, "swiglu", spy_swiglu)
    monkeypatch.setattr(layers, "_stacked_qkv", lambda *args: False)
    model, tokens = _decoder(5)
    with autocast():
        loss = model.loss(tokens, chunk_size=1024)
    loss.backward()
    block = model.blocks[0]
    named = {id(block.attn.q.weight): "q", id(block.attn.k.weight): "k", id(block.attn.v.weight): "v",
             id(block.attn.out.weight): "out", id(block.ffn.gate.weight): "gate", id(block.ffn.down.weight): "down"}
    checked = set()
    for entry in seen:
        name = named.get(id(entry["weight"]))
        if name is None:
            continue
        w = entry["weight"]
        x = download(entry["x"]).reshape(-1, w.shape[1])
        g = download(entry["g"]).reshape(x.shape[0], -1)
        grad = download(w.grad.storage).reshape(w.shape)
        picks = sampled(w.shape[0], 6, seed=len(checked))
        if entry["kind"] == "linear":
            expected = g[:, picks].T @ x
            assert ora.rel_frobenius(grad[picks], expected) <= FP32_TOL, name
        else:
            hidden, inner = w.shape
            _, gate, up = amd_lm.swiglu_gemm(entry["x"], layers._bf16(w.storage), layers._bf16(entry["up_weight"].storage),
                                             x.shape[0], inner, hidden, save=True)
            gate = download(gate).reshape(-1, hidden)[:, picks]
            up = download(up).reshape(-1, hidden)[:, picks]
            s = 1 / (1 + np.exp(-gate))
            d_gate = stored(g[:, picks] * up * s * (1 + gate * (1 - s)), "bfloat16")
            d_up = stored(g[:, picks] * gate * s, "bfloat16")
            up_grad = download(entry["up_weight"].grad.storage).reshape(w.shape)
            assert ora.rel_frobenius(grad[picks], d_gate.T @ x) <= BF16_TOL, "gate"
            assert ora.rel_frobenius(up_grad[picks], d_up.T @ x) <= BF16_TOL, "up"
            checked.add("up")
        checked.add(name)
    assert checked == {"q", "k", "v", "out", "gate", "up", "down"}

    # the stacked q/k/v GEMM of the default path: the same gradients, bit for bit
    monkeypatch.setattr(layers, "linear", plain_linear)
    monkeypatch.setattr(layers, "swiglu", plain_swiglu)
    monkeypatch.undo()
    stacked, _ = _decoder(5)
    with autocast():
        again = stacked.loss(tokens, chunk_size=1024)
    again.backward()
    assert again.item() == loss.item()
    # the last block's q and out weight gradients are bit-identical (same
    # upstream gradient, the same products); its k and v weight gradients
    # (512 x 2048 outputs over K = 4096) split K when computed alone, so they
    # differ in fp32 summation order only; the stacked input gradient is one
    # GEMM over K = dq + 2 dkv instead of three products and two adds, so
    # every gradient that flows through it differs in bf16 rounding only
    last = f"blocks.{len(model.blocks) - 1}.attn."
    for (name, p), (_, q) in zip(model.named_parameters(), stacked.named_parameters()):
        if name in (last + "q.weight", last + "out.weight"):
            bits = lambda t: np.frombuffer(t.grad.storage.to_array(), dtype=np.uint8)  # noqa: E731
            assert np.array_equal(bits(p), bits(q)), name
        else:
            tol = FP32_TOL if name.startswith(last) else BF16_TOL
            assert ora.rel_frobenius(download(p.grad.storage), download(q.grad.storage)) <= tol, name
