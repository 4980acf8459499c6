"""TEST INFRASTRUCTURE ONLY — float64 restatement of the decoder loss step.

Only ``tests/`` may import this module, as the checker of the device
decoder.  It composes the per-op restatements of ``oracle.reference`` in the
order of the reference model and chains their backward rules by hand:

  * ``Decoder._hidden`` / ``Decoder.loss`` (src/qutai/lm/decoder.py:99-175):
    embedding lookup, the blocks, the final RMSNorm, the chunked projection
    loss tied to the embedding weight, ``lm + aux_loss_coef * mean(aux)``;
  * ``Block.__call__`` (src/qutai/lm/layers.py:425-433): pre-norm attention
    and FFN with residual adds; ``GQA.__call__`` (layers.py:340-344): q/k/v
    projections, RoPE on q and k, causal grouped attention, out projection;
    ``SwiGLU`` (layers.py:310-311); ``SparseMoE.__call__`` (layers.py:376-402):
    router logits, routing, per-expert SwiGLU over gathered rows, weighted
    combine, the auxiliary load loss;
  * ``projection_loss`` (src/qutai/lm/layers.py:187-257): cross entropy of
    the head rows ``(b, t)``, t < T-1, against ``labels[b][t+1]``, -100
    ignored, divided by the number of counted targets (at least 1).

Parameters are a dict of flat float64 lists under the reference's names
(``Decoder.named_parameters``, decoder.py:39-81).  ``loss_and_gradients``
returns the loss and a dict of gradients; tests/test_decoder_oracle.py pins
the gradients against central differences of ``loss`` itself, and the
masked-target and causality closed forms of tests/test_lm_decoder.py:101-120.
"""
from __future__ import annotations

from random import Random

from . import reference as ref


def parameter_shapes(config) -> dict:
    """name -> shape in the order of Decoder.named_parameters (decoder.py:39-81)."""
    d, heads, kv = config["d_model"], config["n_heads"], config["n_kv_heads"]
    kv_width = kv * (d // heads)
    shapes = {"embedding.weight": (config["vocab_size"], d)}
    for i in range(config["n_layers"]):
        p = f"blocks.{i}."
        shapes[p + "attn_norm.weight"] = (d,)
        shapes[p + "ffn_norm.weight"] = (d,)
        shapes[p + "attn.q.weight"] = (d, d)
        shapes[p + "attn.k.weight"] = (kv_width, d)
        shapes[p + "attn.v.weight"] = (kv_width, d)
        shapes[p + "attn.out.weight"] = (d, d)
        if config["ffn_type"] == "moe":
            shapes[p + "ffn.router.weight"] = (config["n_experts"], d)
            for e in range(config["n_experts"]):
                h = config["d_expert"]
                shapes[p + f"ffn.experts.{e}.gate.weight"] = (h, d)
                shapes[p + f"ffn.experts.{e}.up.weight"] = (h, d)
                shapes[p + f"ffn.experts.{e}.down.weight"] = (d, h)
        else:
            h = config["d_ff"]
            shapes[p + "ffn.gate.weight"] = (h, d)
            shapes[p + "ffn.up.weight"] = (h, d)
            shapes[p + "ffn.down.weight"] = (d, h)
    shapes["norm.weight"] = (d,)
    return shapes


def random_parameters(config, seed, *, std=0.3) -> dict:
    """Gaussian weights (norm weights around 1) large enough that every term
    of the loss moves under a perturbation."""
    rng = Random(seed)
    params = {}
    for name, shape in parameter_shapes(config).items():
        size = 1
        for s in shape:
            size *= s
        if name.endswith("norm.weight"):
            params[name] = [1 + 0.1 * rng.gauss(0, 1) for _ in range(size)]
        else:
            params[name] = [rng.gauss(0, std) for _ in range(size)]
    return params


def _linear(x, w, rows, inner, cols):
    """Y = X W^T with W stored (out, in) (lm/layers.py:35-48)."""
    return ref.gemm(x, w, rows, inner, cols, transpose_right=True)


def _linear_backward(g, x, w, rows, inner, cols):
    """(dX = G W, dW = G^T X) (lm/layers.py:50-66)."""
    return (ref.gemm(g, w, rows, cols, inner),
            ref.gemm(g, x, cols, rows, inner, transpose_left=True))


def _add(a, b):
    return [x + y for x, y in zip(a, b)]


def _add_to(target, source):
    for i, v in enumerate(source):
        target[i] += v


def _swiglu(x, wg, wu, wd, rows, width, hidden):
    gate = _linear(x, wg, rows, width, hidden)
    up = _linear(x, wu, rows, width, hidden)
    act = ref.silu(gate)
    mixed = [a * u for a, u in zip(act, up)]
    return _linear(mixed, wd, rows, hidden, width), (x, gate, up, act, mixed)


def _swiglu_backward(g, saved, wg, wu, wd, rows, width, hidden):
    x, gate, up, act, mixed = saved
    dmixed, dwd = _linear_backward(g, mixed, wd, rows, hidden, width)
    dgate = ref.silu_backward([d * u for d, u in zip(dmixed, up)], gate)
    dup = [d * a for d, a in zip(dmixed, act)]
    dx1, dwg = _linear_backward(dgate, x, wg, rows, width, hidden)
    dx2, dwu = _linear_backward(dup, x, wu, rows, width, hidden)
    return _add(dx1, dx2), dwg, dwu, dwd


def _targets(tokens, labels):
    return [label for row in labels for label in row[1:]]


def forward(config, params, tokens) -> dict:
    """Decoder._hidden (decoder.py:99-132) in float64: the final normalised
    hidden rows ``[batch*time][d_model]`` with everything backward needs."""
    batch, time = len(tokens), len(tokens[0])
    d, heads, kv = config["d_model"], config["n_heads"], config["n_kv_heads"]
    dim = d // heads
    kv_width = kv * dim
    layers, eps, theta = config["n_layers"], config["norm_eps"], config["rope_theta"]
    rows = batch * time
    ids = [t for row in tokens for t in row]

    x = ref.embedding(params["embedding.weight"], ids, d)
    saved_blocks, aux_values = [], []
    for i in range(layers):
        p = f"blocks.{i}."
        a, inv_a = ref.rms_norm(x, params[p + "attn_norm.weight"], d, eps)
        q_pre = _linear(a, params[p + "attn.q.weight"], rows, d, d)
        k_pre = _linear(a, params[p + "attn.k.weight"], rows, d, kv_width)
        v = _linear(a, params[p + "attn.v.weight"], rows, d, kv_width)
        q = ref.rope(q_pre, batch, time, heads, dim, theta)
        k = ref.rope(k_pre, batch, time, kv, dim, theta)
        o, lse = ref.attention(q, k, v, batch, time, heads, kv, dim)
        x_mid = _add(x, _linear(o, params[p + "attn.out.weight"], rows, d, d))
        f, inv_f = ref.rms_norm(x_mid, params[p + "ffn_norm.weight"], d, eps)
        block = dict(x=x, a=a, inv_a=inv_a, q=q, k=k, v=v, o=o, lse=lse, x_mid=x_mid, f=f, inv_f=inv_f)
        if config["ffn_type"] == "moe":
            experts, top_k, hidden = config["n_experts"], config["top_k"], config["d_expert"]
            scores = _linear(f, params[p + "ffn.router.weight"], rows, d, experts)
            route = ref.routing(scores, rows, experts, top_k)
            outputs, expert_saved = [], {}
            for e in range(experts):
                if not route["counts"][e]:
                    continue
                n = route["counts"][e]
                gathered = ref.route_gather(f, route, e, d)
                out_e, s = _swiglu(gathered, params[p + f"ffn.experts.{e}.gate.weight"],
                                   params[p + f"ffn.experts.{e}.up.weight"],
                                   params[p + f"ffn.experts.{e}.down.weight"], n, d, hidden)
                outputs.append((e, out_e))
                expert_saved[e] = s
            y = ref.combine(outputs, route["weights"], route, d)
            block.update(route=route, outputs=outputs, expert_saved=expert_saved)
            aux_values.append(route["aux"])
        else:
            y, s = _swiglu(f, params[p + "ffn.gate.weight"], params[p + "ffn.up.weight"],
                           params[p + "ffn.down.weight"], rows, d, config["d_ff"])
            block.update(ffn_saved=s)
            aux_values.append(0.0)
        x = _add(x_mid, y)
        saved_blocks.append(block)
    hidden_out, inv_out = ref.rms_norm(x, params["norm.weight"], d, eps)
    return dict(batch=batch, time=time, ids=ids, blocks=saved_blocks, aux=aux_values, x=x, hidden=hidden_out,
                inv=inv_out)


def loss_and_gradients(config, params, tokens, labels=None, *, chunk_size=128, gradients=True):
    """(loss, {name: gradient}) of Decoder.loss (decoder.py:141-175) in float64."""
    labels = tokens if labels is None else labels
    state = forward(config, params, tokens)
    batch, time, ids = state["batch"], state["time"], state["ids"]
    saved_blocks, aux_values, x = state["blocks"], state["aux"], state["x"]
    hidden_out, inv_out = state["hidden"], state["inv"]
    d, heads, kv = config["d_model"], config["n_heads"], config["n_kv_heads"]
    dim = d // heads
    kv_width = kv * dim
    vocab, layers, theta = config["vocab_size"], config["n_layers"], config["rope_theta"]
    rows = batch * time
    w_emb = params["embedding.weight"]

    targets = _targets(tokens, labels)
    count = max(1, sum(label != -100 for label in targets))
    lm = 0.0
    chunks = []
    for start in range(0, len(targets), chunk_size):
        n = min(chunk_size, len(targets) - start)
        inputs = ref.head_rows(hidden_out, start, n, d, time)
        logits = _linear(inputs, w_emb, n, d, vocab)
        lm += ref.head_loss(logits, targets, n, vocab, start=start)
        chunks.append((start, n, inputs, logits))
    lm /= count
    aux = sum(aux_values) / layers
    loss = lm + config["aux_loss_coef"] * aux
    if not gradients:
        return loss, None

    grads = {name: [0.0] * len(values) for name, values in params.items()}
    dhidden = [0.0] * (rows * d)
    for start, n, inputs, logits in chunks:
        dlogits = ref.head_gradient(logits, targets, n, vocab, [1.0], count, start=start)
        dinputs, dw = _linear_backward(dlogits, inputs, w_emb, n, d, vocab)
        ref.head_rows_backward(dhidden, dinputs, start, n, d, time)
        _add_to(grads["embedding.weight"], dw)
    dx, dnorm = ref.rms_norm_backward(dhidden, x, params["norm.weight"], inv_out, d)
    _add_to(grads["norm.weight"], dnorm)
    aux_gradient = config["aux_loss_coef"] / layers
    for i in reversed(range(layers)):
        p, s = f"blocks.{i}.", saved_blocks[i]
        dy = dx
        dx_mid = list(dx)
        if config["ffn_type"] == "moe":
            experts, top_k, hidden = config["n_experts"], config["top_k"], config["d_expert"]
            route, outputs = s["route"], s["outputs"]
            *doutputs, dweights = ref.combine_backward(dy, outputs, route["weights"], route, d)
            df = [0.0] * (rows * d)
            for (e, _), dout in zip(outputs, doutputs):
                names = [p + f"ffn.experts.{e}.{n}.weight" for n in ("gate", "up", "down")]
                dgathered, dwg, dwu, dwd = _swiglu_backward(dout, s["expert_saved"][e], *(params[n] for n in names),
                                                            route["counts"][e], d, hidden)
                for name, value in zip(names, (dwg, dwu, dwd)):
                    _add_to(grads[name], value)
                for j, row in enumerate(route["ids"][e]):
                    for c in range(d):
                        df[row * d + c] += dgathered[j * d + c]
            dscores = _add(ref.routing_backward(dweights, route),
                           ref.routing_backward([aux_gradient], route, True))
            df_router, dwr = _linear_backward(dscores, s["f"], params[p + "ffn.router.weight"], rows, d, experts)
            _add_to(df, df_router)
            _add_to(grads[p + "ffn.router.weight"], dwr)
        else:
            names = [p + f"ffn.{n}.weight" for n in ("gate", "up", "down")]
            df, dwg, dwu, dwd = _swiglu_backward(dy, s["ffn_saved"], *(params[n] for n in names), rows, d,
                                                 config["d_ff"])
            for name, value in zip(names, (dwg, dwu, dwd)):
                _add_to(grads[name], value)
        dxf, dwn = ref.rms_norm_backward(df, s["x_mid"], params[p + "ffn_norm.weight"], s["inv_f"], d)
        _add_to(dx_mid, dxf)
        _add_to(grads[p + "ffn_norm.weight"], dwn)
        do, dwo = _linear_backward(dx_mid, s["o"], params[p + "attn.out.weight"], rows, d, d)
        _add_to(grads[p + "attn.out.weight"], dwo)
        dq, dk, dv = ref.attention_backward(do, s["q"], s["k"], s["v"], s["o"], s["lse"], batch, time, heads, kv, dim)
        dq = ref.rope(dq, batch, time, heads, dim, theta, inverse=True)
        dk = ref.rope(dk, batch, time, kv, dim, theta, inverse=True)
        da = [0.0] * (rows * d)
        for g, name, cols in ((dq, "q", d), (dk, "k", kv_width), (dv, "v", kv_width)):
            part, dw = _linear_backward(g, s["a"], params[p + f"attn.{name}.weight"], rows, d, cols)
            _add_to(da, part)
            _add_to(grads[p + f"attn.{name}.weight"], dw)
        dxa, dwa = ref.rms_norm_backward(da, s["x"], params[p + "attn_norm.weight"], s["inv_a"], d)
        _add_to(grads[p + "attn_norm.weight"], dwa)
        dx = _add(dx_mid, dxa)
    _add_to(grads["embedding.weight"], ref.embedding_backward(dx, ids, vocab, d))
    return loss, grads


def loss(config, params, tokens, labels=None, *, chunk_size=128) -> float:
    return loss_and_gradients(config, params, tokens, labels, chunk_size=chunk_size, gradients=False)[0]


def logits(config, params, tokens):
    """Decoder.__call__ (decoder.py:134-139): final hidden rows times the tied
    embedding weight, [batch*time][vocab]."""
    state = forward(config, params, tokens)
    rows = state["batch"] * state["time"]
    return _linear(state["hidden"], params["embedding.weight"], rows, config["d_model"], config["vocab_size"])


def dense_config(**changes) -> dict:
    """The tiny configuration of tests/test_lm_decoder.py:18-31."""
    values = dict(vocab_size=17, n_layers=2, d_model=8, n_heads=2, n_kv_heads=1, d_ff=12, max_seq_len=8,
                  ffn_type="dense", n_experts=3, top_k=2, d_expert=6, rope_theta=10000.0, norm_eps=1e-6,
                  aux_loss_coef=0.01)
    values.update(changes)
    return values

