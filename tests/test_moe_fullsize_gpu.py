"""The MoE training step at config-5 size (8192 tokens, d_model 2048, 8
experts, SwiGLU hidden 1408, top-2) against float64, on
sampled rows: the expert SwiGLU forward (gate, up, activation, down rows and
the combined output), the token gradient, the routing-weight gradient, the
router-logit gradient, and rows of every expert's dW_gate / dW_up / dW_down.

Each stage's reference is computed in float64 from the device's own stored
inputs of that stage (the gathered rows, the saved gate/up/activation/down
blocks, the bf16 parameters and upstream gradient), rounding to bf16 exactly
where the device stores a bf16 tensor (lm/layers.py:291-314, 376-402: every
stored result is a bf16 tensor), so a wrong index, operand or transpose in
any one stage shows as an error of order one while the remaining difference
is the fp32 accumulation order inside each product.  Bars: bf16 storage
within 1e-2 relative Frobenius error over the sampled rows (the north star's
bf16 bar), fp32 results within 1e-5; routing indices bit-exact against the
oracle (cpu_lm.routing, src/qutai/backends/cpu_lm.py:204-242)."""
import numpy as np
import pytest

from oracle import reference as ora
from tests.helpers import download, normal, stored, upload

pytestmark = pytest.mark.gpu

TOKENS, WIDTH, HIDDEN, EXPERTS, TOP_K = 8192, 2048, 1408, 8, 2


def rnd(a):
    return stored(a, "bfloat16")


def _silu(v):
    return v / (1 + np.exp(-v))


def _i64(storage):
    return np.frombuffer(storage.to_array(), dtype=np.int64).copy()


@pytest.fixture(scope="module")
def step():
    from qutai_amd.backends import amd, amd_lm

    amd.get_runtime()
    x = normal(4, TOKENS * WIDTH)
    logits = normal(40, TOKENS * EXPERTS)
    wg = normal(41, EXPERTS * HIDDEN * WIDTH, 0.02)
    wu = normal(42, EXPERTS * HIDDEN * WIDTH, 0.02)
    wd = normal(43, EXPERTS * WIDTH * HIDDEN, 0.02)
    g = normal(44, TOKENS * WIDTH)
    xs, gs = upload(x, "bfloat16"), upload(g, "bfloat16")
    route = amd_lm.routing(upload(logits, "float32"), TOKENS, EXPERTS, TOP_K)
    dev_w = [upload(w, "bfloat16") for w in (wg, wu, wd)]
    y, saved = amd_lm.moe_experts_forward(xs, route, *dev_w, WIDTH, HIDDEN, save=True)
    dx, d_weights, dwg, dwu, dwd = amd_lm.moe_experts_backward(gs, route, saved, WIDTH, HIDDEN,
                                                               x_dtype="bfloat16", weight_dtype="bfloat16")
    d_logits = amd_lm.routing_backward(d_weights, route)
    host = dict(
        x=stored(x, "bfloat16").reshape(TOKENS, WIDTH), g=stored(g, "bfloat16").reshape(TOKENS, WIDTH),
        logits=logits, wg=stored(wg, "bfloat16").reshape(EXPERTS, HIDDEN, WIDTH),
        wu=stored(wu, "bfloat16").reshape(EXPERTS, HIDDEN, WIDTH),
        wd=stored(wd, "bfloat16").reshape(EXPERTS, WIDTH, HIDDEN),
        order=_i64(route["order"]), offsets=_i64(route["offsets"]), locations=_i64(route["locations"]),
        indices=_i64(route["indices"]), weights=download(route["weights"]).astype(np.float64),
        saved_rows=download(saved["rows"]).reshape(-1, WIDTH), gathered=saved["gathered"],
        gate=download(saved["gate"]).reshape(-1, HIDDEN),
        up=download(saved["up"]).reshape(-1, HIDDEN), act=download(saved["act"]).reshape(-1, HIDDEN),
        down=download(saved["down"]).reshape(-1, WIDTH), y=download(y).reshape(TOKENS, WIDTH),
        dx=download(dx).reshape(TOKENS, WIDTH), d_weights=download(d_weights).astype(np.float64),
        dwg=download(dwg).reshape(EXPERTS, HIDDEN, WIDTH), dwu=download(dwu).reshape(EXPERTS, HIDDEN, WIDTH),
        dwd=download(dwd).reshape(EXPERTS, WIDTH, HIDDEN), d_logits=download(d_logits).astype(np.float64))
    # the expert-major routed rows every product reads (through the order
    # inside the GEMMs, or from the saved copy)
    host["rows"] = host["x"][host["order"]] if host["gathered"] else host["saved_rows"]
    host["expert_of"] = np.searchsorted(host["offsets"], np.arange(TOKENS * TOP_K), side="right") - 1
    # row of (token, slot) in the expert-major block: the expert's offset
    # plus the slot's location within the expert's rows
    host["position"] = host["offsets"][host["indices"]] + host["locations"]
    assert np.array_equal(host["order"][host["position"]], np.repeat(np.arange(TOKENS), TOP_K))
    return host


def _sample_tokens(count=24):
    return np.random.default_rng(7).choice(TOKENS, count, replace=False)


def test_routing_matches_the_oracle_and_rows_are_gathered(step):
    """Routing indices, weights and the expert-major order against
    cpu_lm.routing; the token matrix (32 MiB) is read through that order by
    the forward's gate/up GEMM and the backward's dW_gate / dW_up, so the
    saved rows are the token matrix itself, not a routed copy."""
    ref = ora.routing(step["logits"].astype(np.float64).tolist(), TOKENS, EXPERTS, TOP_K)
    assert step["indices"].tolist() == list(ref["indices"])
    assert np.max(np.abs(step["weights"] - np.array(ref["weights"]))) <= 1e-6
    order = np.concatenate([np.array(ids, dtype=np.int64) for ids in ref["ids"]])
    assert step["order"].tolist() == order.tolist()
    assert step["gathered"]
    assert np.array_equal(step["saved_rows"], step["x"])


def test_expert_forward_rows(step):
    """gate = x W_gate^T, up = x W_up^T (bf16), act = bf16(silu(gate)) * up
    (one rounding), down = act W_down^T, y = sum over slots of w * down."""
    positions = np.random.default_rng(8).choice(TOKENS * TOP_K, 48, replace=False)
    e = step["expert_of"][positions]
    rows = step["rows"][positions]
    gate = rnd(np.einsum("pw,phw->ph", rows, step["wg"][e]))
    up = rnd(np.einsum("pw,phw->ph", rows, step["wu"][e]))
    assert ora.rel_frobenius(step["gate"][positions], gate) <= 1e-2
    assert ora.rel_frobenius(step["up"][positions], up) <= 1e-2
    g_dev, u_dev = step["gate"][positions], step["up"][positions]
    act = rnd(rnd(_silu(g_dev)) * u_dev)
    assert ora.rel_frobenius(step["act"][positions], act) <= 1e-2
    down = rnd(np.einsum("ph,pwh->pw", step["act"][positions], step["wd"][e]))
    assert ora.rel_frobenius(step["down"][positions], down) <= 1e-2
    tokens = _sample_tokens()
    y = np.zeros((tokens.size, WIDTH))
    for i, t in enumerate(tokens):
        for s in range(TOP_K):
            y[i] += step["weights"][t * TOP_K + s] * step["down"][step["position"][t * TOP_K + s]]
    assert ora.rel_frobenius(step["y"][tokens], rnd(y)) <= 1e-2


def _d_down(step, positions):
    """combine backward's expert-row gradient: bf16(w * G[token])."""
    tokens = step["order"][positions]
    slot_weight = np.empty(positions.size)
    for i, (p, t) in enumerate(zip(positions, tokens)):
        slot = np.flatnonzero(step["position"][t * TOP_K:(t + 1) * TOP_K] == p)[0]
        slot_weight[i] = step["weights"][t * TOP_K + slot]
    return rnd(slot_weight[:, None] * step["g"][tokens])


def _d_gate_up(d_act, gate, up):
    """silu_mul backward on the stored gate/up values, each output bf16."""
    s = 1 / (1 + np.exp(-gate))
    return rnd(d_act * up * s * (1 + gate * (1 - s))), rnd(d_act * gate * s)


def test_token_and_routing_weight_gradients(step):
    """dx[t] = bf16(sum over slots of dGate W_gate + dUp W_up) (fp32 inside),
    d weight[t, s] = G[t] . down row (fp32), d logits from the routing
    backward (cpu_lm.routing_backward)."""
    tokens = _sample_tokens()
    dx = np.zeros((tokens.size, WIDTH))
    for i, t in enumerate(tokens):
        p = step["position"][t * TOP_K:(t + 1) * TOP_K]
        e = step["expert_of"][p]
        d_down = _d_down(step, p)
        d_act = rnd(np.einsum("pw,pwh->ph", d_down, step["wd"][e]))
        d_gate, d_up = _d_gate_up(d_act, step["gate"][p], step["up"][p])
        dx[i] = (np.einsum("ph,phw->pw", d_gate, step["wg"][e]) + np.einsum("ph,phw->pw", d_up, step["wu"][e])).sum(0)
    assert ora.rel_frobenius(step["dx"][tokens], rnd(dx)) <= 1e-2
    d_weights = np.einsum("tsw,tsw->ts", step["g"][:, None, :].repeat(TOP_K, 1),
                          step["down"][step["position"].reshape(TOKENS, TOP_K)]).ravel()
    assert ora.rel_frobenius(step["d_weights"], d_weights) <= 1e-5
    ref = ora.routing(step["logits"].astype(np.float64).tolist(), TOKENS, EXPERTS, TOP_K)
    d_logits = ora.routing_backward(step["d_weights"].tolist(), ref)
    assert ora.rel_frobenius(step["d_logits"], np.array(d_logits)) <= 1e-5


@pytest.mark.parametrize("expert", range(EXPERTS))
def test_expert_weight_gradient_rows(step, expert):
    """Rows of dW_down = dDown^T act, dW_gate = dGate^T x and dW_up = dUp^T x
    over the expert's routed rows (fp32 sums, one bf16 rounding)."""
    lo, hi = step["offsets"][expert], step["offsets"][expert + 1]
    positions = np.arange(lo, hi)
    rng = np.random.default_rng(100 + expert)
    d_down = _d_down(step, positions)
    out_rows = rng.choice(WIDTH, 3, replace=False)
    dwd = rnd(d_down[:, out_rows].T @ step["act"][positions])
    assert ora.rel_frobenius(step["dwd"][expert, out_rows], dwd) <= 1e-2
    hidden_rows = rng.choice(HIDDEN, 3, replace=False)
    d_act = rnd(d_down @ step["wd"][expert][:, hidden_rows])
    d_gate, d_up = _d_gate_up(d_act, step["gate"][positions][:, hidden_rows], step["up"][positions][:, hidden_rows])
    rows = step["rows"][positions]
    assert ora.rel_frobenius(step["dwg"][expert, hidden_rows], rnd(d_gate.T @ rows)) <= 1e-2
    assert ora.rel_frobenius(step["dwu"][expert, hidden_rows], rnd(d_up.T @ rows)) <= 1e-2
