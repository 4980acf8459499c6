"""Fused SwiGLU GEMM (qutai_amd_gemm_swiglu) against the unfused form it
replaces -- two projections, lm_silu and the multiply
(src/qutai/lm/layers.py:310-311) -- bit for bit: the fused epilogue rounds
gate and up to bf16, silu(gate) to bf16 and the product once, exactly as
the separate bf16 GEMMs and the elementwise kernel do, and every tile sums K
in the same order.  Also against a float64 composition of the oracle's silu
(tolerance 1e-2, bf16 storage), in plain form and grouped by expert with the
config 5 routing of uneven per-expert counts (one expert with no rows)."""
import numpy as np
import pytest

from oracle import reference as ora
from tests.helpers import download, normal, stored, upload

pytestmark = pytest.mark.gpu

BF16_TOL = 1e-2


@pytest.fixture(scope="module")
def amd():
    from qutai_amd.backends import amd as backend

    backend.get_runtime()
    return backend


@pytest.fixture(scope="module")
def lm():
    from qutai_amd.backends import amd_lm

    return amd_lm


def words(storage):
    return np.frombuffer(storage.to_array(), dtype=np.uint16)


def reference_act(x, wg, wu):
    """float64 silu(x wg^T) * (x wu^T) of bf16-stored operands (rows x hidden)."""
    g = x @ wg.T
    u = x @ wu.T
    return np.array(ora.silu(g.ravel().tolist())).reshape(g.shape) * u


@pytest.mark.parametrize("rows,inner,hidden", [(512, 256, 256), (300, 136, 264), (257, 64, 8), (1000, 512, 1408)])
def test_plain_swiglu_matches_unfused_bit_for_bit(amd, lm, rows, inner, hidden):
    x = normal(rows, rows * inner)
    wg, wu = normal(1, hidden * inner, 0.1), normal(2, hidden * inner, 0.1)
    xs, gs, us = (upload(v, "bfloat16") for v in (x, wg, wu))
    act, gate, up = lm.swiglu_gemm(xs, gs, us, rows, inner, hidden, save=True)
    gate_ref = amd.gemm(xs, gs, rows, inner, hidden, transpose_right=True, out_dtype="bfloat16")
    up_ref = amd.gemm(xs, us, rows, inner, hidden, transpose_right=True, out_dtype="bfloat16")
    act_ref = lm.silu_mul(gate_ref, up_ref)
    assert np.array_equal(words(gate), words(gate_ref))
    assert np.array_equal(words(up), words(up_ref))
    assert np.array_equal(words(act), words(act_ref))
    # the form without the saved products writes the same activations
    assert np.array_equal(words(lm.swiglu_gemm(xs, gs, us, rows, inner, hidden)), words(act_ref))
    exact = reference_act(stored(x, "bfloat16").reshape(rows, inner), stored(wg, "bfloat16").reshape(hidden, inner),
                          stored(wu, "bfloat16").reshape(hidden, inner))
    assert ora.rel_frobenius(download(act).reshape(rows, hidden), exact) <= BF16_TOL


@pytest.mark.parametrize("tokens,width,hidden,experts,top_k", [(2048, 256, 200, 8, 2), (700, 128, 1408, 8, 2),
                                                                (64, 64, 136, 16, 1)])
def test_grouped_swiglu_matches_unfused_bit_for_bit(amd, lm, tokens, width, hidden, experts, top_k):
    logits = normal(tokens + 1, tokens * experts)
    route = lm.routing(upload(logits, "float32"), tokens, experts, top_k)
    x = normal(tokens + 2, tokens * width)
    wg, wu = normal(3, experts * hidden * width, 0.1), normal(4, experts * hidden * width, 0.1)
    xs, gs, us = (upload(v, "bfloat16") for v in (x, wg, wu))
    rows = lm.route_gather_all(xs, route, width)
    act, gate, up = lm.swiglu_gemm(rows, gs, us, 0, width, hidden, route=route, save=True)
    gate_ref = lm.grouped_gemm(rows, gs, route, width, hidden, out_dtype="bfloat16")
    up_ref = lm.grouped_gemm(rows, us, route, width, hidden, out_dtype="bfloat16")
    act_ref = lm.silu_mul(gate_ref, up_ref)
    used = int(download(route["offsets"])[-1]) * hidden  # rows past the last expert are not written
    assert np.array_equal(words(gate)[:used], words(gate_ref)[:used])
    assert np.array_equal(words(up)[:used], words(up_ref)[:used])
    assert np.array_equal(words(act)[:used], words(act_ref)[:used])
    # rows read through the route's order inside the GEMM: the same values,
    # with and without the saved products (the training forward)
    act_g = lm.swiglu_gemm(xs, gs, us, 0, width, hidden, route=route, gather=True)
    assert np.array_equal(words(act_g)[:used], words(act)[:used])
    act_gs, gate_gs, up_gs = lm.swiglu_gemm(xs, gs, us, 0, width, hidden, route=route, gather=True, save=True)
    for got, ref in ((act_gs, act), (gate_gs, gate), (up_gs, up)):
        assert np.array_equal(words(got)[:used], words(ref)[:used])
    # float64 check on every expert's first and last row
    offsets = download(route["offsets"]).astype(int).tolist()
    xr = stored(download(rows), "bfloat16").reshape(-1, width)
    gr = stored(wg, "bfloat16").reshape(experts, hidden, width)
    ur = stored(wu, "bfloat16").reshape(experts, hidden, width)
    got = download(act).reshape(-1, hidden)
    for e in range(experts):
        lo, hi = offsets[e], offsets[e + 1]
        for r in sorted({lo, hi - 1}) if hi > lo else ():
            exact = reference_act(xr[r:r + 1], gr[e], ur[e])
            assert ora.rel_frobenius(got[r:r + 1], exact) <= BF16_TOL


@pytest.mark.parametrize("dtype,tokens,width,cols,experts,top_k", [
    ("bfloat16", 1500, 256, 200, 8, 2), ("bfloat16", 700, 1408, 2048, 8, 2), ("float32", 900, 132, 96, 4, 2),
    ("bfloat16", 40, 64, 8, 16, 1)])
def test_grouped_gemm_gather_equals_gathered_block(amd, lm, dtype, tokens, width, cols, experts, top_k):
    """The grouped GEMM reading its rows through `order` (token gather inside
    the operand copy) is bit-identical to the GEMM over the gathered block,
    including experts with no rows and a partial last tile per expert."""
    logits = normal(tokens + 3, tokens * experts)
    route = lm.routing(upload(logits, "float32"), tokens, experts, top_k)
    xs = upload(normal(tokens + 4, tokens * width), dtype)
    ws = upload(normal(5, experts * cols * width, 0.1), dtype)
    rows = lm.route_gather_all(xs, route, width)
    used = int(download(route["offsets"])[-1]) * cols
    for out_dtype in ("float32", dtype):
        ref = download(lm.grouped_gemm(rows, ws, route, width, cols, out_dtype=out_dtype))
        got = download(lm.grouped_gemm(xs, ws, route, width, cols, out_dtype=out_dtype, gather=True))
        assert np.array_equal(got[:used], ref[:used]), out_dtype
    if top_k > 1:
        with pytest.raises(ValueError):  # the gathered form takes the token matrix
            lm.grouped_gemm(rows, ws, route, width, cols, gather=True, out_dtype=dtype)


@pytest.mark.parametrize("dtype,tokens,rows,cols,experts,top_k", [
    ("bfloat16", 1500, 200, 256, 8, 2), ("bfloat16", 8192, 1408, 2048, 8, 2), ("bfloat16", 700, 2048, 1408, 8, 2),
    ("float32", 900, 96, 132, 4, 2), ("bfloat16", 40, 64, 8, 16, 1)])
def test_grouped_k_gather_equals_gathered_block(amd, lm, dtype, tokens, rows, cols, experts, top_k):
    """The grouped-K weight-gradient GEMM reading B's K rows (the token rows)
    through `order` is bit-identical to the GEMM over the gathered block:
    config 5's dW_gate shape, uneven experts, empty experts (16 experts over
    40 tokens), K ranges that end inside a K step, ragged column tiles."""
    logits = normal(tokens + 5, tokens * experts)
    route = lm.routing(upload(logits, "float32"), tokens, experts, top_k)
    xs = upload(normal(tokens + 6, tokens * cols), dtype)
    a = upload(normal(tokens + 7, route["capacity"] * rows), dtype)
    block = lm.route_gather_all(xs, route, cols)
    for out_dtype in ("float32", dtype):
        ref = download(lm.grouped_gemm_k(a, block, route, rows, cols, out_dtype=out_dtype))
        got = download(lm.grouped_gemm_k(a, xs, route, rows, cols, out_dtype=out_dtype, gather=True))
        assert np.array_equal(got, ref), out_dtype
    if top_k > 1:
        with pytest.raises(ValueError):  # the gathered form takes the token matrix
            lm.grouped_gemm_k(a, block, route, rows, cols, gather=True)


def test_grouped_k_gather_index_outside_the_tokens_reads_zeros(amd, lm):
    """Order entries outside the token rows (the row count, -1, and an index
    whose 32-bit byte offset would wrap onto row 1: 2^32 / 128 + 1 rows of
    64 bf16) contribute zero rows to the weight gradients."""
    from array import array

    tokens, rows, cols, experts = 40, 16, 64, 4
    route = lm.routing(upload(normal(80, tokens * experts), "float32"), tokens, experts, 2)
    xs = upload(normal(81, tokens * cols), "bfloat16")
    a = upload(normal(82, route["capacity"] * rows), "bfloat16")
    order = np.frombuffer(route["order"].to_array(), dtype=np.int64).copy()
    bad = {3: tokens, 10: -1, 17: (1 << 32) // 128 + 1}
    for position, index in bad.items():
        order[position] = index
    broken = dict(route, order=amd.storage(array("q", order.tolist()), dtype="int64"))
    got = download(lm.grouped_gemm_k(a, xs, broken, rows, cols, gather=True))
    # the reference block: the gathered rows with the broken positions zeroed
    block = stored(download(xs), "bfloat16").reshape(tokens, cols)[np.clip(order, 0, tokens - 1)]
    block[list(bad)] = 0
    ref = download(lm.grouped_gemm_k(a, upload(block.ravel(), "bfloat16"), route, rows, cols))
    assert np.array_equal(got, ref)


def test_grouped_gemm_gather_index_outside_the_tokens_reads_zeros(amd, lm):
    """Route order entries outside the token rows -- the row count, -1, and
    an index whose 32-bit byte offset would wrap onto row 1 (64 bf16 values
    = 128 bytes per row, 2^32 / 128 + 1) -- give zero rows; every other row
    is unchanged."""
    from array import array

    tokens, width, cols, experts = 40, 64, 32, 4
    route = lm.routing(upload(normal(77, tokens * experts), "float32"), tokens, experts, 2)
    xs = upload(normal(78, tokens * width), "bfloat16")
    ws = upload(normal(79, experts * cols * width, 0.1), "bfloat16")
    ref = download(lm.grouped_gemm(xs, ws, route, width, cols, out_dtype="float32", gather=True)).reshape(-1, cols)
    order = np.frombuffer(route["order"].to_array(), dtype=np.int64).copy()
    bad = {3: tokens, 10: -1, 17: (1 << 32) // 128 + 1}
    for position, index in bad.items():
        order[position] = index
    broken = dict(route, order=amd.storage(array("q", order.tolist()), dtype="int64"))
    got = download(lm.grouped_gemm(xs, ws, broken, width, cols, out_dtype="float32", gather=True)).reshape(-1, cols)
    for position in range(ref.shape[0]):
        if position in bad:
            assert np.all(got[position] == 0), position
        else:
            assert np.array_equal(got[position], ref[position]), position


@pytest.mark.parametrize("dtype,tokens,inner,cols,experts,transpose_right", [
    ("bfloat16", 1500, 128, 200, 8, False), ("bfloat16", 700, 1408, 2048, 8, False),
    ("bfloat16", 600, 64, 96, 4, True), ("float32", 900, 192, 96, 4, False), ("bfloat16", 40, 64, 16, 16, False)])
def test_grouped_gemm_pair_sums_two_products(amd, lm, dtype, tokens, inner, cols, experts, transpose_right):
    """One grouped launch over K = 2 inner summing a b + a_tail b_tail: with
    either half zero it is bit-identical to the other half's grouped GEMM
    (pins both halves' addressing), and with both it matches the two fp32
    products added on the host to fp32 rounding and the float64 product of
    the stored operands."""
    logits = normal(tokens + 7, tokens * experts)
    route = lm.routing(upload(logits, "float32"), tokens, experts, 2 if experts < 16 else 1)  # 16: empty experts
    capacity = route["capacity"]
    used = int(download(route["offsets"])[-1])
    a, a_tail = (upload(normal(seed, capacity * inner), dtype) for seed in (11, 12))
    b, b_tail = (upload(normal(seed, experts * cols * inner, 0.1), dtype) for seed in (13, 14))
    zero = upload(np.zeros(capacity * inner), dtype)
    kw = dict(out_dtype="float32", transpose_right=transpose_right)
    head = download(lm.grouped_gemm(a, b, route, inner, cols, **kw))[:used * cols]
    tail = download(lm.grouped_gemm(a_tail, b_tail, route, inner, cols, **kw))[:used * cols]
    only_head = download(lm.grouped_gemm_pair(a, zero, b, b_tail, route, inner, cols, **kw))[:used * cols]
    only_tail = download(lm.grouped_gemm_pair(zero, a_tail, b, b_tail, route, inner, cols, **kw))[:used * cols]
    assert np.array_equal(only_head, head) and np.array_equal(only_tail, tail)
    both = download(lm.grouped_gemm_pair(a, a_tail, b, b_tail, route, inner, cols, **kw))[:used * cols]
    summed = head.astype(np.float32) + tail.astype(np.float32)
    assert ora.rel_frobenius(both, summed) <= 1e-6
    # float64 product of the stored values for the first expert's rows
    offsets = download(route["offsets"])
    lo, hi = int(offsets[0]), int(offsets[1])
    host = {name: ora.bf16_values(np.frombuffer(t.to_array(), dtype=np.uint16)) if dtype == "bfloat16"
            else np.frombuffer(t.to_array(), dtype=np.float32).astype(np.float64)
            for name, t in (("a", a), ("at", a_tail), ("b", b), ("bt", b_tail))}
    shape = (cols, inner) if transpose_right else (inner, cols)
    w0, wt0 = host["b"][:cols * inner].reshape(shape), host["bt"][:cols * inner].reshape(shape)
    if transpose_right:
        w0, wt0 = w0.T, wt0.T
    exact = host["a"].reshape(capacity, inner)[lo:hi] @ w0 + host["at"].reshape(capacity, inner)[lo:hi] @ wt0
    got = both.reshape(used, cols)[lo:hi]
    assert ora.rel_frobenius(got, exact) <= 1e-5
    with pytest.raises(ValueError):  # the join must fall on a multiple of 64
        lm.grouped_gemm_pair(upload(normal(1, capacity * 72), dtype), upload(normal(2, capacity * 72), dtype),
                             upload(normal(3, experts * cols * 72), dtype), upload(normal(4, experts * cols * 72), dtype),
                             route, 72, cols, **kw)


def test_swiglu_rejects_unsupported_operands(amd, lm):
    x = upload(normal(0, 16 * 12), "bfloat16")
    w = upload(normal(1, 8 * 12), "bfloat16")
    with pytest.raises(ValueError):  # inner not a multiple of 8
        lm.swiglu_gemm(x, w, w, 16, 12, 8)
    xf = upload(normal(0, 16 * 16), "float32")
    wf = upload(normal(1, 8 * 16), "float32")
    with pytest.raises(ValueError):  # fp32 storage keeps the unfused path
        lm.swiglu_gemm(xf, wf, wf, 16, 16, 8)


@pytest.mark.parametrize("mode", ["autocast", "bf16"])
def test_swiglu_layer_fused_equals_unfused(amd, mode):
    """lm SwiGLU (lm/layers.py:291-314) on the bf16 path: the fused op's
    output and every gradient equal the unfused composition's bit for bit."""
    from qutai_amd import Tensor
    from qutai_amd.lm import layers
    from qutai_amd.lm.precision import autocast

    width, hidden, tokens = 128, 200, 96
    dtype = "bfloat16" if mode == "bf16" else "float32"
    layer = layers.SwiGLU(width, hidden, seed=3, std=0.05, dtype=dtype)
    x = Tensor(upload(normal(21, tokens * width), dtype), shape=(tokens, width), requires_grad=True)
    # the output is bf16 in both modes (autocast: bf16 activations)
    g = Tensor(upload(normal(22, tokens * width), "bfloat16"), shape=(tokens, width))
    params = (x, *layer.parameters())

    def run(fused):
        for p in params:
            p.grad = None
        with autocast(mode == "autocast"):
            assert layers._swiglu_fusable(x, layer.gate.weight, layer.up.weight)
            if fused:
                y = layer(x)
            else:
                y = layer.down(layers.silu_mul(layer.gate(x), layer.up(x)))
        y.backward(g)
        return [y.storage.to_array()] + [p.grad.storage.to_array() for p in params]

    fused, unfused = run(True), run(False)
    for name, a, b in zip(("y", "dx", "dWg", "dWu", "dWd"), fused, unfused):
        assert a == b, name
