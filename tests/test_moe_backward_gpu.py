"""MoE training path on the MI355X: routing backward, combine backward,
grouped-K weight-gradient GEMM and the SparseMoE layer's autograd, against
the float64 oracle (cpu_lm.routing_backward / combine_backward,
src/qutai/backends/cpu_lm.py:245-320) and a float64 restatement of the
expert SwiGLU backward (lm/layers.py:291-314, 376-402)."""
import numpy as np
import pytest

from oracle import reference as ora
from tests.helpers import download, normal, stored, upload

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-5
BF16_TOL = 1e-2


@pytest.fixture(scope="module")
def lm():
    from qutai_amd.backends import amd, amd_lm

    amd.get_runtime()
    return amd_lm


def test_routing_backward_weights_and_aux(lm):
    rows, experts, top_k = 1000, 8, 2
    logits = normal(90, rows * experts)
    route = lm.routing(upload(logits, "float32"), rows, experts, top_k)
    reference = ora.routing(logits.astype(np.float64).tolist(), rows, experts, top_k)
    g = normal(91, rows * top_k)
    got = download(lm.routing_backward(upload(g, "float32"), route))
    expected = ora.routing_backward(g.astype(np.float64).tolist(), reference)
    assert ora.rel_frobenius(got, expected) <= FP32_TOL
    aux = download(lm.routing_backward(upload(np.array([0.37], dtype=np.float32), "float32"), route, True))
    expected_aux = ora.routing_backward([float(np.float32(0.37))], reference, auxiliary=True)
    assert ora.rel_frobenius(aux, expected_aux) <= FP32_TOL


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
@pytest.mark.parametrize("width", [64, 36, 2048])  # 16-byte rows (vector kernel) and not (element kernel)
def test_combine_backward_all_and_reference_shape(lm, dtype, width):
    rows, experts, top_k = 517, 5, 3
    scores = [((row * 37 + expert * 11) % 101) / 13 for row in range(rows) for expert in range(experts)]
    route = lm.routing(upload(np.array(scores, dtype=np.float32), "float32"), rows, experts, top_k)
    reference = ora.routing([float(np.float32(s)) for s in scores], rows, experts, top_k)
    block = normal(92, route["capacity"] * width)
    g = normal(93, rows * width)
    d_block, d_w = lm.combine_backward_all(upload(g, dtype), upload(block, dtype), route, width)
    offsets = np.concatenate([[0], np.cumsum(reference["counts"])])
    outputs = [(e, stored(block, dtype)[offsets[e] * width:offsets[e + 1] * width].tolist())
               for e in range(experts) if reference["counts"][e]]
    weights = download(route["weights"]).astype(np.float64).tolist()
    *grads, dw = ora.combine_backward(stored(g, dtype).tolist(), outputs, weights, reference, width)
    expected_block = np.concatenate([np.array(x) for x in grads])
    tol = FP32_TOL if dtype == "float32" else BF16_TOL
    assert ora.rel_frobenius(download(d_block), expected_block) <= tol
    assert ora.rel_frobenius(download(d_w), dw) <= FP32_TOL
    # the reference-shaped wrapper returns the same rows per expert
    outs = [(e, upload(np.array(v, dtype=np.float32), dtype)) for e, v in outputs]
    *parts, dw2 = lm.combine_backward(upload(g, dtype), outs, route["weights"], route, width)
    for part, ref in zip(parts, grads):
        assert ora.rel_frobenius(download(part), ref) <= tol


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_grouped_k_weight_gradient_gemm(lm, dtype):
    # config-5-like uneven expert sizes (C5 logits), 1408 x 2048 products per expert
    rows, experts, top_k = 8192, 8, 2
    logits = normal(4, rows * experts)
    route = lm.routing(upload(logits, "float32"), rows, experts, top_k)
    m, n = (256, 512) if dtype == "float32" else (1408, 2048)
    a = normal(94, route["capacity"] * m)
    b = normal(95, route["capacity"] * n)
    out = lm.grouped_gemm_k(upload(a, dtype), upload(b, dtype), route, m, n)
    got = download(out).reshape(experts, m, n)
    offsets = np.concatenate([[0], np.cumsum(route["counts"])])
    A = stored(a, dtype).reshape(-1, m)
    B = stored(b, dtype).reshape(-1, n)
    for e in (0, 3, 7):
        lo, hi = offsets[e], offsets[e + 1]
        sample = list(range(0, m, max(1, m // 48))) + [m - 1]
        expected = ora.gemm_f64(A[lo:hi], B[lo:hi], m, hi - lo, n, transpose_left=True, row_list=sample)
        assert ora.rel_frobenius(got[e][sample], expected) <= FP32_TOL


def test_grouped_k_empty_group_writes_zeros(lm):
    rows, experts, top_k = 6, 4, 1
    # every token picks expert 1 or 2: experts 0 and 3 are empty
    scores = np.full((rows, experts), -5.0, dtype=np.float32)
    scores[:3, 1] = 5.0
    scores[3:, 2] = 5.0
    route = lm.routing(upload(scores.ravel(), "float32"), rows, experts, top_k)
    assert route["counts"] == (0, 3, 3, 0)
    a, b = normal(96, rows * 8), normal(97, rows * 8)
    got = download(lm.grouped_gemm_k(upload(a, "float32"), upload(b, "float32"), route, 8, 8)).reshape(4, 8, 8)
    assert not got[0].any() and not got[3].any()
    A, B = a.reshape(rows, 8).astype(np.float64), b.reshape(rows, 8).astype(np.float64)
    assert ora.rel_frobenius(got[1], A[:3].T @ B[:3]) <= FP32_TOL


def _silu(z):
    return z / (1 + np.exp(-z))


def moe_reference(x, wr, wg, wu, wd, top_k, G, c):
    """float64 forward + backward of SparseMoE for loss = sum(y * G) + c * aux."""
    tokens, width = x.shape
    experts = wr.shape[0]
    scores = x @ wr.T
    route = ora.routing(scores.ravel().tolist(), tokens, experts, top_k)
    y = np.zeros_like(x)
    dx = np.zeros_like(x)
    dwg, dwu, dwd = np.zeros_like(wg), np.zeros_like(wu), np.zeros_like(wd)
    dweights = np.zeros(tokens * top_k)
    for r in range(tokens):
        for s in range(top_k):
            e = route["indices"][r * top_k + s]
            w = route["weights"][r * top_k + s]
            hg, hu = wg[e] @ x[r], wu[e] @ x[r]
            a = _silu(hg) * hu
            o = wd[e] @ a
            y[r] += w * o
            do = w * G[r]
            dweights[r * top_k + s] = G[r] @ o
            da = wd[e].T @ do
            dwd[e] += np.outer(do, a)
            sig = 1 / (1 + np.exp(-hg))
            dhg = da * hu * sig * (1 + hg * (1 - sig))
            dhu = da * _silu(hg)
            dx[r] += wg[e].T @ dhg + wu[e].T @ dhu
            dwg[e] += np.outer(dhg, x[r])
            dwu[e] += np.outer(dhu, x[r])
    ds = np.array(ora.routing_backward(dweights.tolist(), route)) + np.array(
        ora.routing_backward([c], route, auxiliary=True))
    ds = ds.reshape(tokens, experts)
    dwr = ds.T @ x
    dx += ds @ wr
    return y, route["aux"], dx, dwr, dwg, dwu, dwd


def test_sparse_moe_layer_forward_and_all_gradients(lm):
    from qutai_amd import Tensor
    from qutai_amd.lm.layers import SparseMoE

    tokens, width, hidden, experts, top_k = 96, 32, 24, 4, 2
    layer = SparseMoE(width, hidden, experts, top_k, seed=5)
    xv = normal(98, tokens * width)
    x = Tensor(upload(xv, "float32"), shape=(tokens, width), requires_grad=True)
    y, aux = layer(x)
    G = normal(99, tokens * width)
    c = 0.25
    y.backward(Tensor(upload(G, "float32"), shape=y.shape))
    aux.backward(Tensor(upload(np.array([c], dtype=np.float32), "float32"), shape=()))
    f64 = lambda t, shape: download(t.storage).astype(np.float64).reshape(shape)  # noqa: E731
    wr = f64(layer.router.weight, (experts, width))
    wg, wu = f64(layer.w_gate, (experts, hidden, width)), f64(layer.w_up, (experts, hidden, width))
    wd = f64(layer.w_down, (experts, width, hidden))
    ry, raux, rdx, rdwr, rdwg, rdwu, rdwd = moe_reference(xv.reshape(tokens, width).astype(np.float64), wr, wg, wu,
                                                          wd, top_k, G.reshape(tokens, width).astype(np.float64),
                                                          float(np.float32(c)))
    # fp32 storage, true fp32 MFMA products: the reference's own GPU pin
    # for the MoE layer (tests/test_lm_moe.py:105-138) is 2e-5
    tol = 2e-5
    errors = dict(y=ora.rel_frobenius(f64(y, (tokens, width)), ry),
                  x=ora.rel_frobenius(f64(x.grad, (tokens, width)), rdx),
                  router=ora.rel_frobenius(f64(layer.router.weight.grad, (experts, width)), rdwr),
                  w_gate=ora.rel_frobenius(f64(layer.w_gate.grad, wg.shape), rdwg),
                  w_up=ora.rel_frobenius(f64(layer.w_up.grad, wu.shape), rdwu),
                  w_down=ora.rel_frobenius(f64(layer.w_down.grad, wd.shape), rdwd))
    print({k: f"{v:.2e}" for k, v in errors.items()})
    assert abs(download(aux.storage)[0] - raux) <= 1e-5 * max(1, abs(raux))
    assert max(errors.values()) <= tol, errors
    assert sum(layer.last_counts) == tokens * top_k


@pytest.mark.parametrize("dtype,width,hidden", [("bfloat16", 256, 200), ("float32", 256, 200),
                                                ("bfloat16", 36, 20)])
def test_backward_through_the_order_equals_the_gathered_copy(lm, dtype, width, hidden):
    """The training forward reads the token rows through the route's order
    (no routed copy), and the backward's dW_gate / dW_up read them the same
    way: every output and gradient is bit-identical to the backward over the
    gathered block (uneven experts, one with no rows; widths that are not a
    multiple of 8 run on the zero-padded token matrix)."""
    tokens, experts, top_k = 700, 8, 2
    logits = normal(95, tokens * experts)
    logits[1::experts] -= 50.0  # expert 1 gets no tokens
    route = lm.routing(upload(logits, "float32"), tokens, experts, top_k)
    xs = upload(normal(96, tokens * width), dtype)
    ws = [upload(normal(97 + i, experts * hidden * width, 0.05), dtype) for i in range(3)]
    g = upload(normal(100, tokens * width), dtype)
    y, saved = lm.moe_experts_forward(xs, route, *ws, width, hidden, save=True)
    assert saved["gathered"] and (saved["rows"] is xs) == (width % 8 == 0)
    padded = (width + 7) // 8 * 8
    copy = dict(saved, rows=lm.route_gather_all(saved["rows"], route, padded), gathered=False)
    through = lm.moe_experts_backward(g, route, saved, width, hidden, x_dtype=dtype, weight_dtype=dtype)
    copied = lm.moe_experts_backward(g, route, copy, width, hidden, x_dtype=dtype, weight_dtype=dtype)
    for a, b in zip(through, copied):
        assert np.array_equal(np.frombuffer(a.to_array(), np.uint8), np.frombuffer(b.to_array(), np.uint8))
    y_plain = lm.moe_experts_forward(xs, route, *ws, width, hidden)  # the forward alone gathers too
    assert np.array_equal(np.frombuffer(y.to_array(), np.uint8), np.frombuffer(y_plain.to_array(), np.uint8))


def test_gather_backward_rounds_fp32_slot_sums_once_to_bf16(lm):
    """The token gradient of the gather: fp32 expert rows summed over each
    token's slots straight into bf16 equals the fp32 sum rounded afterwards
    (one rounding either way), bit for bit; ragged width too."""
    from qutai_amd.backends import amd

    for rows, width in ((700, 256), (97, 12)):
        route = lm.routing(upload(normal(rows, rows * 8), "float32"), rows, 8, 2)
        d_rows = upload(normal(rows + 1, route["capacity"] * width), "float32")
        wide = lm.route_gather_backward_all(d_rows, route, width)
        narrow = lm.route_gather_backward_all(d_rows, route, width, out_dtype="bfloat16")
        assert narrow.dtype == "bfloat16"
        assert narrow.to_array() == amd.from_storage(wide, dtype="bfloat16").to_array()
