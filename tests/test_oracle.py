"""Pins the CPU oracle before it is trusted as the parity reference.

Each oracle function is checked against the reference's own known-answer
tests (golden vectors, cited per test), against what mathematics fixes
(closed forms, invariants), and against an independent restatement (the
Python loop vs the compiled C loop, bit for bit; numpy within tolerance),
chosen so that a dropped term, a swapped index or a transposed operand
fails at least one check.
"""
import math
import random

import numpy as np
import pytest

from oracle import reference as ora


# ---- GEMM / matmul --------------------------------------------------------------

def test_matmul_golden_vectors_from_reference_tests():
    # tests/test_batched_matmul.py:28-37
    assert ora.matmul([1, 2, 3], [4, 5, 6], (3,), (3,)) == [32]
    assert ora.matmul([1, 2], [3, 4, 5, 6, 7, 8], (2,), (2, 3)) == [15, 18, 21]
    assert ora.matmul([1, 2, 3, 4], [5, 6], (2, 2), (2,)) == [17, 39]
    # tests/test_batched_matmul.py:39-42
    matrices = [1, 2, 3, 4, 5, 6, 7, 8]
    assert ora.matmul([1, 2], matrices, (2,), (2, 2, 2)) == [7, 10, 19, 22]
    assert ora.matmul(matrices, [1, 2], (2, 2, 2), (2,)) == [5, 11, 17, 23]
    # tests/test_gemm_precision.py:86-90: left broadcast over a batch of 2
    assert ora.matmul([1, 2, 3, 4, 5, 6], [1, 2, 3, 4, 5, 6, 6, 5, 4, 3, 2, 1], (2, 3), (2, 3, 2)) == [
        22, 28, 49, 64, 20, 14, 56, 41]


def test_matmul_batch_broadcast_does_not_mix_matrices():
    # tests/test_batched_matmul.py:44-53, brute force over both broadcast axes
    left = list(range(1, 13))
    right = list(range(1, 19))
    a = np.array(left, dtype=float).reshape(2, 1, 2, 3)
    b = np.array(right, dtype=float).reshape(1, 3, 3, 2)
    expected = [sum(a[g][0][r][k] * b[0][z][k][c] for k in range(3))
                for g in range(2) for z in range(3) for r in range(2) for c in range(2)]
    assert ora.matmul(left, right, (2, 1, 2, 3), (1, 3, 3, 2)) == expected


def test_accumulation_order_is_sequential_k():
    # tests/test_batched_matmul.py:105-106: (1e16 + 1) - 1e16 == 0 only in order
    assert ora.matmul([1e16, 1, -1e16], [1, 1, 1], (1, 3), (3, 1)) == [0.0]
    out = ora.gemm_f64(np.array([1e16, 1, -1e16]), np.array([1.0, 1, 1]), 1, 3, 1)
    assert out.tolist() == [[0.0]]


def test_linear_known_answers_through_matmul():
    # tests/test_layers.py:23-33: X @ W + b with W stored (in, out)
    w = [1, 2, 3, 4, 5, 6]
    x = [1, 2, -1, 0]
    y = ora.matmul(x, w, (2, 2), (2, 3))
    bias = [0.5, -0.5, 1]
    assert [v + bias[i % 3] for i, v in enumerate(y)] == [9.5, 11.5, 16, -0.5, -2.5, -2]
    # tests/test_layers.py:35-43: gradients of sum(X @ W + b)
    ones = [1.0] * 4
    dx = ora.gemm(ones, [1, 2, 3, 4], 2, 2, 2, transpose_right=True)
    dw = ora.gemm([1, 2, 3, 4], ones, 2, 2, 2, transpose_left=True)
    assert dx == [3, 7, 3, 7]
    assert dw == [4, 4, 6, 6]


def test_gemm_transposes_follow_the_reference_index_maps():
    rng = random.Random(11)
    m, k, n = 3, 4, 5
    a = [rng.uniform(-1, 1) for _ in range(m * k)]
    b = [rng.uniform(-1, 1) for _ in range(k * n)]
    A, B = np.array(a).reshape(m, k), np.array(b).reshape(k, n)
    for ta in (False, True):
        for tb in (False, True):
            a_in = (A.T if ta else A).ravel().tolist()
            b_in = (B.T if tb else B).ravel().tolist()
            got = ora.gemm(a_in, b_in, m, k, n, transpose_left=ta, transpose_right=tb)
            assert np.allclose(np.array(got).reshape(m, n), A @ B, rtol=1e-13, atol=1e-13)


def test_python_and_compiled_gemm_agree_bit_for_bit():
    rng = np.random.default_rng(5)
    for (m, k, n) in [(7, 13, 5), (16, 64, 9), (1, 1, 1), (3, 0, 2)]:
        for ta in (False, True):
            for tb in (False, True):
                a = rng.standard_normal(m * k)
                b = rng.standard_normal(k * n)
                old = rng.standard_normal(m * n)
                for accumulate in (False, True):
                    py = ora.gemm(a.tolist(), b.tolist(), m, k, n, transpose_left=ta, transpose_right=tb,
                                  out=old.tolist() if accumulate else None, accumulate=accumulate)
                    c = ora.gemm_f64(a, b, m, k, n, transpose_left=ta, transpose_right=tb,
                                     out=old if accumulate else None, accumulate=accumulate)
                    assert c.ravel().tolist() == py


def test_compiled_gemm_row_subset_and_threads_do_not_change_bits():
    rng = np.random.default_rng(6)
    m, k, n = 37, 300, 23
    a, b = rng.standard_normal(m * k), rng.standard_normal(k * n)
    full = ora.gemm_f64(a, b, m, k, n, threads=1)
    rows = [0, 5, 36, 17]
    part = ora.gemm_f64(a, b, m, k, n, row_list=rows, threads=3)
    assert np.array_equal(part, full[rows])
    assert np.array_equal(ora.gemm_f64(a, b, m, k, n, threads=7), full)
    assert np.allclose(full, a.reshape(m, k) @ b.reshape(k, n), rtol=1e-12, atol=1e-12)


def test_long_reduction_closed_form():
    # tests/test_gemm_precision.py:191-206 in miniature: 0.5 * -0.25 summed k times
    k = 8193
    out = ora.gemm_f64(np.full(2 * k, 0.5), np.full(k * 3, -0.25), 2, k, 3, out=np.full(6, 0.25), accumulate=True)
    assert (out == -k * 0.125 + 0.25).all()


# ---- bf16 ---------------------------------------------------------------------

def test_bf16_rounding_golden_values():
    # tests/test_bfloat16_storage.py:20-24 inputs; the expected values follow
    # from round-to-nearest-even: 1 + 2^-8 is a tie between 1 and 1 + 2^-7
    # (even mantissa 1), 1 + 3*2^-8 a tie between 1 + 2^-7 and 1 + 2^-6.
    assert ora.bf16(1.00390625) == 1.0
    assert ora.bf16(1.01171875) == 1.015625
    assert ora.bf16(0.0) == 0.0 and math.copysign(1, ora.bf16(-0.0)) == -1
    assert ora.bf16(-2.71828) == -2.71875
    assert ora.bf16(1e30) == 202 * 2.0 ** 92  # 1e30 = 201.93 ulps of 2^92 -> 202
    assert ora.bf16(math.inf) == math.inf and ora.bf16(-math.inf) == -math.inf
    assert math.isnan(ora.bf16(math.nan))
    # tests/test_gemm_precision.py:99-112 autocast values
    assert [ora.bf16(x) for x in (0.1, 0.2, 0.3, 0.4)] == [0.10009765625, 0.2001953125, 0.30078125, 0.400390625]


def test_bf16_three_restatements_agree():
    rng = np.random.default_rng(7)
    x = np.concatenate([rng.standard_normal(4000) * 10.0 ** rng.integers(-30, 30, 4000),
                        np.array([0, -0.0, np.inf, -np.inf, np.nan, 1.00390625, 1.01171875], np.float32)])
    x = x.astype(np.float32)
    words_np = ora.bf16_words(x)
    words_c = ora.bf16_round_c(x)
    assert np.array_equal(words_np, words_c)
    py = [ora.bf16(float(v)) for v in x]
    vals = ora.bf16_values(words_np)
    for got, want in zip(vals.tolist(), py):
        assert (math.isnan(got) and math.isnan(want)) or got == want
    # every rounded value is within half a bf16 ulp (2^-8 relative) of its input
    finite = np.isfinite(x) & (x != 0)
    rel = np.abs(vals[finite].astype(np.float64) - x[finite]) / np.abs(x[finite].astype(np.float64))
    assert rel.max() <= 2.0 ** -8


# ---- softmax / silu -------------------------------------------------------------

def test_softmax_known_answer_and_invariants():
    # tests/test_attention.py:10-22: scores [1/sqrt2, 0] -> e^(1/sqrt2)/(e^(1/sqrt2)+1)
    p = math.exp(1 / math.sqrt(2)) / (math.exp(1 / math.sqrt(2)) + 1)
    got = ora.softmax([1 / math.sqrt(2), 0.0, 0.0, 1 / math.sqrt(2)], (2, 2), 1)
    assert got == pytest.approx([p, 1 - p, 1 - p, p], rel=1e-15)
    rng = random.Random(3)
    row = [rng.gauss(0, 3) for _ in range(50)]
    out = ora.softmax(row, (1, 50), 1)
    assert math.fsum(out) == pytest.approx(1.0, abs=1e-15)
    shifted = ora.softmax([v + 1000 for v in row], (1, 50), 1)
    assert shifted == pytest.approx(out, rel=1e-12)
    # axis other than the last walks the strided groups
    two = ora.softmax([0.0, 1.0, 2.0, 3.0], (2, 2), 0)
    q = 1 / (1 + math.exp(2))
    assert two == pytest.approx([q, q, 1 - q, 1 - q], rel=1e-15)


def test_silu_closed_forms():
    xs = [-30.0, -2.0, -0.5, 0.0, 0.5, 2.0, 30.0]
    ys = ora.silu(xs)
    assert ys[3] == 0.0
    for x, y in zip(xs, ys):
        assert y == pytest.approx(x / (1 + math.exp(-x)), rel=1e-14)
    # silu(x) - silu(-x) = x
    for x in (0.3, 1.7, 5.0):
        a, b = ora.silu([x, -x])
        assert a - b == pytest.approx(x, rel=1e-14)


# ---- routing / gather / combine --------------------------------------------------

def test_routing_golden_vector():
    # tests/test_lm_moe.py:65-71
    route = ora.routing([3.0, 2.0, -1.0, -1.0, 2.0, 3.0], 2, 3, 2)
    assert route["indices"] == [0, 1, 2, 1]
    assert route["counts"] == (1, 2, 1)
    assert sum(route["weights"][:2]) == pytest.approx(1)
    assert sum(route["weights"][2:]) == pytest.approx(1)
    assert route["ids"] == [[0], [0, 1], [1]]
    assert route["slots"] == [[0], [1, 1], [0]]


def test_routing_brute_force_invariants():
    # the 517 x 5 x 3 case of tests/test_lm_moe.py:140-147, checked against a
    # direct brute-force definition of each output
    rows, experts, top_k = 517, 5, 3
    scores = [((row * 37 + expert * 11) % 101) / 13 for row in range(rows) for expert in range(experts)]
    route = ora.routing(scores, rows, experts, top_k)
    for row in range(rows):
        s = scores[row * experts:(row + 1) * experts]
        # lexicographic (value desc, index asc) order = stable descending sort
        order = sorted(range(experts), key=lambda e: (-s[e], e))[:top_k]
        assert route["indices"][row * top_k:(row + 1) * top_k] == order
        w = route["weights"][row * top_k:(row + 1) * top_k]
        assert math.fsum(w) == pytest.approx(1, abs=1e-15)
        assert w == sorted(w, reverse=True)
    for e in range(experts):
        pairs = [(r, slot) for r in range(rows) for slot in range(top_k) if route["indices"][r * top_k + slot] == e]
        assert route["ids"][e] == [r for r, _ in pairs]
        assert route["slots"][e] == [slot for _, slot in pairs]
    assert sum(route["counts"]) == rows * top_k
    util = route["utilization"]
    probs = route["probs"]
    aux = experts * math.fsum(util[e] * math.fsum(probs[r * experts + e] for r in range(rows)) / rows
                              for e in range(experts))
    assert route["aux"] == pytest.approx(aux, rel=1e-12)


def test_gather_and_combine_round_trip():
    rng = random.Random(9)
    rows, experts, top_k, width = 11, 4, 2, 3
    scores = [rng.gauss(0, 1) for _ in range(rows * experts)]
    route = ora.routing(scores, rows, experts, top_k)
    x = [rng.gauss(0, 1) for _ in range(rows * width)]
    outputs = [(e, ora.route_gather(x, route, e, width)) for e in range(experts) if route["counts"][e]]
    for e, values in outputs:
        for i, row in enumerate(route["ids"][e]):
            assert values[i * width:(i + 1) * width] == x[row * width:(row + 1) * width]
    # identity experts: combine returns x scaled by the weight sum (= 1)
    y = ora.combine(outputs, route["weights"], route, width)
    assert y == pytest.approx(x, rel=1e-12, abs=1e-12)
    # a single unit weight reproduces the expert rows exactly
    one = dict(route, top_k=1, ids=[[0, 2]], slots=[[0, 0]], rows=3)
    assert ora.combine([(0, [1.0, 2.0, 3.0, 4.0])], [1.0, 0.0, 1.0], one, 2) == [1.0, 2.0, 0.0, 0.0, 3.0, 4.0]


# ---- attention ----------------------------------------------------------------------

def test_attention_hand_computed_golden():
    # tests/test_attention.py:10-22: identity projections of [[1,0],[0,1]],
    # non-causal, D = 2 -> rows [p, 1-p], [1-p, p] with p = e^(1/sqrt2)/(e^(1/sqrt2)+1)
    p = math.exp(1 / math.sqrt(2)) / (math.exp(1 / math.sqrt(2)) + 1)
    x = [1.0, 0.0, 0.0, 1.0]
    out, lse = ora.attention(x, x, x, 1, 2, 1, 1, 2, causal=False)
    assert out == pytest.approx([p, 1 - p, 1 - p, p], rel=1e-15)
    assert lse[0] == pytest.approx(math.log(math.exp(1 / math.sqrt(2)) + 1), rel=1e-15)
    # causal: the first query sees only itself
    out, lse = ora.attention(x, x, x, 1, 2, 1, 1, 2)
    assert out[:2] == [1.0, 0.0] and lse[0] == pytest.approx(1 / math.sqrt(2), rel=1e-15)


def test_attention_closed_forms_and_head_mapping():
    rng = random.Random(5)
    batch, time, heads, kv_heads, dim = 2, 5, 4, 2, 3
    q = [rng.gauss(0, 1) for _ in range(batch * time * heads * dim)]
    # K = 0: uniform weights over the visible keys -> prefix mean of V; lse = log(t + 1)
    k0 = [0.0] * (batch * time * kv_heads * dim)
    v = [rng.gauss(0, 1) for _ in range(batch * time * kv_heads * dim)]
    out, lse = ora.attention(q, k0, v, batch, time, heads, kv_heads, dim)
    for b in range(batch):
        for t in range(time):
            for h in range(heads):
                kh = h // 2
                for j in range(dim):
                    mean = sum(v[((b * time + s) * kv_heads + kh) * dim + j] for s in range(t + 1)) / (t + 1)
                    assert out[((b * time + t) * heads + h) * dim + j] == pytest.approx(mean, rel=1e-12, abs=1e-14)
                assert lse[(b * time + t) * heads + h] == pytest.approx(math.log(t + 1), rel=1e-14)
    # V constant per kv head: every output row equals its kv head's constant
    k = [rng.gauss(0, 1) for _ in range(len(k0))]
    vc = [float(10 * b + kh + 1) for b in range(batch) for _ in range(time) for kh in range(kv_heads)
          for _ in range(dim)]
    out, _ = ora.attention(q, k, vc, batch, time, heads, kv_heads, dim)
    for b in range(batch):
        for t in range(time):
            for h in range(heads):
                row = out[((b * time + t) * heads + h) * dim:((b * time + t) * heads + h + 1) * dim]
                assert row == pytest.approx([10 * b + h // 2 + 1] * dim, rel=1e-14)


def test_attention_numpy_form_agrees_with_the_loop():
    rng = np.random.default_rng(6)
    batch, time, heads, kv_heads, dim = 2, 7, 4, 2, 5
    q = rng.standard_normal((batch, time, heads, dim))
    k = rng.standard_normal((batch, time, kv_heads, dim))
    v = rng.standard_normal((batch, time, kv_heads, dim))
    for causal in (True, False):
        out, lse = ora.attention(q.ravel().tolist(), k.ravel().tolist(), v.ravel().tolist(), batch, time, heads,
                                 kv_heads, dim, causal=causal)
        out = np.array(out).reshape(q.shape)
        lse = np.array(lse).reshape(batch, time, heads)
        for b in range(batch):
            for h in range(heads):
                o, l = ora.attention_np(q[b, :, h], k[b, :, h // 2], v[b, :, h // 2], causal=causal)
                assert np.abs(o - out[b, :, h]).max() < 1e-12
                assert np.abs(l - lse[b, :, h]).max() < 1e-12


def test_attention_backward_matches_finite_differences_and_numpy_form():
    rng = np.random.default_rng(7)
    batch, time, heads, kv_heads, dim = 1, 4, 2, 1, 3
    q = rng.standard_normal(batch * time * heads * dim) * 0.5
    k = rng.standard_normal(batch * time * kv_heads * dim) * 0.5
    v = rng.standard_normal(batch * time * kv_heads * dim) * 0.5
    g = rng.standard_normal(q.size)
    dims = (batch, time, heads, kv_heads, dim)
    out, lse = ora.attention(q.tolist(), k.tolist(), v.tolist(), *dims)
    dq, dk, dv = ora.attention_backward(g.tolist(), q.tolist(), k.tolist(), v.tolist(), out, lse, *dims)

    def loss(qq, kk, vv):
        o, _ = ora.attention(qq.tolist(), kk.tolist(), vv.tolist(), *dims)
        return float(np.dot(o, g))

    eps = 1e-6
    for tensor, grad in ((q, dq), (k, dk), (v, dv)):
        for i in range(tensor.size):
            up, down = tensor.copy(), tensor.copy()
            up[i] += eps
            down[i] -= eps
            args = [q, k, v]
            index = [id(q), id(k), id(v)].index(id(tensor))
            args_up, args_down = list(args), list(args)
            args_up[index], args_down[index] = up, down
            numeric = (loss(*args_up) - loss(*args_down)) / (2 * eps)
            assert grad[i] == pytest.approx(numeric, rel=1e-5, abs=1e-8)
    # numpy form, GQA: heads 0 and 1 share kv head 0, so dk/dv sum over both
    qa, ga, oa = (np.array(x).reshape(time, heads, dim) for x in (q, g, out))
    la = np.array(lse).reshape(time, heads)
    ka, va = k.reshape(time, dim), v.reshape(time, dim)
    parts = [ora.attention_backward_np(ga[:, h], qa[:, h], ka, va, oa[:, h], la[:, h]) for h in range(heads)]
    assert np.abs(np.stack([p[0] for p in parts], 1).ravel() - dq).max() < 1e-12
    assert np.abs(sum(p[1] for p in parts).ravel() - dk).max() < 1e-12
    assert np.abs(sum(p[2] for p in parts).ravel() - dv).max() < 1e-12


def test_non_causal_numpy_attention_backward_matches_finite_differences():
    """attention_backward_np(causal=False) against central differences of
    attention_np(causal=False) (the nn attention form)."""
    rng = np.random.default_rng(8)
    time, dim = 5, 3
    q, k, v = (rng.standard_normal((time, dim)) * 0.7 for _ in range(3))
    g = rng.standard_normal((time, dim))
    out, lse = ora.attention_np(q, k, v, causal=False, scale=0.6)
    dq, dk, dv = ora.attention_backward_np(g, q, k, v, out, lse, scale=0.6, causal=False)
    eps = 1e-6
    for tensor, grad in ((q, dq), (k, dk), (v, dv)):
        for i in np.ndindex(tensor.shape):
            saved = tensor[i]
            tensor[i] = saved + eps
            up = float((ora.attention_np(q, k, v, causal=False, scale=0.6)[0] * g).sum())
            tensor[i] = saved - eps
            down = float((ora.attention_np(q, k, v, causal=False, scale=0.6)[0] * g).sum())
            tensor[i] = saved
            assert grad[i] == pytest.approx((up - down) / (2 * eps), rel=1e-6, abs=1e-9)


# ---- routing / combine backward ----------------------------------------------------

def _renormalised_weights(scores, route):
    """The routing weights as a function of the logits with the selection held
    fixed: w_s = exp(z_e) / sum over selected exp(z_f)."""
    rows, experts, top_k = route["rows"], route["experts"], route["top_k"]
    out = []
    for row in range(rows):
        sel = route["indices"][row * top_k:(row + 1) * top_k]
        z = [scores[row * experts + e] for e in sel]
        m = max(z)
        ex = [math.exp(v - m) for v in z]
        out.extend(v / math.fsum(ex) for v in ex)
    return out


def test_routing_backward_matches_finite_differences():
    rng = random.Random(12)
    rows, experts, top_k = 5, 4, 2
    scores = [rng.gauss(0, 1) for _ in range(rows * experts)]
    route = ora.routing(scores, rows, experts, top_k)
    g = [rng.gauss(0, 1) for _ in range(rows * top_k)]
    got = ora.routing_backward(g, route)
    eps = 1e-6
    for i in range(rows * experts):
        up, down = list(scores), list(scores)
        up[i] += eps
        down[i] -= eps
        f = lambda s: math.fsum(a * b for a, b in zip(g, _renormalised_weights(s, route)))  # noqa: E731
        assert got[i] == pytest.approx((f(up) - f(down)) / (2 * eps), abs=1e-8)
    # aux: d/dz of E * sum_e util_e * mean_r softmax(z_r)_e with util fixed
    c = [0.7]
    aux = ora.routing_backward(c, route, auxiliary=True)
    util = route["utilization"]

    def aux_of(s):
        total = 0.0
        for row in range(rows):
            z = s[row * experts:(row + 1) * experts]
            m = max(z)
            ex = [math.exp(v - m) for v in z]
            total += math.fsum(u * v / math.fsum(ex) for u, v in zip(util, ex))
        return c[0] * experts * total / rows

    for i in range(rows * experts):
        up, down = list(scores), list(scores)
        up[i] += eps
        down[i] -= eps
        assert aux[i] == pytest.approx((aux_of(up) - aux_of(down)) / (2 * eps), abs=1e-8)


def test_combine_backward_matches_finite_differences():
    rng = random.Random(13)
    rows, experts, top_k, width = 6, 3, 2, 4
    route = ora.routing([rng.gauss(0, 1) for _ in range(rows * experts)], rows, experts, top_k)
    outputs = [(e, [rng.gauss(0, 1) for _ in range(route["counts"][e] * width)]) for e in range(experts)
               if route["counts"][e]]
    weights = list(route["weights"])
    g = [rng.gauss(0, 1) for _ in range(rows * width)]
    *grads, dw = ora.combine_backward(g, outputs, weights, route, width)
    loss = lambda outs, w: math.fsum(a * b for a, b in zip(g, ora.combine(outs, w, route, width)))  # noqa: E731
    eps = 1e-6
    for i in range(len(weights)):
        up, down = list(weights), list(weights)
        up[i] += eps
        down[i] -= eps
        assert dw[i] == pytest.approx((loss(outputs, up) - loss(outputs, down)) / (2 * eps), abs=1e-8)
    for n, (e, values) in enumerate(outputs):
        for i in range(len(values)):
            up = [(f, list(v)) for f, v in outputs]
            down = [(f, list(v)) for f, v in outputs]
            up[n][1][i] += eps
            down[n][1][i] -= eps
            assert grads[n][i] == pytest.approx((loss(up, weights) - loss(down, weights)) / (2 * eps), abs=1e-8)


# ---- decoder glue ------------------------------------------------------------------

def _fd(f, x, i, eps=1e-6):
    up, down = list(x), list(x)
    up[i] += eps
    down[i] -= eps
    return (f(up) - f(down)) / (2 * eps)


def test_embedding_gather_and_scatter_round_trip():
    width, vocab = 3, 5
    weight = [float(i) for i in range(vocab * width)]
    ids = [4, 0, 4, 2]
    assert ora.embedding(weight, ids, width) == [12.0, 13.0, 14.0, 0.0, 1.0, 2.0, 12.0, 13.0, 14.0, 6.0, 7.0, 8.0]
    g = [1.0] * (len(ids) * width)
    grad = ora.embedding_backward(g, ids, vocab, width)
    # token 4 appears twice, 0 and 2 once, 1 and 3 never
    assert grad == [1.0] * 3 + [0.0] * 3 + [1.0] * 3 + [0.0] * 3 + [2.0] * 3


def test_rms_norm_closed_form_and_backward_finite_differences():
    # a constant row c: mean square c^2, out = c / sqrt(c^2 + eps) * w
    out, inv = ora.rms_norm([2.0] * 4, [1.0, 2.0, 3.0, 4.0], 4, 0.0)
    assert out == pytest.approx([1.0, 2.0, 3.0, 4.0], rel=1e-15) and inv == pytest.approx([0.5], rel=1e-15)
    rng = random.Random(14)
    width, rows, eps = 5, 3, 1e-5
    x = [rng.gauss(0, 1) for _ in range(rows * width)]
    w = [rng.gauss(1, 0.2) for _ in range(width)]
    g = [rng.gauss(0, 1) for _ in range(rows * width)]
    _, inv = ora.rms_norm(x, w, width, eps)
    dx, dw = ora.rms_norm_backward(g, x, w, inv, width)
    loss_x = lambda xx: math.fsum(a * b for a, b in zip(g, ora.rms_norm(xx, w, width, eps)[0]))  # noqa: E731
    loss_w = lambda ww: math.fsum(a * b for a, b in zip(g, ora.rms_norm(x, ww, width, eps)[0]))  # noqa: E731
    for i in range(len(x)):
        assert dx[i] == pytest.approx(_fd(loss_x, x, i), rel=1e-6, abs=1e-8)
    for j in range(width):
        assert dw[j] == pytest.approx(_fd(loss_w, w, j), rel=1e-6, abs=1e-8)


def test_silu_backward_finite_differences():
    xs = [-3.0, -0.5, 0.0, 0.7, 4.0]
    g = [1.0, -2.0, 0.5, 3.0, 1.5]
    d = ora.silu_backward(g, xs)
    for i, x in enumerate(xs):
        assert d[i] == pytest.approx(g[i] * _fd(lambda v: ora.silu(v)[i], xs, i), rel=1e-7)


def test_rope_inverse_norm_and_positions():
    rng = random.Random(15)
    batch, time, heads, dim, theta = 2, 3, 2, 6, 10000.0
    x = [rng.gauss(0, 1) for _ in range(batch * time * heads * dim)]
    y = ora.rope(x, batch, time, heads, dim, theta, offset=5)
    back = ora.rope(y, batch, time, heads, dim, theta, offset=5, inverse=True)
    assert back == pytest.approx(x, abs=1e-12)
    # each pair keeps its norm
    for i in range(0, len(x), 2):
        assert math.hypot(y[i], y[i + 1]) == pytest.approx(math.hypot(x[i], x[i + 1]), rel=1e-12)
    # position 0 (offset 0) is the identity; pair 0 of position t turns by t radians
    z = ora.rope(x, batch, time, heads, dim, theta)
    assert z[:heads * dim] == pytest.approx(x[:heads * dim], abs=1e-15)
    i = (1 * heads + 0) * dim  # b 0, t 1, h 0, pair 0
    assert z[i] == pytest.approx(x[i] * math.cos(1) - x[i + 1] * math.sin(1), rel=1e-12)


def test_head_rows_select_prediction_positions():
    width, time = 2, 4  # each sequence contributes its first time-1 rows
    values = [float(v) for v in range(2 * time * width)]  # 2 sequences
    rows = ora.head_rows(values, 0, 6, width, time)
    expected_rows = [0, 1, 2, 4, 5, 6]
    assert rows == [values[r * width + j] for r in expected_rows for j in range(width)]
    target = [0.0] * len(values)
    ora.head_rows_backward(target, [1.0] * 12, 0, 6, width, time)
    assert [target[r * width] for r in range(2 * time)] == [1, 1, 1, 0, 1, 1, 1, 0]


def test_head_loss_and_gradient_closed_forms():
    vocab = 4
    logits = [0.0] * vocab + [1.0, 2.0, 3.0, 4.0]
    labels = [2, -100]
    # uniform logits: log(V); the ignored row adds nothing
    assert ora.head_loss(logits, labels, 2, vocab) == pytest.approx(math.log(vocab), rel=1e-15)
    grad = ora.head_gradient(logits, labels, 2, vocab, [1.0], 1)
    assert grad[:vocab] == pytest.approx([0.25, 0.25, -0.75, 0.25], rel=1e-15)
    assert grad[vocab:] == [0, 0, 0, 0]
    # the gradient is the derivative of the loss
    rng = random.Random(16)
    z = [rng.gauss(0, 1) for _ in range(2 * vocab)]
    g = ora.head_gradient(z, [1, 3], 2, vocab, [1.0], 1)
    for i in range(len(z)):
        assert g[i] == pytest.approx(_fd(lambda v: ora.head_loss(v, [1, 3], 2, vocab), z, i), rel=1e-6, abs=1e-9)


# ---- generic tensor functions (broadcast, transpose, sums, element-wise) ---------------

def test_generic_ops_golden_vectors():
    # tests/test_operations.py:19-28 (broadcast arithmetic)
    assert ora.binary([1, 2, 3, 4, 5, 6], ora.broadcast([10, 20, 30], (3,), (2, 3)), "add") == [11, 22, 33, 14, 25,
                                                                                               36]
    assert ora.binary(ora.broadcast([1, 2], (2, 1), (2, 3)), ora.broadcast([10, 20, 30], (3,), (2, 3)),
                      "multiply") == [10, 20, 30, 20, 40, 60]
    assert ora.binary(ora.broadcast([10], (), (2,)), [1, 2], "subtract") == [9, 8]
    assert ora.binary([3, 8], [2, 4], "divide") == [1.5, 2]
    assert ora.binary([1, 2, 3, 4], ora.broadcast([10, 20], (2,), (2, 1, 2)), "add") == [11, 22, 13, 24]
    # tests/test_operations.py:30-33 (unary)
    assert ora.unary([1, -2], "negate") == [-1, 2]
    assert ora.unary([1, -2, 3, -4], "square") == [1, 4, 9, 16]
    assert ora.unary([-2, 0, 3], "relu") == [0, 0, 3]
    # tests/test_operations.py:35-40, 54-61 (transpose)
    assert ora.transpose([1, 2, 3, 4, 5, 6], (2, 3)) == [1, 4, 2, 5, 3, 6]
    assert ora.transpose(list(range(1, 13)), (2, 2, 3), (0, 2, 1)) == [1, 4, 2, 5, 3, 6, 7, 10, 8, 11, 9, 12]
    # tests/test_operations.py:63-73 (reductions), :75-79 (empty axes)
    data, shape = [1, 2, 3, 4, 5, 6], (2, 3)
    assert ora.reduce_sum(data) == [21]
    assert ora.reduce_sum(data, shape, 0) == [5, 7, 9]
    assert ora.reduce_sum(data, shape, -1) == [6, 15]
    assert ora.mean(data) == [3.5]
    assert ora.mean(data, shape, 0) == [2.5, 3.5, 4.5]
    assert ora.mean(data, shape, 1) == [2, 5]
    assert ora.reduce_sum([]) == [0]
    assert ora.reduce_sum([], (2, 0), 1) == [0, 0]
    assert ora.mean([], (2, 0), 0) == []
    with pytest.raises(ValueError):
        ora.mean([], (2, 0), 1)
    # tests/test_attention_cache.py:40-47 (append along the length axis)
    keys = ora.concatenate(([1, 2, 3, 4], [5, 6, 7, 8]), ((2, 2, 1, 1), (2, 2, 1, 1)), axis=2)
    assert keys == [1, 5, 2, 6, 3, 7, 4, 8]


def test_generic_ops_against_numpy_and_closed_forms():
    rng = np.random.default_rng(11)
    x = rng.standard_normal((3, 4, 5))
    flat = x.ravel().tolist()
    for axes in ((2, 0, 1), (1, 2, 0), (0, 2, 1), None):
        expected = np.transpose(x, axes).ravel()
        got = ora.transpose(flat, x.shape, axes)
        assert got == expected.tolist()
        # the inverse permutation restores the input
        order = tuple(reversed(range(3))) if axes is None else axes
        inverse = tuple(order.index(a) for a in range(3))
        assert ora.transpose(got, tuple(x.shape[a] for a in order), inverse) == flat
    for axis in (0, 1, 2, -1):
        np.testing.assert_allclose(ora.reduce_sum(flat, x.shape, axis), x.sum(axis=axis).ravel(), rtol=1e-13)
    np.testing.assert_allclose(ora.broadcast([1.0, 2.0, 3.0, 4.0], (4, 1), (2, 4, 3)),
                               np.broadcast_to(np.arange(1.0, 5.0).reshape(4, 1), (2, 4, 3)).ravel())
    # unbroadcast(broadcast(v)) = v times the number of copies
    source = rng.standard_normal((4, 1))
    wide = ora.broadcast(source.ravel().tolist(), (4, 1), (2, 4, 3))
    np.testing.assert_allclose(ora.unbroadcast(wide, (2, 4, 3), (4, 1)), 6 * source.ravel(), rtol=1e-13)
    # scatter adds repeated positions; gather(scatter) over distinct positions is the identity
    positions = [3, 0, 3, 1, 3]
    values = [1.0, 2.0, 4.0, 8.0, 16.0]
    expected = np.zeros(5)
    np.add.at(expected, positions, values)
    assert ora.scatter(values, positions, 5) == expected.tolist()
    assert ora.gather(ora.scatter([5.0, 6.0], [4, 1], 5), [4, 1]) == [5.0, 6.0]
    np.testing.assert_array_equal(ora.concatenate((flat[:20], flat[20:]), ((1, 4, 5), (2, 4, 5)), 0), flat)
    a, b = x[:, :1], x[:, 1:]
    np.testing.assert_array_equal(ora.concatenate((a.ravel().tolist(), b.ravel().tolist()), (a.shape, b.shape), 1),
                                  flat)
    # closed forms of the element-wise functions
    assert ora.unary([0.0], "gelu") == [0.0] and ora.unary([0.0], "gelu_backward", gradient=[1.0]) == [0.5]
    v = rng.standard_normal(7).tolist()
    np.testing.assert_allclose(ora.unary(ora.unary(v, "exp"), "log"), v, rtol=1e-13, atol=1e-15)
    np.testing.assert_allclose(ora.unary(v, "tanh_backward", gradient=[1.0] * 7), 1 - np.tanh(v) ** 2, rtol=1e-13)
    np.testing.assert_allclose(ora.unary(v, "atan_backward", gradient=[2.0] * 7), 2 / (1 + np.square(v)),
                               rtol=1e-13)
    np.testing.assert_allclose(ora.unary(v, "divide_scalar", factor=4.0), np.array(v) / 4, rtol=0)
    # gelu against its definition through the normal CDF: x * Phi(x)
    from statistics import NormalDist
    np.testing.assert_allclose(ora.unary(v, "gelu"), [t * NormalDist().cdf(t) for t in v], rtol=1e-12, atol=1e-15)
    # gelu' from central differences of gelu
    h = 1e-6
    numeric = (np.array(ora.unary([t + h for t in v], "gelu")) - np.array(ora.unary([t - h for t in v], "gelu"))) / (
        2 * h)
    np.testing.assert_allclose(ora.unary(v, "gelu_backward", gradient=[1.0] * 7), numeric, rtol=1e-7, atol=1e-9)
    # softmax over a middle axis against numpy
    s = np.array(ora.softmax(flat, x.shape, 1)).reshape(x.shape)
    e = np.exp(x - x.max(axis=1, keepdims=True))
    np.testing.assert_allclose(s, e / e.sum(axis=1, keepdims=True), rtol=1e-13)
