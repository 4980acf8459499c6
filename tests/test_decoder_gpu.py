"""Decoder glue kernels on the MI355X (the rest of a Decoder.loss step:
embedding, RMSNorm, SiLU, RoPE, the loss head's rows / cross entropy /
gradient, add_into, scale, concatenate) against the float64 oracle
restatements of cpu_lm (src/qutai/backends/cpu_lm.py:49-138, 323-371).
fp32 results within 1e-5 relative Frobenius error, bf16 results within
1e-2, gathers and scatters exact."""
from random import Random

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


@pytest.fixture(scope="module")
def base():
    from qutai_amd.backends import amd

    return amd


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
@pytest.mark.parametrize("width", [24, 27, 2048])  # 4 features per thread (24, 2048) or elementwise (27)
def test_embedding_forward_and_backward(lm, dtype, width):
    vocab = 37
    table = normal(110, vocab * width)
    ids = [Random(1).randrange(vocab) for _ in range(200)]
    out = lm.embedding(upload(table, "float32"), ids, width, out_dtype=dtype)
    expected = np.array(ora.embedding(stored(table, "float32").tolist(), ids, width))
    assert download(out).tobytes() == stored(expected, dtype).astype(np.float32).tobytes()
    g = normal(111, len(ids) * width)
    grad = lm.embedding_backward(upload(g, dtype), ids, vocab, width)
    assert grad.dtype == "float32"
    reference = ora.embedding_backward(stored(g, dtype).tolist(), ids, vocab, width)
    assert ora.rel_frobenius(download(grad), reference) <= FP32_TOL
    # the sums go in place into an existing table gradient: old + row sums
    start = normal(112, vocab * width)
    into = upload(start, "float32")
    assert lm.embedding_backward(upload(g, dtype), ids, vocab, width, out=into) is into
    assert np.array_equal(download(into), start + download(grad))
    with pytest.raises(ValueError):
        lm.embedding(upload(table, "bfloat16"), ids, width)  # bf16 table: not the accumulation dtype


@pytest.mark.parametrize("dtype,rows,width", [("float32", 37, 40), ("bfloat16", 300, 2048), ("float32", 4096, 2048),
                                               ("bfloat16", 65, 768), ("float32", 129, 256), ("float32", 70, 2304)])
def test_rms_norm_forward_and_backward(lm, base, dtype, rows, width):
    eps = 1e-5
    x = normal(112, rows * width, 2.0)
    w = (1 + 0.1 * normal(113, width)).astype(np.float32)
    g = normal(114, rows * width)
    out, inv = lm.rms_norm(upload(x, dtype), upload(w, "float32"), width, eps)
    assert (out.dtype, inv.dtype) == ("float32", "float32")
    sample = sorted({0, rows - 1, *Random(2).sample(range(rows), min(rows, 24))})
    xs = stored(x, dtype).reshape(rows, width)
    ws = w.astype(np.float64).tolist()
    sub_x = xs[sample].ravel().tolist()
    ref_out, ref_inv = ora.rms_norm(sub_x, ws, width, eps)
    assert ora.rel_frobenius(download(out).reshape(rows, width)[sample], np.array(ref_out).reshape(-1, width)) <= FP32_TOL
    assert ora.rel_frobenius(download(inv)[sample], ref_inv) <= FP32_TOL
    # the bf16 companion output: same fp32 results, and the copy is the cast
    # kernel's rounding of them bit for bit
    out2, inv2, copy = lm.rms_norm(upload(x, dtype), upload(w, "float32"), width, eps, bf16_copy=True)
    assert np.array_equal(download(out2), download(out)) and np.array_equal(download(inv2), download(inv))
    assert copy.dtype == "bfloat16"
    assert np.array_equal(np.frombuffer(copy.to_array(), np.uint16),
                          np.frombuffer(base.from_storage(out, dtype="bfloat16").to_array(), np.uint16))
    dx, dw = lm.rms_norm_backward(upload(g, "float32"), upload(x, dtype), upload(w, "float32"), inv, width)
    assert (dx.dtype, dw.dtype) == (dtype, "float32")
    gs = g.astype(np.float64).reshape(rows, width)
    inv_host = download(inv).astype(np.float64)
    ref_dx, _ = ora.rms_norm_backward(gs[sample].ravel().tolist(), sub_x, ws, inv_host[sample].tolist(), width)
    tol = FP32_TOL if dtype == "float32" else BF16_TOL
    assert ora.rel_frobenius(download(dx).reshape(rows, width)[sample], np.array(ref_dx).reshape(-1, width)) <= tol
    # dw over every row (numpy float64 of the same formula, fixed by the oracle's loop)
    ref_dw = (gs * xs * inv_host[:, None]).sum(axis=0)
    assert ora.rel_frobenius(download(dw), ref_dw) <= FP32_TOL
    _, ref_dw_loop = ora.rms_norm_backward(gs[:8].ravel().tolist(), xs[:8].ravel().tolist(), ws,
                                           inv_host[:8].tolist(), width)
    assert np.allclose((gs[:8] * xs[:8] * inv_host[:8, None]).sum(axis=0), ref_dw_loop, rtol=1e-12)


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_silu_forward_and_backward(lm, dtype):
    x, g = normal(115, 10007, 3.0), normal(116, 10007)
    out = download(lm.silu(upload(x, dtype)))
    xs, gs = stored(x, dtype), stored(g, dtype)
    tol = FP32_TOL if dtype == "float32" else BF16_TOL
    assert ora.rel_frobenius(out, ora.silu(xs.tolist())) <= tol
    d = download(lm.silu_backward(upload(g, dtype), upload(x, dtype)))
    assert ora.rel_frobenius(d, ora.silu_backward(gs.tolist(), xs.tolist())) <= tol


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_rope_forward_inverse_and_offset(lm, dtype):
    batch, time, heads, dim, theta = 2, 33, 4, 16, 10000.0
    x = normal(117, batch * time * heads * dim)
    y = lm.rope(upload(x, dtype), batch, time, heads, dim, theta, offset=7)
    ref = ora.rope(stored(x, dtype).tolist(), batch, time, heads, dim, theta, offset=7)
    tol = FP32_TOL if dtype == "float32" else BF16_TOL
    assert ora.rel_frobenius(download(y), ref) <= tol
    back = lm.rope(y, batch, time, heads, dim, theta, offset=7, inverse=True)
    assert ora.rel_frobenius(download(back), stored(x, dtype)) <= (1e-5 if dtype == "float32" else 2e-2)
    # the kernel that shares one angle per (position, pair) over the heads
    # gives each head exactly what the one-head kernel gives it
    got = np.frombuffer(y.to_array(), dtype=np.uint16 if dtype == "bfloat16" else np.float32)
    got = got.reshape(batch, time, heads, dim)
    for h in range(heads):
        single = lm.rope(upload(x.reshape(batch, time, heads, dim)[:, :, h].copy(), dtype), batch, time, 1, dim, theta,
                         offset=7)
        want = np.frombuffer(single.to_array(), dtype=got.dtype).reshape(batch, time, dim)
        assert np.array_equal(got[:, :, h], want)


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
@pytest.mark.parametrize("width", [8, 13, 2048])  # 16-byte chunks per row (8, 2048) or elementwise (13)
def test_head_rows_and_backward(lm, dtype, width):
    batch, time = 3, 6
    h = normal(118, batch * time * width)
    rows = batch * (time - 1)
    got = download(lm.head_rows(upload(h, dtype), 4, 9, width, time))
    assert got.tobytes() == stored(np.array(ora.head_rows(stored(h, dtype).tolist(), 4, 9, width, time)),
                                   dtype).astype(np.float32).tobytes()
    g = normal(119, 9 * width)
    start = normal(117, batch * time * width)
    target = upload(start, dtype)
    lm.head_rows_backward(target, upload(g, dtype), 4, 9, width, time)
    added = [0.0] * (batch * time * width)
    ora.head_rows_backward(added, stored(g, dtype).tolist(), 4, 9, width, time)
    # one fp32 addition per element (zero where no row lands), then the storage rounding
    sums = stored(start, dtype).astype(np.float32) + np.array(added, dtype=np.float32)
    assert np.array_equal(download(target), stored(sums, dtype))
    assert rows == 15


@pytest.mark.parametrize("dtype,rows,vocab", [("float32", 7, 13), ("bfloat16", 40, 32000), ("float32", 512, 32000)])
def test_head_loss_and_gradient(lm, dtype, rows, vocab):
    logits = normal(120, rows * vocab, 2.0)
    rng = Random(3)
    labels = [rng.randrange(vocab) for _ in range(rows + 2)]
    labels[1] = -100  # ignored position
    prepared = lm.prepare_labels(labels)
    start = 2
    loss = lm.head_loss(upload(logits, dtype), prepared, rows, vocab, start=start)
    ls = stored(logits, dtype)
    expected = ora.head_loss(ls.tolist(), labels, rows, vocab, start=start)
    assert abs(download(loss)[0] - expected) <= 1e-5 * max(1.0, abs(expected)) * (1 if dtype == "float32" else 10)
    g = upload(np.array([0.75], dtype=np.float32), "float32")
    grad = lm.head_gradient(upload(logits, dtype), prepared, rows, vocab, g, 5, start=start)
    ref = ora.head_gradient(ls.tolist(), labels, rows, vocab, [0.75], 5, start=start)
    assert ora.rel_frobenius(download(grad), ref) <= (FP32_TOL if dtype == "float32" else BF16_TOL)
    with pytest.raises(ValueError):
        lm.head_loss(upload(logits, dtype), prepared, rows, vocab, start=len(labels))  # label range


@pytest.mark.parametrize("dtype,rows,vocab,block", [("float32", 7, 13, 5), ("float32", 33, 1000, 256),
                                                     ("bfloat16", 40, 32000, 8192), ("bfloat16", 64, 3000, 3000)])
def test_head_vocab_blocks_match_row_head(lm, base, dtype, rows, vocab, block):
    """The vocabulary-blocked head (stats folded over column blocks, ragged
    last block, labels in every block and -100 rows) gives the row head's
    loss and gradient (cuda_lm.py:629-660 restated by the oracle)."""
    logits = normal(121, rows * vocab, 2.0).reshape(rows, vocab)
    rng = Random(5)
    labels = [rng.randrange(vocab) for _ in range(rows)]
    labels[1] = -100
    labels[2] = vocab - 1  # in the last (ragged) block
    prepared = lm.prepare_labels(labels)
    stats = base.AMDStorage(2 * rows, "float32")
    picked = base.AMDStorage(rows, "float32")
    blocks = [(c0, min(block, vocab - c0)) for c0 in range(0, vocab, block)]
    for c0, cols in blocks:
        lm.head_block_stats(upload(logits[:, c0:c0 + cols], dtype), prepared, stats, picked, rows, cols, c0,
                            first=c0 == 0)
    loss = download(lm.head_block_loss(stats, picked, prepared, rows))[0]
    ls = stored(logits, dtype)
    expected = ora.head_loss(ls.ravel().tolist(), labels, rows, vocab)
    assert abs(loss - expected) <= 1e-5 * max(1.0, abs(expected)) * (1 if dtype == "float32" else 10)
    g = upload(np.array([0.75], dtype=np.float32), "float32")
    grad = np.concatenate([download(lm.head_block_gradient(upload(logits[:, c0:c0 + cols], dtype), prepared, stats,
                                                           g, rows, cols, c0, 5)).reshape(rows, cols)
                           for c0, cols in blocks], axis=1)
    ref = np.array(ora.head_gradient(ls.ravel().tolist(), labels, rows, vocab, [0.75], 5)).reshape(rows, vocab)
    assert ora.rel_frobenius(grad, ref) <= (FP32_TOL if dtype == "float32" else BF16_TOL)
    assert not grad[1].any()  # ignored row


def test_vocab_block_bound(lm):
    from qutai_amd.lm.layers import vocab_block

    assert vocab_block(1024, 4096, 32768) == 8192          # 4 blocks of 1024 x 32768 logits
    assert vocab_block(128, 4096, 32768) == 1024
    assert vocab_block(5000, 4096, 32768) == 32768         # all rows fit: one block
    assert vocab_block(1, 4096, 1000) == 8                 # floor of 8 columns
    for chunk, rows, vocab in ((3, 10, 13), (16, 200, 511), (100, 4096, 32000)):
        b = vocab_block(chunk, rows, vocab)
        assert b % 8 == 0 or b == vocab
        assert rows * b <= max(chunk * vocab, rows * 8)


def test_add_into_scale_concatenate(lm, base):
    a, b = normal(121, 1000), normal(122, 1000)
    t = upload(a, "float32")
    lm.add_into(t, upload(b, "float32"))
    assert np.array_equal(download(t), (a + b).astype(np.float32))
    assert np.array_equal(download(base.scale(upload(a, "float32"), 0.25)), (a * np.float32(0.25)).astype(np.float32))
    x = upload(np.arange(6, dtype=np.float32), "float32")
    y = upload(np.arange(10, 13, dtype=np.float32), "float32")
    assert download(base.concatenate((x, y), ((6,), (3,)))).tolist() == [0, 1, 2, 3, 4, 5, 10, 11, 12]
    m = base.concatenate((x, y), ((3, 2), (3, 1)), axis=1)
    assert download(m).tolist() == [0, 1, 10, 2, 3, 11, 4, 5, 12]


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_repitch_pads_and_crops_exactly(lm, dtype):
    x = normal(123, (3, 5, 6))
    padded = lm.repitch(upload(x, dtype), 3, 5, 6, 7, 8)
    expected = np.zeros((3, 7, 8))
    expected[:, :5, :6] = stored(x, dtype)
    assert np.array_equal(download(padded).reshape(3, 7, 8), expected)
    back = lm.repitch(padded, 3, 7, 8, 5, 6)
    assert np.array_equal(download(back).reshape(3, 5, 6), stored(x, dtype))
    with pytest.raises(ValueError):
        lm.repitch(padded, 3, 5, 6, 5, 6)  # size does not match the stated shape


def test_residual_add_widened_equals_cast_then_add(base):
    """residual_add (lm/layers.py:31-32) of fp32 x and a bf16 update: the
    one-pass form equals x + update.to(float32) bit for bit, forward and both
    gradients (ragged length: vector body and scalar tail)."""
    from qutai_amd import Tensor
    from qutai_amd.lm.layers import residual_add

    n = 4 * 1000 + 3
    x = Tensor(upload(normal(31, n), "float32"), shape=(n,), requires_grad=True)
    u = Tensor(upload(normal(32, n), "bfloat16"), shape=(n,), requires_grad=True)
    g = Tensor(upload(normal(33, n), "float32"), shape=(n,))
    results = []
    for fused in (True, False):
        x.grad = u.grad = None
        y = residual_add(x, u) if fused else x + u.to(dtype="float32")
        y.backward(g)
        results.append([t.storage.to_array() for t in (y, x.grad, u.grad)])
    assert results[0] == results[1]



@pytest.mark.parametrize("leaf", [True, False])
def test_linear_input_gradients_sum_in_the_gemm(base, leaf):
    """Two Linears of one fp32 activation under autocast (the k and v
    projections): the second dX = G W is added by the GEMM's accumulate
    epilogue into the first, for a leaf input (tensor.py) and for a
    non-leaf one (the backward loop's fresh gradients).  Bit-exact against
    the two products from separate GEMMs added in fp32 on the host (a + b
    equals b + a, so the order the pass meets them in does not matter)."""
    from qutai_amd import Tensor
    from qutai_amd.backends.precision import set_matmul_precision
    from qutai_amd.lm.layers import linear, scaled

    rows, inner, out_features = 300, 256, 200
    x0 = Tensor(upload(normal(41, rows * inner), "float32"), shape=(rows, inner), requires_grad=True)
    w1, w2 = (Tensor(upload(normal(seed, out_features * inner, 0.05), "float32"), shape=(out_features, inner),
                     requires_grad=True) for seed in (42, 43))
    g = upload(normal(44, rows * out_features), "bfloat16")
    with set_matmul_precision("bfloat16"):
        x = x0 if leaf else scaled(x0, 2.0)
        y = linear(x, w1) + linear(x, w2)
        y.backward(Tensor(g, shape=y.shape))
        a, b = (download(base.gemm(g, base.from_storage(w.storage, dtype="bfloat16"), rows, out_features, inner,
                                   out_dtype="float32")).astype(np.float32) for w in (w1, w2))
    want = (a + b) * np.float32(1.0 if leaf else 2.0)
    assert np.array_equal(download(x0.grad.storage).astype(np.float32), want)


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_rope_and_copy_on_column_slices(lm, dtype):
    """RoPE reading the q / k columns of a stacked [positions][dq + 2 dkv]
    matrix and writing into such columns gives the bits of RoPE on the
    contiguous slice, leaving the other columns alone; copy_rows moves a
    column slice exactly.  Column ranges outside the rows are rejected."""
    batch, time, dq, dkv, theta = 2, 19, 256, 128, 10000.0
    total, positions = dq + 2 * dkv, batch * time
    words = np.uint16 if dtype == "bfloat16" else np.float32
    x = normal(131, positions * total).reshape(positions, total)
    stacked = upload(x, dtype)
    host = np.frombuffer(stacked.to_array(), dtype=words).reshape(positions, total)
    for column, width, heads in ((0, dq, 4), (dq, dkv, 2)):
        got = lm.rope(stacked, batch, time, heads, 64, theta, column=column, row=total)
        want = lm.rope(upload(x[:, column:column + width].copy(), dtype), batch, time, heads, 64, theta)
        assert np.array_equal(np.frombuffer(got.to_array(), dtype=words), np.frombuffer(want.to_array(), dtype=words))
        # the inverse written back into the same columns of another stacked block
        target = upload(np.zeros((positions, total)), dtype)
        lm.rope(got, batch, time, heads, 64, theta, inverse=True, out=target, out_column=column, out_row=total)
        back = np.frombuffer(target.to_array(), dtype=words).reshape(positions, total)
        plain = lm.rope(want, batch, time, heads, 64, theta, inverse=True)
        assert np.array_equal(back[:, column:column + width],
                              np.frombuffer(plain.to_array(), dtype=words).reshape(positions, width))
        assert not back[:, :column].any() and not back[:, column + width:].any()
    v = lm.copy_rows(stacked, positions, dkv, column=dq + dkv, row=total)
    assert np.array_equal(np.frombuffer(v.to_array(), dtype=words).reshape(positions, dkv), host[:, dq + dkv:])
    target = upload(np.zeros((positions, total)), dtype)
    lm.copy_rows(v, positions, dkv, out=target, out_column=dq, out_row=total)
    back = np.frombuffer(target.to_array(), dtype=words).reshape(positions, total)
    assert np.array_equal(back[:, dq:dq + dkv], host[:, dq + dkv:]) and not back[:, :dq].any()
    # odd widths and pitches take the element path
    odd = lm.copy_rows(stacked, positions, 37, column=3, row=total)
    assert np.array_equal(np.frombuffer(odd.to_array(), dtype=words).reshape(positions, 37), host[:, 3:40])
    with pytest.raises(ValueError):
        lm.rope(stacked, batch, time, heads, 64, theta, column=total - 64, row=total)
    with pytest.raises(ValueError):
        lm.copy_rows(stacked, positions, dkv, column=total - dkv + 1, row=total)


@pytest.mark.parametrize("x_dtype", ["float32", "bfloat16"])
def test_stacked_qkv_attention_matches_separate_projections(base, x_dtype):
    """GQA's q/k/v projections as one GEMM on the stacked weight (bf16 path,
    fp32 master weights under autocast): the attention output is bit-identical
    to the separate projections + RoPE + attention, the weight gradients are
    bit-identical (each is its own row block of one product summed over the
    same rows in the same order), and the input gradient, which sums its three
    terms in one accumulator instead of two rounded additions, agrees to fp32
    rounding."""
    from qutai_amd import Tensor
    from qutai_amd.backends.precision import set_matmul_precision
    from qutai_amd.lm.layers import attention, gqa_attention, linear, rope

    batch, time, heads, kv_heads, width, theta = 2, 128, 4, 2, 192, 10000.0
    dq, dkv = heads * 64, kv_heads * 64
    x = Tensor(upload(normal(71, batch * time * width), x_dtype), shape=(batch, time, width), requires_grad=True)
    ws = [Tensor(upload(normal(72 + i, rows * width, 0.05), "float32"), shape=(rows, width), requires_grad=True)
          for i, rows in enumerate((dq, dkv, dkv))]
    g = Tensor(upload(normal(75, batch * time * dq), "bfloat16"), shape=(batch, time, dq))
    results = []
    with set_matmul_precision("bfloat16"):
        for fused in (True, False):
            for t in (x, *ws):
                t.grad = None
            if fused:
                y = gqa_attention(x, *ws, heads, kv_heads, theta)
            else:
                q = rope(linear(x, ws[0]), heads, theta)
                k = rope(linear(x, ws[1]), kv_heads, theta)
                y = attention(q, k, linear(x, ws[2]), heads, kv_heads)
            y.backward(g)
            words = np.uint16 if x_dtype == "bfloat16" else np.float32
            results.append((np.frombuffer(y.storage.to_array(), dtype=np.uint16).copy(),
                            [download(w.grad.storage) for w in ws],
                            np.frombuffer(x.grad.storage.to_array(), dtype=words).copy()))
    (y1, dw1, dx1), (y2, dw2, dx2) = results
    assert np.array_equal(y1, y2)
    for a, b in zip(dw1, dw2):
        assert np.array_equal(a, b)
    if x_dtype == "float32":
        assert ora.rel_frobenius(dx1.astype(np.float64), dx2.astype(np.float64)) <= 1e-6
    else:
        assert ora.rel_frobenius(ora.bf16_values(dx1), ora.bf16_values(dx2)) <= 1e-2


@pytest.mark.parametrize("rows,width", [(300, 2048), (37, 100)])
def test_rms_norm_backward_adds_the_residual(lm, rows, width):
    """dx = residual + dx as the kernel stores it (the 16-byte column path at
    width 2048, the generic path at 100): bit-exact against the plain dx
    added to the residual in fp32 on the host; dweight unchanged."""
    x, w = normal(51, rows * width), normal(52, width, 0.5) + 1.0
    g, res = normal(53, rows * width), normal(54, rows * width)
    xs, ws = upload(x, "float32"), upload(w, "float32")
    _, inv = lm.rms_norm(xs, ws, width, 1e-5)
    dx, dw = lm.rms_norm_backward(upload(g, "float32"), xs, ws, inv, width)
    rx, rw = lm.rms_norm_backward(upload(g, "float32"), xs, ws, inv, width, residual=upload(res, "float32"))
    assert np.array_equal(download(rx).astype(np.float32), res + download(dx).astype(np.float32))
    assert np.array_equal(download(rw), download(dw))


@pytest.mark.parametrize("leaf", [True, False])
def test_norm_input_gradient_sums_with_the_residual(base, leaf):
    """y = x + rms_norm(x): the backward pass sums the add's gradient G and
    the norm's dx inside the norm kernel (non-leaf x) or adds dx into the
    leaf's gradient; bit-exact against dx + G in fp32 on the host."""
    from qutai_amd import Tensor
    from qutai_amd.backends import amd_lm
    from qutai_amd.lm.layers import rms_norm, scaled

    rows, width = 64, 2048
    x0 = Tensor(upload(normal(61, rows * width), "float32"), shape=(rows, width), requires_grad=True)
    w = Tensor(upload(normal(62, width, 0.5) + 1.0, "float32"), shape=(width,), requires_grad=True)
    g = normal(63, rows * width)
    x = x0 if leaf else scaled(x0, 2.0)
    y = x + rms_norm(x, w, 1e-5)
    y.backward(Tensor(upload(g, "float32"), shape=y.shape))
    _, inv = amd_lm.rms_norm(x.storage, w.storage, width, 1e-5)
    dx, dw = amd_lm.rms_norm_backward(upload(g, "float32"), x.storage, w.storage, inv, width)
    want = (g + download(dx).astype(np.float32)) * np.float32(1.0 if leaf else 2.0)
    assert np.array_equal(download(x0.grad.storage).astype(np.float32), want)
    assert np.array_equal(download(w.grad.storage), download(dw))


def test_head_kept_logits_equal_recomputed():
    """projection_loss keeps the forward's logit blocks for the backward
    (keep_logits=True): loss and both gradients bit-identical to the
    recomputing form, and a second backward over the retained graph (the
    kept blocks were overwritten by the first) adds the same gradients."""
    from qutai_amd import Tensor
    from qutai_amd.backends.precision import set_matmul_precision
    from qutai_amd.lm import layers

    batch, time, width, vocab = 2, 48, 256, 3000
    labels = [[(7 * t + 3 * r) % vocab for t in range(time)] for r in range(batch)]
    labels[0][5] = -100
    results = []
    for keep in (True, False):
        h = Tensor(upload(normal(71, batch * time * width), "float32"), shape=(batch, time, width),
                   requires_grad=True)
        w = Tensor(upload(normal(72, vocab * width, 0.05), "float32"), shape=(vocab, width), requires_grad=True)
        with set_matmul_precision("bfloat16"):
            loss = layers.projection_loss(h, w, labels, chunk_size=16, keep_logits=keep)
            loss.backward()
            first = [download(t.grad.storage).copy() for t in (h, w)]
            loss.backward()
        second = [download(t.grad.storage) for t in (h, w)]
        results.append((download(loss.storage), first))
        for a, b2 in zip(first, second):
            assert np.array_equal((a.astype(np.float32) * 2), b2.astype(np.float32))
    assert np.array_equal(results[0][0], results[1][0])
    for a, b2 in zip(results[0][1], results[1][1]):
        assert np.array_equal(a, b2)


def test_head_small_chunk_bounds_forward_memory():
    """The caller's chunk_size still bounds the loss head's memory: with 2048
    prediction rows and chunk 64 the logits are not kept (32 MB of fp32
    logits in all), and the forward's peak stays near one 1 MB block; asking
    for keep_logits=True holds all of them until the backward."""
    from qutai_amd import Tensor
    from qutai_amd.backends import amd
    from qutai_amd.lm import layers

    batch, time, width, vocab = 2, 1025, 64, 4096
    labels = [[(5 * t + r) % vocab for t in range(time)] for r in range(batch)]
    h = Tensor(upload(normal(81, batch * time * width), "float32"), shape=(batch, time, width), requires_grad=True)
    w = Tensor(upload(normal(82, vocab * width, 0.05), "float32"), shape=(vocab, width), requires_grad=True)
    full = batch * (time - 1) * vocab * 4
    growth = {}
    for keep in (None, True):
        amd.synchronize()
        base = amd.memory_stats()["allocated_bytes"]
        amd.reset_peak_memory_stats()
        loss = layers.projection_loss(h, w, labels, chunk_size=64, keep_logits=keep)
        amd.synchronize()
        growth[keep] = amd.memory_stats()["peak_allocated_bytes"] - base
        del loss
    assert growth[None] < full // 4, growth
    assert growth[True] >= full, growth
