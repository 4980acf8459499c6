"""Generic tensor functions of the amd backend (broadcast, any transpose,
element-wise arithmetic, sums over any axis, softmax over any axis,
concatenation, gather/scatter, slices) on the MI355X, against the float64
oracle restatements of the reference CPU backend and the reference tests'
known answers; plus the reference's broadcasting Tensor semantics and
KV-cache attention inference."""
import math

import numpy as np
import pytest

from oracle import reference as ora
from tests.helpers import download, normal, stored, upload

pytestmark = pytest.mark.gpu

TOL = {"float32": 1e-6, "float64": 1e-13, "bfloat16": 8e-3}  # relative, per element


@pytest.fixture(scope="module")
def amd():
    from qutai_amd.backends import amd as backend

    backend.get_runtime()
    return backend


def close(got, expected, dtype, scale=None):
    got, expected = np.asarray(got, np.float64), np.asarray(expected, np.float64)
    assert got.shape == expected.shape
    bound = TOL[dtype] * (np.abs(expected) + (scale if scale is not None else 1e-30))
    assert np.all(np.abs(got - expected) <= bound), np.max(np.abs(got - expected) - bound)


# ---- reference known answers through the Tensor front-end ---------------------------------

def test_operations_golden_vectors(amd):
    import qutai_amd as qt
    from qutai_amd import Tensor

    def t(data):
        return Tensor(data, device="amd", dtype="float32")

    # tests/test_operations.py:19-28
    assert qt.add(t([[1, 2, 3], [4, 5, 6]]), t([10, 20, 30])).tolist() == [[11, 22, 33], [14, 25, 36]]
    assert qt.multiply(t([[1], [2]]), t([10, 20, 30])).tolist() == [[10, 20, 30], [20, 40, 60]]
    assert qt.subtract(t(10), t([1, 2])).tolist() == [9, 8]
    assert qt.divide(t([3, 8]), t([2, 4])).tolist() == [1.5, 2]
    assert qt.add(t([[[1, 2]], [[3, 4]]]), t([10, 20])).tolist() == [[[11, 22]], [[13, 24]]]
    with pytest.raises(ValueError):
        qt.add(t([[1, 2, 3]]), t([1, 2]))
    # :30-33
    assert (-t([1, -2])).tolist() == [-1, 2]
    assert t([[1, -2], [3, -4]]).square().tolist() == [[1, 4], [9, 16]]
    assert qt.relu(t([-2, 0, 3])).tolist() == [0, 0, 3]
    # :35-61
    data = t([[1, 2, 3], [4, 5, 6]])
    assert data.transpose().tolist() == [[1, 4], [2, 5], [3, 6]]
    assert data.transpose().transpose().tolist() == data.tolist()
    assert data.reshape((-1, 2)).tolist() == [[1, 2], [3, 4], [5, 6]]
    cube = t([[[1, 2, 3], [4, 5, 6]], [[7, 8, 9], [10, 11, 12]]])
    assert cube.transpose((0, 2, 1)).tolist() == [[[1, 4], [2, 5], [3, 6]], [[7, 10], [8, 11], [9, 12]]]
    assert cube.transpose().shape == (3, 2, 2)
    with pytest.raises(ValueError):
        data.transpose((0, 0))
    # :63-73
    assert qt.sum(data).item() == 21
    assert qt.sum(data, axis=0).tolist() == [5, 7, 9]
    assert qt.sum(data, axis=-1, keepdims=True).tolist() == [[6], [15]]
    assert qt.mean(data).item() == 3.5
    assert qt.mean(data, axis=0).tolist() == [2.5, 3.5, 4.5]
    assert qt.mean(data, axis=1, keepdims=True).tolist() == [[2], [5]]
    assert qt.sum(data, keepdims=True).tolist() == [[21]]
    with pytest.raises(ValueError):
        qt.sum(data, axis=2)
    # :75-85 (empty axes)
    empty_rows = Tensor(amd.full(0, dtype="float32"), shape=(2, 0))
    assert qt.sum(empty_rows, axis=1, keepdims=True).tolist() == [[0], [0]]
    assert qt.mean(empty_rows, axis=0).tolist() == []
    with pytest.raises(ValueError):
        qt.mean(empty_rows, axis=1)
    assert qt.sum(Tensor(amd.full(0, dtype="float32"), shape=(0,))).item() == 0
    # :87-95 (a plain number joins the Tensor's device and dtype)
    grid = t([[1, 2], [3, 4]])
    assert (grid + 1).tolist() == [[2, 3], [4, 5]]
    assert (grid / 2).tolist() == [[0.5, 1], [1.5, 2]]
    assert (2 * grid - grid).tolist() == grid.tolist()


def test_division_by_zero_raises(amd):
    left = upload(np.ones(40), "float32")
    right = upload(np.r_[np.ones(39), 0.0], "float32")
    with pytest.raises(ZeroDivisionError):
        amd.divide(left, right)
    with pytest.raises(ZeroDivisionError):
        amd.divide_scalar(left, 0.0)
    assert download(amd.divide(left, amd.full(40, 2.0, dtype="float32"))).tolist() == [0.5] * 40
    with pytest.raises(ValueError):
        amd.log(upload(np.r_[np.ones(9), -1.0], "float32"))


# ---- backend functions against the oracle -------------------------------------------------

@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float64"])
@pytest.mark.parametrize("shape,target", [((3,), (4, 5, 3)), ((4, 1, 3), (4, 5, 3)), ((1,), (37,)), ((), (2, 3)),
                                          ((5, 1), (5, 16)), ((2, 1, 8), (2, 9, 8)), ((1, 64), (33, 64))])
def test_broadcast(amd, dtype, shape, target):
    x = normal(1, shape if shape else ())
    got = download(amd.broadcast(upload(np.atleast_1d(x), dtype), shape, target))
    expected = ora.broadcast(stored(np.atleast_1d(x), dtype).ravel().tolist(), shape, target)
    assert got.tolist() == expected  # a copy: bit-exact


@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float64"])
@pytest.mark.parametrize("shape,axes", [((3, 4, 5), (2, 0, 1)), ((2, 3, 4, 8), (0, 2, 1, 3)), ((6, 7), None),
                                        ((4, 9, 33), (0, 2, 1)), ((2, 3, 4, 5), (3, 2, 1, 0)),
                                        ((8, 16, 64, 64), (0, 2, 1, 3)), ((5,), None), ((2, 1, 3), (1, 2, 0))])
def test_transpose(amd, dtype, shape, axes):
    x = normal(2, shape)
    got = download(amd.transpose(upload(x, dtype), shape, axes))
    assert got.tolist() == np.transpose(stored(x, dtype), axes).ravel().tolist()
    if x.size <= 4096:
        assert got.tolist() == ora.transpose(stored(x, dtype).ravel().tolist(), shape, axes)


@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float64"])
@pytest.mark.parametrize("operation", ["add", "subtract", "multiply", "divide"])
@pytest.mark.parametrize("size", [1, 7, 64, 1003])
def test_binary(amd, dtype, operation, size):
    a = normal(3, size)
    b = normal(4, size) + np.float32(3.0)
    got = download(getattr(amd, operation)(upload(a, dtype), upload(b, dtype)))
    expected = ora.binary(stored(a, dtype).tolist(), stored(b, dtype).tolist(), operation)
    # one rounding of the exact result to the storage type
    close(got, stored(np.asarray(expected), dtype) if dtype != "float64" else expected, dtype)


UNARY = ["negate", "square", "relu", "gelu", "exp", "log", "tanh", "atan", "relu_backward", "gelu_backward",
         "tanh_backward", "atan_backward"]


@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float64"])
@pytest.mark.parametrize("operation", UNARY)
def test_unary(amd, dtype, operation):
    x = normal(5, 1003, 2.0)
    if operation == "log":
        x = np.abs(x) + np.float32(0.1)
    g = normal(6, 1003)
    values, grads = upload(x, dtype), upload(g, dtype)
    if operation.endswith("_backward"):
        got = download(getattr(amd, operation)(grads, values))
        expected = ora.unary(stored(x, dtype).tolist(), operation, gradient=stored(g, dtype).tolist())
    else:
        got = download(getattr(amd, operation)(values))
        expected = ora.unary(stored(x, dtype).tolist(), operation)
    expected = np.asarray(expected)
    # math-library functions: a few ulps of the result, plus the fp32
    # cancellation of 1 + erf(x / sqrt 2) in gelu, which scales with |x| |g|
    rtol, atol = {"float32": (4e-6, 1e-6), "float64": (1e-13, 1e-14), "bfloat16": (8e-3, 1e-5)}[dtype]
    scale = (1 + np.abs(stored(x, dtype))) * (1 + np.abs(stored(g, dtype)))
    assert np.all(np.abs(got - expected) <= rtol * np.abs(expected) + atol * scale)


@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float64"])
def test_scalar_scale_and_divide(amd, dtype):
    x = normal(7, 517)
    got = download(amd.divide_scalar(upload(x, dtype), 8.0))
    close(got, stored(stored(x, dtype) / 8.0, dtype), dtype)
    got = download(amd.scale(upload(x, dtype), 0.25))
    close(got, stored(stored(x, dtype) * 0.25, dtype), dtype)
    target = upload(x, dtype)
    amd.scale_into(target, 2.0)
    amd.add_into(target, upload(x, dtype))
    close(download(target), stored(3 * stored(x, dtype), dtype), dtype)


@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float64"])
@pytest.mark.parametrize("shape,axis", [((3, 4, 5), 0), ((3, 4, 5), 1), ((3, 4, 5), 2), ((3, 4, 5), None),
                                        ((7, 300), 1), ((300, 7), 0), ((2, 0, 3), 1), ((0, 4), 0)])
def test_sum_small(amd, dtype, shape, axis):
    x = normal(8, shape)
    got = download(amd.sum(upload(x, dtype), shape, axis))
    values = stored(x, dtype)
    expected = np.asarray(ora.reduce_sum(values.ravel().tolist(), shape, axis))
    width = x.size if axis is None else shape[axis]
    accumulate = 1.2e-16 if dtype == "float64" else 6e-8  # bf16 accumulates in fp32
    rounding = {"float32": 6e-8, "float64": 1.2e-16, "bfloat16": 3.9e-3}[dtype]
    magnitude = np.abs(values).sum(axis=axis).ravel() if x.size else np.zeros_like(expected)
    assert np.all(np.abs(got - expected) <= width * accumulate * magnitude + rounding * np.abs(expected))


@pytest.mark.parametrize("dtype", ["float32", "float64"])
@pytest.mark.parametrize("shape,axis", [((1 << 22,), None), ((3, 1 << 20), 1), ((1 << 16, 48), 0),
                                        ((4, 100000, 3), 1), ((4096, 2048), 0), ((4096, 2048), 1)])
def test_sum_large(amd, dtype, shape, axis):
    """The split reductions (partial sums in the workspace) against numpy
    float64, within the fp32 error bound n * eps * sum |x|."""
    x = normal(9, shape)
    got = download(amd.sum(upload(x, dtype), shape, axis))
    exact = x.astype(np.float64).sum(axis=axis).ravel()
    width = x.size if axis is None else shape[axis]
    bound = (width * (6e-8 if dtype == "float32" else 1.2e-16)) * np.abs(x.astype(np.float64)).sum(axis=axis).ravel()
    assert np.all(np.abs(got - exact) <= bound + 1e-30)
    again = download(amd.sum(upload(x, dtype), shape, axis))
    assert got.tobytes() == again.tobytes()  # fixed order: bit-repeatable


@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float64"])
def test_sum_many_short_rows(amd, dtype):
    """Row sums over more rows than one grid of the capped launch holds
    (300000 rows of 4: the waves stride over the rows) against numpy float64."""
    shape = (300000, 4)
    x = normal(21, shape)
    got = download(amd.sum(upload(x, dtype), shape, 1))
    values = stored(x, dtype).reshape(shape).astype(np.float64)
    expected = values.sum(axis=1)
    accumulate = 1.2e-16 if dtype == "float64" else 6e-8
    rounding = {"float32": 6e-8, "float64": 1.2e-16, "bfloat16": 3.9e-3}[dtype]
    assert np.all(np.abs(got - expected) <= 4 * accumulate * np.abs(values).sum(axis=1) + rounding * np.abs(expected))


@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float64"])
@pytest.mark.parametrize("shape,axis", [((3, 4, 5), 0), ((3, 4, 5), 1), ((3, 4, 5), 2), ((2, 300, 7), 1),
                                        ((16, 2048), 1), ((5, 3), 0)])
def test_softmax_any_axis(amd, dtype, shape, axis):
    x = normal(10, shape, 3.0)
    got = download(amd.softmax(upload(x, dtype), shape, axis))
    expected = np.asarray(ora.softmax(stored(x, dtype).ravel().tolist(), shape, axis))
    # fp32: the hardware exp2 of (x - max) * log2(e) costs a few ulps at
    # |x - max| ~ 20; bf16: one rounding of each probability
    tol = {"float32": 1e-5, "float64": 1e-13, "bfloat16": 8e-3}[dtype]
    assert np.all(np.abs(got - expected) <= tol * expected + 1e-9)


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_concatenate_gather_scatter(amd, dtype):
    a, b = normal(11, (2, 3, 4, 8)), normal(12, (2, 3, 5, 8))
    got = download(amd.concatenate((upload(a, dtype), upload(b, dtype)), (a.shape, b.shape), axis=2))
    assert got.tolist() == ora.concatenate((stored(a, dtype).ravel().tolist(), stored(b, dtype).ravel().tolist()),
                                           (a.shape, b.shape), 2)
    x = normal(13, 50)
    positions = [49, 0, 7, 7, 13, 2]
    assert download(amd.gather(upload(x, dtype), positions)).tolist() == ora.gather(stored(x, dtype).tolist(),
                                                                                     positions)
    values = normal(14, 6)
    got = download(amd.scatter(upload(values, dtype), positions, 50))
    expected = np.asarray(ora.scatter(stored(values, dtype).tolist(), positions, 50))
    close(got, stored(expected, dtype) if dtype == "bfloat16" else expected, dtype, scale=1e-6)
    with pytest.raises(IndexError):
        amd.gather(upload(x, dtype), [50])


def test_slices_and_their_gradient(amd):
    from qutai_amd import Tensor

    x = normal(15, (4, 6, 5))
    tensor = Tensor(upload(x, "float32"), shape=x.shape, requires_grad=True)
    for index in ((slice(None), slice(1, 5, 2)), (2,), (Ellipsis, slice(None, None, -1)), (slice(1, 3), None, 4),
                  (-1, slice(2, None), slice(None, None, 2))):
        part = tensor[index]
        assert part.shape == x[index].shape
        assert np.array(part.tolist()).ravel().tolist() == x[index].ravel().astype(np.float64).tolist()
        tensor.zero_grad()
        part.sum().backward()
        mask = np.zeros_like(x, dtype=np.float64)
        mask[index] = 1.0
        assert np.array(tensor.grad.tolist()).ravel().tolist() == mask.ravel().tolist()


# ---- autograd of the broadcasting front-end ------------------------------------------------

def test_broadcast_gradients_against_float64(amd):
    """d/dx of sum(w * op(x, y)) for broadcasting shapes, against numpy
    float64 on the fp32-stored inputs."""
    from qutai_amd import Tensor

    x, y = normal(16, (3, 1, 5)), normal(17, (4, 5)) + np.float32(4.0)
    w = normal(18, (3, 4, 5))
    X, Y = stored(x, "float32"), stored(y, "float32")
    W = stored(w, "float32")
    grads = {
        "add": (np.broadcast_to(W, W.shape), W),
        "subtract": (W, -W),
        "multiply": (W * Y, W * X),
        "divide": (W / Y, -W * X / Y ** 2),
    }
    for operation, (gx, gy) in grads.items():
        tx = Tensor(upload(x, "float32"), shape=x.shape, requires_grad=True)
        ty = Tensor(upload(y, "float32"), shape=y.shape, requires_grad=True)
        tw = Tensor(upload(w, "float32"), shape=w.shape)
        result = {"add": tx + ty, "subtract": tx - ty, "multiply": tx * ty, "divide": tx / ty}[operation]
        (result * tw).sum().backward()
        expected_x = np.broadcast_to(gx, W.shape).sum(axis=1, keepdims=True)
        expected_y = np.broadcast_to(gy, W.shape).sum(axis=0)
        np.testing.assert_allclose(np.array(tx.grad.tolist()), expected_x, rtol=2e-5, atol=1e-5)
        np.testing.assert_allclose(np.array(ty.grad.tolist()), expected_y, rtol=2e-5, atol=1e-5)


def test_softmax_middle_axis_gradient(amd):
    """Gradient of sum(w * softmax(x, axis=1)) = p * (w - sum(w p)) along the
    axis (src/qutai/core/operations/normalization.py:18-25)."""
    import qutai_amd as qt
    from qutai_amd import Tensor

    x, w = normal(19, (3, 6, 4), 2.0), normal(20, (3, 6, 4))
    tx = Tensor(upload(x, "float64"), shape=x.shape, requires_grad=True)
    (qt.softmax(tx, axis=1) * Tensor(upload(w, "float64"), shape=w.shape)).sum().backward()
    X, W = x.astype(np.float64), w.astype(np.float64)
    p = np.exp(X - X.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    expected = p * (W - (W * p).sum(axis=1, keepdims=True))
    np.testing.assert_allclose(np.array(tx.grad.tolist()), expected, rtol=1e-12, atol=1e-14)


def test_matmul_gradient_layouts(amd):
    """Every batch layout of the product gradient (equal batches, shared
    right, shared left, mixed broadcast, vectors) against float64 numpy."""
    from qutai_amd import Tensor

    cases = [((2, 3, 4), (2, 4, 5)), ((2, 3, 3, 4), (4, 5)), ((3, 4), (2, 3, 4, 5)), ((2, 1, 3, 4), (1, 3, 4, 5)),
             ((4,), (2, 4, 5)), ((2, 3, 4), (4,)), ((1, 3, 4), (2, 4, 5))]
    for left_shape, right_shape in cases:
        a, b = normal(21, left_shape), normal(22, right_shape)
        ta = Tensor(upload(a, "float64"), shape=a.shape, requires_grad=True)
        tb = Tensor(upload(b, "float64"), shape=b.shape, requires_grad=True)
        out = ta @ tb
        expected = np.matmul(a.astype(np.float64), b.astype(np.float64))
        assert out.shape == expected.shape
        g = normal(23, expected.shape)
        out.backward(Tensor(upload(g, "float64"), shape=g.shape))
        # reference gradients from numpy's own broadcasting rules
        A, B, G = a.astype(np.float64), b.astype(np.float64), g.astype(np.float64)
        A2 = A[None, :] if A.ndim == 1 else A
        B2 = B[:, None] if B.ndim == 1 else B
        G2 = G.reshape(np.matmul(A2, B2).shape)
        np.testing.assert_allclose(np.array(ta.grad.tolist()).ravel(),
                                   reduce_to(np.matmul(G2, np.swapaxes(B2, -1, -2)), A2.shape).ravel(),
                                   rtol=1e-12, atol=1e-13)
        np.testing.assert_allclose(np.array(tb.grad.tolist()).ravel(),
                                   reduce_to(np.matmul(np.swapaxes(A2, -1, -2), G2), B2.shape).ravel(),
                                   rtol=1e-12, atol=1e-13)


def reduce_to(values, shape):
    """Sum a broadcast result back to ``shape`` (numpy's reverse of broadcasting)."""
    while values.ndim > len(shape):
        values = values.sum(axis=0)
    axes = tuple(i for i, n in enumerate(shape) if n == 1 and values.shape[i] != 1)
    return values.sum(axis=axes, keepdims=True) if axes else values


# ---- KV-cache attention inference (src/qutai/nn/layers.py:345-355, nn/cache.py) --------------

def test_cached_multihead_attention_matches_full_causal(amd):
    """tests/test_attention_cache.py:19-32 on the amd device: chunked cached
    calls equal the full causal forward, with no graph recorded."""
    from qutai_amd import Tensor, nn
    from qutai_amd.core.context import set_recording

    layer = nn.MultiHeadAttention(4, heads=2, causal=True, seed=7, device="amd", dtype="float64")
    data = [[[0.1 * (batch * 20 + row * 4 + feature) for feature in range(4)] for row in range(5)]
            for batch in range(2)]
    inputs = Tensor(data, device="amd", dtype="float64", requires_grad=True)
    with set_recording(False):
        expected = np.array(layer(inputs).tolist())
    cache = nn.KVCache()
    for start, stop in ((0, 2), (2, 4), (4, 5)):
        actual = layer(inputs[:, start:stop], cache=cache)
        np.testing.assert_allclose(np.array(actual.tolist()), expected[:, start:stop], rtol=1e-12, atol=1e-13)
        assert cache.length == stop and cache.keys.shape == (2, 2, stop, 2)
        assert not actual.requires_grad and actual.parents == ()
    with pytest.raises(ValueError):
        nn.MultiHeadAttention(4, heads=2, device="amd")(inputs, cache=nn.KVCache())


def test_cached_attention_fp32_against_float64_oracle(amd):
    """Decode-style use at a real head size: 8 heads of 64, a 192-token
    prefill then single tokens, checked per head against the float64
    attention of the cached keys with the causal offset."""
    from qutai_amd import Tensor, nn

    features, heads, length = 512, 8, 200
    layer = nn.MultiHeadAttention(features, heads=heads, causal=True, seed=3, device="amd", dtype="float32")
    x = normal(24, (1, length, features))
    inputs = Tensor(upload(x, "float32"), shape=x.shape)
    cache = nn.KVCache()
    outputs = [np.array(layer(inputs[:, :192], cache=cache).tolist())]
    for t in range(192, length):
        outputs.append(np.array(layer(inputs[:, t:t + 1], cache=cache).tolist()))
    got = np.concatenate(outputs, axis=1)[0]
    # float64 reference from the layer's own fp32 weights
    weight = {name: np.array(getattr(layer, name).weight.tolist()) for name in ("query", "key", "value", "output")}
    X = x[0].astype(np.float64)
    q, k, v = (X @ weight[name] for name in ("query", "key", "value"))
    head = features // heads
    mixed = np.concatenate([ora.attention_np(q[:, h * head:(h + 1) * head], k[:, h * head:(h + 1) * head],
                                             v[:, h * head:(h + 1) * head], causal=True)[0] for h in range(heads)],
                           axis=1)
    expected = mixed @ weight["output"]
    assert ora.rel_frobenius(got, expected) <= 1e-5
    assert math.isfinite(float(got.sum()))


def test_normal_draws_are_seeded(amd):
    """cuda.normal's role for nn Dropout (nn/layers.py:87): N(mean, std)
    values, the same values for the same seed."""
    a = download(amd.normal(20000, 2.0, 0.5, seed=3, dtype="float32"))
    b = download(amd.normal(20000, 2.0, 0.5, seed=3, dtype="float32"))
    assert np.array_equal(a, b)
    assert abs(a.mean() - 2.0) < 0.02 and abs(a.std() - 0.5) < 0.02
    with pytest.raises(ValueError):
        amd.normal(4, dtype="int64")
