"""Host-side logic without a GPU: argument validation of the GEMM boundary
(the reference's ValueError contract, src/qutai/backends/cuda.py:305-334),
matmul shape rules and autograd plumbing on a numpy stand-in backend, and the
lazy runtime import.  No kernel is launched."""
import subprocess
import sys

import numpy as np
import pytest

from qutai_amd.backends import amd, device
from qutai_amd.backends.storage import Storage


class NoRuntime:
    def free(self, ptr):
        pass


def fake_storage(size, dtype, ptr=1 << 20):
    """An AMDStorage shell with no device allocation (validation only)."""
    s = object.__new__(amd.AMDStorage)
    s.dtype, s._size, s.ptr = dtype, size, ptr
    s.runtime = NoRuntime()
    return s


class FakeBackend:
    """numpy stand-in with the backend-module protocol used by the front-end."""

    class Store(Storage):
        device = "fake"

        def __init__(self, values, dtype="float32"):
            self.values = np.asarray(values, dtype=np.float64).ravel()
            self.dtype = dtype

        @property
        def size(self):
            return self.values.size

        @property
        def nbytes(self):
            return self.values.size * 4

        def copy(self):
            return FakeBackend.Store(self.values.copy(), self.dtype)

        def tolist(self):
            return self.values.tolist()

    @staticmethod
    def storage(values, dtype="float32"):
        return FakeBackend.Store(list(values), dtype)

    @staticmethod
    def full(size, value=0.0, dtype="float32"):
        return FakeBackend.Store(np.full(size, value), dtype)

    @staticmethod
    def add(a, b):
        return FakeBackend.Store(a.values + b.values, a.dtype)

    @staticmethod
    def matmul(left, right, ls, rs):
        a = left.values.reshape((1,) * (len(rs) - len(ls)) + tuple(ls) if len(ls) < len(rs) else ls)
        b = right.values.reshape((1,) * (len(ls) - len(rs)) + tuple(rs) if len(rs) < len(ls) else rs)
        return FakeBackend.Store(np.matmul(a, b), left.dtype)

    @staticmethod
    def gemm(a, b, rows, inner, cols, *, batch=1, transpose_left=False, transpose_right=False, left_stride=None,
             right_stride=None, out_dtype=None, **_):
        def operand(values, stride, shape, dense):
            stride = dense if stride is None else stride
            return np.stack([values[z * stride:z * stride + dense].reshape(shape) for z in range(batch)])

        A = operand(a.values, left_stride, (inner, rows) if transpose_left else (rows, inner), rows * inner)
        B = operand(b.values, right_stride, (cols, inner) if transpose_right else (inner, cols), inner * cols)
        A = A.transpose(0, 2, 1) if transpose_left else A
        B = B.transpose(0, 2, 1) if transpose_right else B
        return FakeBackend.Store(A @ B, out_dtype or a.dtype)

    @staticmethod
    def transpose(values, shape, axes=None):
        return FakeBackend.Store(values.values.reshape(shape).transpose(axes), values.dtype)

    @staticmethod
    def unbroadcast(values, shape, target):
        v = values.values.reshape(shape)
        padded = (1,) * (len(shape) - len(target)) + tuple(target)
        for axis, n in enumerate(padded):
            if n == 1 and shape[axis] != 1:
                v = v.sum(axis=axis, keepdims=True)
        return FakeBackend.Store(v, values.dtype)

    @staticmethod
    def sum(values, shape=None, axis=None):
        if axis is None:
            return FakeBackend.Store([values.values.sum()], values.dtype)
        return FakeBackend.Store(values.values.reshape(shape).sum(axis=axis), values.dtype)

    @staticmethod
    def broadcast(values, shape, target):
        if tuple(shape) == tuple(target):
            return values
        return FakeBackend.Store(np.broadcast_to(values.values.reshape(shape), target).copy(), values.dtype)


@pytest.fixture
def fake_device(monkeypatch):
    monkeypatch.setitem(device._BACKENDS, "fake", FakeBackend)
    return "fake"


# ---- GEMM boundary validation (no device call is reached) -------------------------

def test_gemm_rejects_what_the_reference_rejects():
    a = fake_storage(4, "float32")
    out_alias = a
    with pytest.raises(ValueError):
        amd.gemm(a, a, 2, 2, 2, out=out_alias)                 # aliasing
    with pytest.raises(ValueError):
        amd.gemm(a, a, 2, 2, 2, accumulate=True)               # accumulate without out
    with pytest.raises(ValueError):
        amd.gemm(a, a, 2, 2, 2, out=fake_storage(4, "bfloat16", 1 << 30))  # wrong out dtype (fp32 default)
    with pytest.raises(ValueError):
        amd.gemm(a, a, 2, 2, 2, left_stride=-1)                # negative stride
    with pytest.raises(ValueError):
        amd.gemm(a, a, 3, 2, 2)                                # storage too small
    with pytest.raises(ValueError):
        amd.gemm(fake_storage(4, "float64"), a, 2, 2, 2)       # f64 with f32
    with pytest.raises(ValueError):
        amd.gemm(a, a, 2, 2, 2, out_dtype="float64")           # f64 out from f32 inputs
    with pytest.raises(ValueError):
        amd.gemm(a, a, 2.0, 2, 2)                              # non-integer dims
    with pytest.raises(ValueError):
        amd.gemm([1, 2], a, 1, 2, 1)                           # not a device storage
    with pytest.raises(ValueError):
        amd.gemm(fake_storage(4, "int64"), a, 2, 2, 2)         # unsupported dtype


def test_zero_size_output_returns_before_any_device_work():
    empty, fifteen = fake_storage(0, "float32"), fake_storage(15, "float32", 1 << 24)
    out = fake_storage(0, "float32", 1 << 30)
    assert amd.gemm(empty, fifteen, 0, 5, 3, out=out) is out
    assert amd.gemm(fifteen, empty, 3, 5, 0, out=out) is out
    with pytest.raises(ValueError):
        amd.gemm(empty, empty, 0, 5, 3, out=out)  # B must still hold inner x cols values


def test_get_backend_checks_device_and_dtype(fake_device):
    s = FakeBackend.Store([1.0, 2.0])
    t = FakeBackend.Store([1.0], dtype="bfloat16")
    assert device.get_backend(s) is FakeBackend
    with pytest.raises(ValueError):
        device.get_backend(s, t)
    with pytest.raises(ValueError):
        device.get_backend("cuda")


# ---- front-end shape rules and autograd on the stand-in backend --------------------

def test_matmul_shapes_and_known_answers(fake_device):
    import qutai_amd as qt
    from qutai_amd import Tensor

    # tests/test_batched_matmul.py:28-53 on the host stand-in
    assert qt.matmul(Tensor([1, 2, 3], device="fake"), Tensor([4, 5, 6], device="fake")).item() == 32
    r = qt.matmul(Tensor([1, 2], device="fake"), Tensor([[3, 4, 5], [6, 7, 8]], device="fake"))
    assert r.shape == (3,) and r.tolist() == [15, 18, 21]
    left = Tensor(list(range(1, 13)), shape=(2, 1, 2, 3), device="fake")
    right = Tensor(list(range(1, 19)), shape=(1, 3, 3, 2), device="fake")
    assert qt.matmul(left, right).shape == (2, 3, 2, 2)
    for bad_left, bad_right in [((2,), (3,)), ((2, 2, 3), (3, 3, 2))]:
        with pytest.raises(ValueError):
            qt.matmul(Tensor([0.0] * int(np.prod(bad_left)), shape=bad_left, device="fake"),
                      Tensor([0.0] * int(np.prod(bad_right)), shape=bad_right, device="fake"))


def test_matmul_gradient_rules(fake_device):
    import qutai_amd as qt
    from qutai_amd import Tensor

    # tests/test_batched_matmul.py:55-67: shared weight, vector x batched matrices
    left = Tensor(list(range(1, 13)), shape=(2, 2, 3), requires_grad=True, device="fake")
    weight = Tensor([[7, 8], [9, 10], [11, 12]], requires_grad=True, device="fake")
    qt.sum(qt.matmul(left, weight)).backward()
    assert left.grad.tolist() == [[[15, 19, 23]] * 2] * 2
    assert weight.grad.tolist() == [[22, 22], [26, 26], [30, 30]]
    vector = Tensor([1, 2], requires_grad=True, device="fake")
    mats = Tensor([[[3, 4], [5, 6]], [[7, 8], [9, 10]]], requires_grad=True, device="fake")
    qt.matmul(vector, mats).backward(Tensor([[1, 2], [3, 4]], device="fake"))
    assert vector.grad.tolist() == [64, 84]
    assert mats.grad.tolist() == [[[1, 2], [2, 4]], [[3, 4], [6, 8]]]


def test_precision_token_restores_previous_value():
    from qutai_amd.backends.precision import matmul_precision, set_matmul_precision

    assert matmul_precision() is None
    with set_matmul_precision("bfloat16"):
        assert matmul_precision() == "bfloat16"
        with set_matmul_precision(None):
            assert matmul_precision() is None
        assert matmul_precision() == "bfloat16"
    assert matmul_precision() is None
    with pytest.raises(ValueError):
        set_matmul_precision("float16")


def test_importing_the_package_does_not_touch_the_gpu():
    code = ("import qutai_amd, qutai_amd.lm, qutai_amd.nn; from qutai_amd.backends import amd_runtime; "
            "assert amd_runtime._runtime is None; print('lazy')")
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, cwd=str(
        __import__("pathlib").Path(__file__).resolve().parent.parent))
    assert out.returncode == 0 and "lazy" in out.stdout


def test_owned_gradient_marks_are_taken_once():
    """A rule's freshly allocated gradient (grad.owned) is kept by the first
    leaf that receives it; any later receiver copies (core/grad.py)."""
    from qutai_amd.core.grad import owned, take_owned

    class Box:
        pass

    box = Box()
    assert owned(None) is None
    assert not take_owned(box)
    assert owned(box) is box
    assert take_owned(box)
    assert not take_owned(box)


def test_deferred_gradient_adds_in_place_only_into_this_pass_grad(fake_device):
    """A DeferredGradient (the embedding table's row sums) is added in place
    into a leaf gradient created by the same backward pass, and materialised
    otherwise, so a grad kept from an earlier pass is never written
    (core/grad.py, core/tensor.py)."""
    from qutai_amd import Tensor
    from qutai_amd.core.grad import DeferredGradient, owned, record

    class Rows(DeferredGradient):
        device, dtype, size = "fake", "float32", 3
        added_in_place = 0

        def materialize(self):
            return FakeBackend.Store(np.array([0.0, 5.0, 0.0]), "float32")

        def add_into(self, storage):
            Rows.added_in_place += 1
            storage.values[1] += 5.0

    w = Tensor(FakeBackend.Store(np.zeros(3), "float32"), shape=(3,), requires_grad=True)
    y = record(Tensor(FakeBackend.Store(np.zeros(1), "float32"), shape=()), (w, w),
               lambda g: (owned(FakeBackend.Store(np.array([1.0, 1.0, 1.0]), "float32")), Rows()))
    y.backward()
    assert w.grad.storage.values.tolist() == [1.0, 6.0, 1.0] and Rows.added_in_place == 1
    kept = w.grad.storage
    # a second pass: the deferred part meets the grad of the first pass and is materialised
    y2 = record(Tensor(FakeBackend.Store(np.zeros(1), "float32"), shape=()), (w,), lambda g: (Rows(),))
    y2.backward()
    assert Rows.added_in_place == 1
    assert kept.values.tolist() == [1.0, 6.0, 1.0]
    assert w.grad.storage.values.tolist() == [1.0, 11.0, 1.0]


def test_scatter_grouping_is_a_stable_counting_sort():
    """amd.scatter's host grouping: targets' sources in input order (the
    stable sort of positions), offsets of every target, empty input."""
    from array import array

    rng = np.random.default_rng(3)
    for n, size in ((0, 4), (1, 1), (500, 7), (4000, 300)):
        index = array("q", rng.integers(0, size, n).tolist())
        start, order = amd._group_by_target(index, size)
        assert list(order) == sorted(range(n), key=index.__getitem__)
        assert list(start) == [0] + np.cumsum(np.bincount(np.asarray(index, dtype=np.int64), minlength=size)).tolist()


def test_moe_forward_reads_rows_through_the_order_only_below_2_gib():
    """The routed-row read inside the grouped GEMMs addresses the token
    matrix with 32-bit offsets (qutai_amd_gemm_grouped / _swiglu / _grouped_k
    refuse a token matrix of 2 GiB or more on that path), so larger inputs
    take the gathered copy, in the forward alone and in training."""
    from qutai_amd.backends import amd_lm

    assert amd_lm._rows_through_order(8192 * 2048 * 2, dtype="bfloat16")
    assert amd_lm._rows_through_order(8192 * 2048 * 4, dtype="float32")
    assert not amd_lm._rows_through_order(1 << 31, dtype="bfloat16")
    assert amd_lm._rows_through_order((1 << 31) - 2, dtype="bfloat16")
    assert not amd_lm._rows_through_order(1024, dtype="float64")
