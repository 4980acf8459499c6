"""The activation-checkpoint contract (src/qutai/lm/recompute.py:11-79) on the
host, with numpy-backed stand-in storages and hand-written backward rules:
the forward runs once without recording, the backward runs the function
again under the forward's matmul precision, argument and declared-parameter
gradients are exact, a tensor that is both receives the sum of its parts,
an undeclared trainable tensor raises ValueError, and non-Tensor inputs or
results raise TypeError.  The cases follow the reference's own
tests/test_recompute.py:48-93 and 127-134 (replay count, repeated and
unused inputs, a declared capture that is also an argument, backward under
a recording pause); every expected value is a closed form."""
import numpy as np
import pytest

from qutai_amd.backends.precision import matmul_precision, set_matmul_precision
from qutai_amd.backends.storage import Storage
from qutai_amd.core import grad
from qutai_amd.core.context import set_recording
from qutai_amd.core.tensor import Tensor
from qutai_amd.lm import recompute


class HostStorage(Storage):
    device, dtype = "amd", "float32"

    def __init__(self, values):
        self.values = np.asarray(values, dtype=np.float64).ravel()

    @property
    def size(self):
        return self.values.size

    @property
    def nbytes(self):
        return 4 * self.values.size


def leaf(values, requires_grad=True):
    return Tensor(HostStorage(values), shape=(len(values),), requires_grad=requires_grad)


def multiply(x, y):
    """x * y with its product rule, recorded."""
    out = Tensor(HostStorage(x.storage.values * y.storage.values), shape=x.shape)
    return grad.record(out, (x, y), lambda g: (HostStorage(g.values * y.storage.values),
                                               HostStorage(g.values * x.storage.values)))


def plus(x, y):
    out = Tensor(HostStorage(x.storage.values + y.storage.values), shape=x.shape)
    return grad.record(out, (x, y), lambda g: (g, g))


class HostBackend:
    @staticmethod
    def add(a, b):
        return HostStorage(a.values + b.values)


@pytest.fixture(autouse=True)
def host_add(monkeypatch):
    monkeypatch.setattr(recompute, "get_backend", lambda device: HostBackend)
    monkeypatch.setattr(grad, "get_backend", lambda device: HostBackend)


def run_backward(output, seed):
    return grad.backward(output, HostStorage(seed))


def test_argument_and_declared_parameter_gradients_and_replay():
    x, w = leaf([1.0, 2.0, 3.0]), leaf([0.5, -1.0, 4.0])
    calls, precisions = [], []

    def function(value):
        calls.append(1)
        precisions.append(matmul_precision())
        return multiply(multiply(value, w), value)  # x^2 w

    with set_matmul_precision("bfloat16"):
        y = recompute.checkpoint(function, x, parameters=(w, w))
    assert len(calls) == 1 and y.parents == (x, w)
    assert np.array_equal(y.storage.values, [0.5, -4.0, 36.0])
    with set_matmul_precision(None):
        leaves = run_backward(y, [1.0, 1.0, 2.0])
    assert len(calls) == 2 and precisions == ["bfloat16", "bfloat16"]
    assert np.allclose(leaves[x].values, [1.0, -4.0, 48.0])    # 2 x w g
    assert np.allclose(leaves[w].values, [1.0, 4.0, 18.0])     # x^2 g


def test_tensor_that_is_argument_and_parameter_gets_both_parts():
    x, w = leaf([2.0, -1.0]), leaf([3.0, 5.0])

    def function(value):
        return multiply(value, w)  # value * w, with w closed over

    y = recompute.checkpoint(function, w, parameters=(w,))  # w * w
    assert y.parents == (w,)
    leaves = run_backward(y, [1.0, 1.0])
    assert np.allclose(leaves[w].values, [6.0, 10.0])  # argument part w + parameter part w
    z = recompute.checkpoint(function, x, parameters=(w,))
    leaves = run_backward(z, [1.0, 2.0])
    assert np.allclose(leaves[x].values, [3.0, 10.0]) and np.allclose(leaves[w].values, [2.0, -2.0])


def test_frozen_inputs_get_no_gradient():
    x, w = leaf([1.0, 2.0], requires_grad=False), leaf([4.0, 4.0])
    y = recompute.checkpoint(lambda value: multiply(value, w), x, parameters=(w,))
    replay = y.backward_rule
    assert replay(HostStorage([1.0, 1.0]))[0] is None


def test_undeclared_trainable_tensor_raises():
    x, hidden = leaf([1.0, 2.0]), leaf([3.0, 4.0])
    y = recompute.checkpoint(lambda value: multiply(value, hidden), x)
    with pytest.raises(ValueError):
        run_backward(y, [1.0, 1.0])


def test_non_tensor_inputs_and_results_raise():
    x = leaf([1.0])
    with pytest.raises(TypeError):
        recompute.checkpoint(lambda value: value, [1.0])
    with pytest.raises(TypeError):
        recompute.checkpoint(lambda value: value, x, parameters=([1.0],))
    with pytest.raises(TypeError):
        recompute.checkpoint(lambda value: (value, value), x)


def test_repeated_and_unused_inputs_and_recording_pause():
    """(a + b) * w over (x, x, unused): x gets 2 w, unused nothing, w gets
    a + b (tests/test_recompute.py:75-93); the backward runs with recording
    paused and still rebuilds the graph (:127-134)."""
    x, unused, w = leaf([2.0]), leaf([3.0]), leaf([4.0])
    y = recompute.checkpoint(lambda a, b, c: multiply(plus(a, b), w), x, x, unused, parameters=(w,))
    assert y.parents == (x, unused, w)
    with set_recording(False):
        leaves = run_backward(y, [1.0])
    assert np.allclose(leaves[x].values, [8.0]) and np.allclose(leaves[w].values, [4.0])
    assert unused not in leaves
    with set_recording(False):
        assert not recompute.checkpoint(lambda a: multiply(a, a), x).requires_grad
