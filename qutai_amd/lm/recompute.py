"""Activation recomputation (the contract of src/qutai/lm/recompute.py:11-79).

``checkpoint(function, *arguments, parameters=...)`` evaluates ``function``
with graph recording off and keeps only its output.  The output's backward
rule is a ``_Replay``: it evaluates the function again with recording on,
under the matmul precision that was in force for the forward, on stand-in
leaves that share the arguments' storage, back-propagates through that
second graph, and hands every leaf gradient to the input it belongs to.
Parameters the function closes over must be declared, because they are
graph inputs of the checkpointed node like the arguments; a recomputed
graph that reaches any other trainable tensor raises ``ValueError``.  A
tensor that is both an argument and a declared parameter receives the sum of
its two parts."""
from __future__ import annotations

from ..backends.device import get_backend
from ..backends.precision import matmul_precision, set_matmul_precision
from ..core import grad
from ..core.context import set_recording
from ..core.tensor import Tensor


def _unique(tensors):
    """The tensors in first-seen order, each once (identity, not value)."""
    seen, result = set(), []
    for tensor in tensors:
        if id(tensor) not in seen:
            seen.add(id(tensor))
            result.append(tensor)
    return tuple(result)


def _single_tensor(value):
    if not isinstance(value, Tensor):
        raise TypeError("a checkpointed function must return one Tensor")
    return value


class _Replay:
    """Backward rule of one checkpointed call (see the module docstring)."""

    def __init__(self, function, arguments, parameters, precision):
        self.function, self.arguments, self.parameters = function, arguments, parameters
        self.precision = precision
        self.inputs = _unique((*arguments, *parameters))  # the graph parents, in this order

    def __call__(self, gradient):
        position = {id(tensor): i for i, tensor in enumerate(self.inputs)}
        # one stand-in leaf per argument position, sharing its storage: the
        # argument part of a tensor's gradient arrives on the stand-in, the
        # closed-over part on the tensor itself
        stand_ins = [Tensor(a.storage, shape=a.shape, requires_grad=a.requires_grad) for a in self.arguments]
        owner = {id(s): position[id(a)] for s, a in zip(stand_ins, self.arguments)}
        for parameter in self.parameters:
            owner[id(parameter)] = position[id(parameter)]
        with set_recording(True), set_matmul_precision(self.precision):
            rerun = _single_tensor(self.function(*stand_ins))
            leaf_gradients = grad.backward(rerun, gradient, retain_graph=False) if rerun.requires_grad else {}
        totals = [None] * len(self.inputs)
        for leaf, part in leaf_gradients.items():
            slot = owner.get(id(leaf))
            if slot is None:
                raise ValueError("the recomputed function reached a trainable Tensor not passed as a parameter")
            if totals[slot] is None:
                totals[slot] = part
            else:
                totals[slot] = get_backend(self.inputs[slot].device).add(totals[slot], part)
        return tuple(total if tensor.requires_grad else None for total, tensor in zip(totals, self.inputs))


def checkpoint(function, *arguments, parameters=()):
    parameters = _unique(parameters)
    for value in (*arguments, *parameters):
        if not isinstance(value, Tensor):
            raise TypeError("checkpoint arguments and parameters must be Tensors")
    with set_recording(False):
        output = _single_tensor(function(*arguments))
    replay = _Replay(function, arguments, parameters, matmul_precision())
    return grad.record(Tensor(output.storage, shape=output.shape), replay.inputs, replay)
