"""Activation recomputation (src/qutai/lm/recompute.py:11-79).

``checkpoint`` runs a side-effect-free function without recording, keeps
only its output, and in backward runs it again with recording on (under the
matmul precision of the forward) to get the gradients of its arguments and
of the parameters it closes over.  The parameters must be passed
explicitly: a trainable tensor reached by the recomputed graph that is
neither an argument nor a declared parameter raises ``ValueError``."""
from __future__ import annotations

from ..backends.device import get_backend
from ..backends.precision import matmul_precision, set_matmul_precision
from ..core import grad
from ..core.context import set_recording
from ..core.tensor import Tensor


def checkpoint(function, *arguments, parameters=()):
    parameters = tuple(dict.fromkeys(parameters))
    if not all(isinstance(value, Tensor) for value in (*arguments, *parameters)):
        raise TypeError("checkpoint arguments and parameters must be Tensors")
    parents = tuple(dict.fromkeys((*arguments, *parameters)))
    with set_recording(False):
        output = function(*arguments)
    if not isinstance(output, Tensor):
        raise TypeError("a checkpointed function must return one Tensor")
    precision = matmul_precision()

    def backward(gradient):
        # fresh leaves for the arguments: their identity separates argument
        # gradients from parameter gradients when one tensor is both
        stand_ins = {value: Tensor(value.storage, shape=value.shape, requires_grad=value.requires_grad)
                     for value in arguments}
        with set_recording(True), set_matmul_precision(precision):
            rerun = function(*(stand_ins[value] for value in arguments))
            if not isinstance(rerun, Tensor):
                raise TypeError("a checkpointed function must return one Tensor")
            leaves = grad.backward(rerun, gradient, retain_graph=False) if rerun.requires_grad else {}
        declared = set(parameters)
        known = set(stand_ins.values()) | declared
        if any(leaf not in known for leaf in leaves):
            raise ValueError("the recomputed function reached a trainable Tensor not passed as a parameter")
        results = []
        for value in parents:
            if not value.requires_grad:
                results.append(None)
                continue
            part = leaves.get(stand_ins[value]) if value in stand_ins else None
            if value in declared and value in leaves:
                part = leaves[value] if part is None else get_backend(value.device).add(part, leaves[value])
            results.append(part)
        return tuple(results)

    return grad.record(Tensor(output.storage, shape=output.shape), parents, backward)
