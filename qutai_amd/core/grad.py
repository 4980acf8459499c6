"""Reverse-mode graph: record and backward (src/qutai/core/grad.py:7-65)."""
from __future__ import annotations

from ..backends.device import get_backend
from .context import is_recording


def record(result, parents, rule=None):
    """Keep the parents and the bound local backward rule on the result."""
    result.requires_grad = is_recording() and any(parent.requires_grad for parent in parents)
    if result.requires_grad:
        result.parents = parents
        result.backward_rule = rule
    return result


def owned(storage):
    """Mark a gradient storage that its backward rule has just allocated and
    hands to no one else: the leaf that receives it first may keep it as its
    ``grad`` instead of copying it (the copy isolates storages a rule passes
    on to several tensors).  Returns the storage; None passes through."""
    if storage is not None:
        storage.owned_gradient = True
    return storage


def take_owned(storage):
    """True (once) when ``storage`` was marked by ``owned``."""
    if getattr(storage, "owned_gradient", False):
        storage.owned_gradient = False
        return True
    return False


class DeferredGradient:
    """A gradient contribution a rule describes instead of materialising:
    ``materialize()`` gives the dense storage, and ``add_into(storage)``
    adds it in place into a gradient that this backward pass created (the
    embedding table's row sums: a few rows of a [vocab][width] gradient; a
    Linear's fp32 dX = G W, summed by the GEMM's accumulate epilogue).
    ``add_into`` must give the same values as ``storage + materialize()``.
    Has ``device``, ``dtype`` and ``size`` like a storage."""

    def materialize(self):
        raise NotImplementedError

    def add_into(self, storage):
        raise NotImplementedError

    def sum_with(self, existing, in_place):
        """existing + this contribution.  ``in_place``: ``existing`` is a
        gradient this pass allocated and no rule holds, so it may be
        written; otherwise the sum goes to a new storage."""
        if in_place:
            self.add_into(existing)
            return existing
        return get_backend(existing.device).add(existing, self.materialize())


def _dense(contribution):
    return contribution.materialize() if isinstance(contribution, DeferredGradient) else contribution


def _topological_order(output):
    order, seen, pending = [], set(), [(output, False)]
    while pending:
        tensor, expanded = pending.pop()
        if expanded:
            order.append(tensor)
        elif tensor not in seen:
            seen.add(tensor)
            if getattr(tensor, "_graph_released", False):
                raise RuntimeError("graph already released; run forward again or retain the graph")
            if tensor.parents and tensor.backward_rule is None:
                raise NotImplementedError("graph contains an operation without a backward rule")
            pending.append((tensor, True))
            pending.extend((parent, False) for parent in tensor.parents if parent.requires_grad)
    return order


def backward(output, gradient, *, retain_graph=True, leaf_sink=None):
    """Propagate ``gradient``; leaves go to ``leaf_sink`` (or a returned dict)."""
    order = _topological_order(output)
    gradients = {output: gradient}
    # non-leaf gradients this loop allocated (a materialised deferred
    # contribution or a sum): no rule holds them, so later deferred
    # contributions may be added into them in place
    fresh = set()
    leaves = {}
    while order:
        tensor = order.pop()
        incoming = gradients.pop(tensor, None)
        if incoming is None:
            continue
        rule = tensor.backward_rule
        if rule is None:
            if leaf_sink is None:
                leaves[tensor] = _dense(incoming)
            else:
                leaf_sink(tensor, incoming)
            continue
        contributions = rule(incoming)
        parents = tensor.parents
        if not retain_graph:
            tensor.parents, tensor.backward_rule, tensor._graph_released = (), None, True
        for parent, contribution in zip(parents, contributions, strict=True):
            if parent.requires_grad and contribution is not None:
                if leaf_sink is not None and parent.backward_rule is None:
                    leaf_sink(parent, contribution)
                elif parent in gradients:
                    existing = gradients[parent]
                    if isinstance(contribution, DeferredGradient) and contribution.dtype == existing.dtype:
                        gradients[parent] = contribution.sum_with(existing, parent in fresh)
                        fresh.add(parent)
                    else:
                        contribution = _dense(contribution)
                        gradients[parent] = get_backend(contribution.device).add(existing, contribution)
                        fresh.add(parent)
                else:
                    if isinstance(contribution, DeferredGradient):
                        fresh.add(parent)
                    gradients[parent] = _dense(contribution)
    return leaves
