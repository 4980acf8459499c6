"""Decoder-LM kernels of the amd device (sibling of src/qutai/backends/cuda_lm.py).

Same names and argument meaning as the reference LM backend for the
contraction path: ``gemm`` (cuda_lm.py:31-55), ``routing`` (:368-449),
``route_gather`` / ``route_gather_backward`` (:471-502), ``combine`` /
``combine_backward`` (:505-581), ``silu`` products, ``take``.  Additions that
the MI355X design needs: ``route_gather_all`` and ``combine_all`` (one launch
for every expert), ``grouped_gemm`` and ``moe_experts_forward`` (the expert
projections as grouped GEMMs whose per-expert row ranges stay in device
memory, so no host synchronisation sizes them).
"""
from __future__ import annotations

from array import array
from bisect import bisect_left
from functools import partial
from random import Random

from . import amd
from .amd import _TYPES, AMDStorage, code
from .amd_runtime import get_runtime
from ..core.grad import DeferredGradient


def normal(size, mean=0.0, std=1.0, *, seed=None, dtype="float32"):
    """Host-drawn N(mean, std) values (Random(seed).gauss, as the CPU path
    draws them: src/qutai/backends/cpu_lm.py:6-8), uploaded once."""
    random = Random(seed)
    return amd.storage(array("f", (random.gauss(mean, std) for _ in range(size))), dtype=dtype)


def gemm(a, b, rows, inner, cols, *, transpose_left=False, transpose_right=False, out_dtype=None, out=None,
         accumulate=False):
    """LM GEMM without batch/strides (src/qutai/backends/cuda_lm.py:31-55)."""
    return amd.gemm(a, b, rows, inner, cols, transpose_left=transpose_left, transpose_right=transpose_right,
                    out_dtype=out_dtype, out=out, accumulate=accumulate)


def take(values, start, size):
    return amd.take(values, start, size)


def silu_mul(gate: AMDStorage, up: AMDStorage) -> AMDStorage:
    """silu(gate) * up with the reference's per-op rounding."""
    if (gate.dtype, gate.size) != (up.dtype, up.size):
        raise ValueError("silu_mul needs operands of equal dtype and size")
    out = AMDStorage(gate.size, gate.dtype)
    if gate.size:
        out.runtime.call("qutai_amd_silu_mul", gate.ptr, up.ptr, out.ptr, gate.size, code(gate.dtype))
    return out


def silu_mul_backward(gradient, gate, up):
    dgate, dup = AMDStorage(gate.size, gate.dtype), AMDStorage(up.size, up.dtype)
    if gate.size:
        dgate.runtime.call("qutai_amd_silu_mul_backward", gradient.ptr, gate.ptr, up.ptr, dgate.ptr, dup.ptr,
                           gate.size, code(gate.dtype))
    return dgate, dup


def _route_workspace_bytes(runtime, rows, experts, top_k):
    """Workspace of the chunked routing path (0: the per-expert pack)."""
    return runtime.lib.qutai_amd_route_workspace_size(rows, experts, top_k)


def routing(scores, rows, experts, top_k, *, download_counts=True):
    """Router softmax, top-k selection and stable per-expert packing.

    Returns the dict of ``cuda_lm.routing`` (cuda_lm.py:436-449): probs,
    weights, indices, counts, ids, slots, locations, utilization, aux, rows,
    experts, top_k, capacity; plus ``offsets`` ([experts+1], device) and
    ``order`` (token ids expert-major, device) used by the one-launch gather
    and the grouped GEMMs.  ``counts`` is a host tuple (one device read, as
    in the reference) unless ``download_counts`` is False.
    """
    if scores.dtype == "bfloat16":
        scores = amd.from_storage(scores, dtype="float32")
    if scores.dtype != "float32":
        raise ValueError("amd routing takes float32 or bfloat16 router scores")
    if experts <= 0 or not 0 < top_k <= experts or scores.size != rows * experts:
        raise ValueError("routing needs 0 < top_k <= experts and rows * experts scores")
    capacity = rows * top_k
    probs = AMDStorage(rows * experts, "float32")
    weights = AMDStorage(capacity, "float32")
    indices = AMDStorage(capacity, "int64")
    counts = AMDStorage(experts, "int64")
    ids = AMDStorage(experts * capacity, "int64")
    slots = AMDStorage(experts * capacity, "int64")
    locations = AMDStorage(capacity, "int64")
    offsets = AMDStorage(experts + 1, "int64")
    order = AMDStorage(capacity, "int64")
    utilization = AMDStorage(experts, "float32")
    aux = AMDStorage(1, "float32")
    runtime = get_runtime()
    need = _route_workspace_bytes(runtime, rows, experts, top_k)
    workspace = AMDStorage((need + 3) // 4, "float32") if need else None
    runtime.call("qutai_amd_route", scores.ptr, probs.ptr, weights.ptr, indices.ptr, counts.ptr, ids.ptr, slots.ptr,
                 locations.ptr, offsets.ptr, order.ptr, utilization.ptr, aux.ptr, rows, experts, top_k,
                 workspace.ptr if workspace else None, need)
    host_counts = tuple(counts.to_array().tolist()) if download_counts else None
    return dict(probs=probs, weights=weights, indices=indices, counts=host_counts, count_buffer=counts, ids=ids,
                slots=slots, locations=locations, offsets=offsets, order=order, utilization=utilization, aux=aux,
                rows=rows, experts=experts, top_k=top_k, capacity=capacity)


def _host_offsets(route):
    counts = route["counts"]
    if counts is None:
        raise ValueError("per-expert calls need the host counts (routing(..., download_counts=True))")
    starts = [0]
    for count in counts:
        starts.append(starts[-1] + count)
    return starts


def route_gather(values, route, expert, width):
    """Rows of one expert, in token order (cuda_lm.py:471-485)."""
    start = _host_offsets(route)[expert]
    count = route["counts"][expert]
    result = AMDStorage(count * width, values.dtype)
    if count * width:
        result.runtime.call("qutai_amd_route_gather", values.ptr, route["order"].ptr + 8 * start, result.ptr, count,
                            width, 0, code(values.dtype))
    return result


def route_gather_backward(gradient, route, expert, width):
    """Scatter one expert's row gradients back to token rows (cuda_lm.py:488-502)."""
    start = _host_offsets(route)[expert]
    count = route["counts"][expert]
    result = amd.full(route["rows"] * width, 0.0, dtype=gradient.dtype)
    if count * width:
        result.runtime.call("qutai_amd_route_gather", gradient.ptr, route["order"].ptr + 8 * start, result.ptr,
                            count, width, 1, code(gradient.dtype))
    return result


def route_gather_all(values, route, width):
    """All experts' token rows in one expert-major block [rows*top_k, width]."""
    total = route["capacity"]
    result = AMDStorage(total * width, values.dtype)
    if total * width:
        result.runtime.call("qutai_amd_route_gather", values.ptr, route["order"].ptr, result.ptr, total, width, 0,
                            code(values.dtype))
    return result


def combine_all(expert_rows, route, width):
    """y[row] = sum_slot weight * expert output row, from the expert-major
    block produced by the grouped GEMMs (one launch, fp32 sum, one rounding)."""
    result = AMDStorage(route["rows"] * width, expert_rows.dtype)
    if result.size:
        result.runtime.call("qutai_amd_combine", expert_rows.ptr, route["weights"].ptr, route["indices"].ptr,
                            route["locations"].ptr, route["offsets"].ptr, result.ptr, route["rows"], width,
                            route["top_k"], code(expert_rows.dtype), code(expert_rows.dtype))
    return result


def combine(outputs, weights, route, width):
    """Reference-shaped combine over a list of (expert, rows) outputs
    (cuda_lm.py:505-541): the rows are laid out expert-major and combined
    in one launch."""
    if weights is not route["weights"]:
        route = dict(route, weights=weights)
    dtype = outputs[0][1].dtype if outputs else "float32"
    block = AMDStorage(route["capacity"] * width, dtype)
    starts = _host_offsets(route)
    item = 2 if dtype == "bfloat16" else 4
    for expert, values in outputs:
        if values.size:
            block.runtime.copy(block.ptr + starts[expert] * width * item, values.ptr, values.nbytes)
    return combine_all(block, route, width)


def grouped_gemm(rows_block, weight_stack, route, inner, cols, *, out_dtype="bfloat16", transpose_right=True,
                 out=None, accumulate=False, gather=False):
    """out[offsets[e]:offsets[e+1]] (+)= rows_block[offsets[e]:offsets[e+1]] @ op(W_e)
    for every expert in one launch, the row ranges read on the device.  With
    ``transpose_right`` W_e = weight_stack[e] is stored (cols, inner) and used
    transposed (the forward X W^T); without, it is stored (inner, cols) (the
    backward dY W).  With ``gather`` rows_block is the token matrix
    [rows][inner] and the expert-major rows are read through ``order``
    inside the GEMM (no gathered copy)."""
    experts = route["experts"]
    if weight_stack.size != experts * cols * inner or rows_block.dtype != weight_stack.dtype:
        raise ValueError("grouped_gemm needs [experts] weights of cols*inner values in the rows' dtype")
    source = route["rows"] if gather else route["capacity"]
    if rows_block.size != source * inner:
        raise ValueError("grouped_gemm rows do not match the route (rows x inner, or capacity x inner)")
    if out is None:
        if accumulate:
            raise ValueError("accumulate needs out")
        out = AMDStorage(route["capacity"] * cols, out_dtype)
    elif out.dtype != out_dtype or out.size != route["capacity"] * cols:
        raise ValueError("out must hold capacity x cols values of out_dtype")
    if out.size:
        out.runtime.call("qutai_amd_gemm_grouped", rows_block.ptr, weight_stack.ptr, out.ptr, route["offsets"].ptr,
                         experts, route["capacity"], inner, cols, cols * inner, int(transpose_right),
                         code(rows_block.dtype), code(out_dtype), int(accumulate),
                         route["order"].ptr if gather else None, source if gather else 0, mfma=True)
    return out


def grouped_gemm_pair(rows_block, rows_tail, weight_stack, weight_tail, route, inner, cols, *,
                      out_dtype="float32", transpose_right=False):
    """out[offsets[e]:offsets[e+1]] = rows_block[..] @ op(W_e) + rows_tail[..] @ op(Wtail_e)
    in one launch and one accumulator (qutai_amd_gemm_grouped_pair): the two
    products of grouped_gemm summed over K = 2 * inner without an fp32
    partial in between; inner a multiple of 64."""
    experts = route["experts"]
    for block, stack in ((rows_block, weight_stack), (rows_tail, weight_tail)):
        if stack.size != experts * cols * inner or block.dtype != stack.dtype or block.dtype != rows_block.dtype:
            raise ValueError("grouped_gemm_pair needs [experts] weights of cols*inner values in the rows' dtype")
        if block.size != route["capacity"] * inner:
            raise ValueError("grouped_gemm_pair rows must be capacity x inner")
    if inner % 64:
        raise ValueError("grouped_gemm_pair joins its two halves at a multiple of 64")
    out = AMDStorage(route["capacity"] * cols, out_dtype)
    if out.size:
        out.runtime.call("qutai_amd_gemm_grouped_pair", rows_block.ptr, rows_tail.ptr, weight_stack.ptr,
                         weight_tail.ptr, out.ptr, route["offsets"].ptr, experts, route["capacity"], inner, cols,
                         cols * inner, int(transpose_right), code(rows_block.dtype), code(out_dtype), 0, mfma=True)
    return out


def swiglu_gemm(rows_block, w_gate, w_up, rows, inner, hidden, *, route=None, save=False, gather=False):
    """silu(rows_block @ W_gate^T) * (rows_block @ W_up^T) in one bf16 GEMM
    (qutai_amd_gemm_swiglu), with the unfused form's roundings.  With
    ``route`` the rows are grouped by expert and W_* are [experts][hidden][inner]
    stacks; without, one [hidden][inner] weight pair and ``rows`` rows.  With
    ``gather`` (grouped only) rows_block is the token matrix and the routed
    rows are read through ``order`` inside the GEMM.  With ``save`` the bf16
    gate and up products are returned too (for the backward): (act, gate, up)."""
    if route is not None:
        rows, groups = route["capacity"], route["experts"]
    elif gather:
        raise ValueError("swiglu_gemm gathers rows only for a route")
    else:
        groups = 1
    source = route["rows"] if gather else rows
    if rows_block.dtype != "bfloat16" or {w_gate.dtype, w_up.dtype} != {"bfloat16"}:
        raise ValueError("swiglu_gemm runs bf16 operands")
    if rows_block.size != source * inner or w_gate.size != groups * hidden * inner or w_up.size != w_gate.size:
        raise ValueError("swiglu_gemm operand sizes do not match rows, inner and hidden")
    act = AMDStorage(rows * hidden, "bfloat16")
    gate = AMDStorage(rows * hidden, "bfloat16") if save else None
    up = AMDStorage(rows * hidden, "bfloat16") if save else None
    if act.size:
        act.runtime.call("qutai_amd_gemm_swiglu", rows_block.ptr, w_gate.ptr, w_up.ptr, act.ptr,
                         gate.ptr if save else None, up.ptr if save else None,
                         route["offsets"].ptr if route is not None else None, groups, rows, inner, hidden,
                         hidden * inner, code("bfloat16"), route["order"].ptr if gather else None,
                         source if gather else 0, mfma=True)
    return (act, gate, up) if save else act


def grouped_gemm_k(a_block, b_block, route, rows, cols, *, out_dtype="float32", gather=False):
    """out[e] = A_e^T B_e for every expert, A_e / B_e the expert-major routed
    rows of a_block ([capacity][rows]) and b_block ([capacity][cols]): the
    per-expert weight gradients in one launch (an expert with no rows gets
    zeros).  With ``gather`` b_block is the token matrix ([route rows][cols])
    and B_e's rows are read through the route's ``order`` inside the GEMM."""
    experts = route["experts"]
    b_rows = route["rows"] if gather else route["capacity"]
    if a_block.dtype != b_block.dtype or a_block.size != route["capacity"] * rows or b_block.size != b_rows * cols:
        raise ValueError("grouped_gemm_k needs [capacity][rows] and [capacity][cols] (gathered: [tokens][cols]) "
                         "blocks of one dtype")
    out = AMDStorage(experts * rows * cols, out_dtype)
    if out.size:
        out.runtime.call("qutai_amd_gemm_grouped_k", a_block.ptr, b_block.ptr, out.ptr, route["offsets"].ptr, experts,
                         rows, cols, route["capacity"], code(a_block.dtype), code(out_dtype), 0,
                         route["order"].ptr if gather else None, b_rows if gather else 0, mfma=True)
    return out


def _as_dtype(values, dtype):
    return values if values.dtype == dtype else amd.from_storage(values, dtype=dtype)


def repitch(values, batches, rows, cols, new_rows, new_cols):
    """[batches][rows][cols] -> [batches][new_rows][new_cols], zero padded or cropped."""
    if values.size != batches * rows * cols:
        raise ValueError("repitch source size does not match its shape")
    out = AMDStorage(batches * new_rows * new_cols, values.dtype)
    if out.size:
        out.runtime.call("qutai_amd_repitch", values.ptr, out.ptr, batches, rows, cols, new_rows, new_cols,
                         code(values.dtype))
    return out


def _pad8(n):
    return (n + 7) // 8 * 8


def _rows_through_order(token_bytes, *, dtype):
    """Whether the expert products read the routed token rows through the
    route's ``order`` inside the grouped GEMMs (the forward's gate/up and,
    in training, the backward's dW_gate / dW_up) instead of copying them:
    bf16 or fp32 tokens and a token matrix below 2 GiB (the GEMMs address it
    with 32-bit byte offsets of one buffer descriptor)."""
    return dtype in ("bfloat16", "float32") and token_bytes < (1 << 31)


def moe_experts_forward(x, route, w_gate, w_up, w_down, width, hidden, *, save=False):
    """Expert SwiGLU for every routed (token, slot): gather, grouped gate/up
    and silu(gate) * up (one fused grouped GEMM for bf16, same roundings),
    grouped down, weighted combine (lm/layers.py:395-399).
    Weights of another dtype than x (fp32 master weights, bf16 activations)
    are rounded to x's dtype for the products, as the reference's mixed GEMM
    does.  Widths that are not multiples of 8 run zero padded to the next
    multiple (padded weight rows and columns are zero, so the padded outputs
    are zero and the cropped result is exact).  With ``save`` the
    intermediates for ``moe_experts_backward`` are returned too."""
    wp, hp = _pad8(width), _pad8(hidden)
    experts = route["experts"]
    wg, wu, wd = (_as_dtype(w, x.dtype) for w in (w_gate, w_up, w_down))
    fused = _rows_through_order(x.nbytes, dtype=x.dtype)
    rows = x if fused else route_gather_all(x, route, width)
    if (wp, hp) != (width, hidden):
        wg, wu = (repitch(w, experts, hidden, width, hp, wp) for w in (wg, wu))
        wd = repitch(wd, experts, width, hidden, wp, hp)
        rows = repitch(rows, 1, route["rows"] if fused else route["capacity"], width,
                       route["rows"] if fused else route["capacity"], wp)
    if x.dtype == "bfloat16" and save:
        act, gate, up = swiglu_gemm(rows, wg, wu, 0, wp, hp, route=route, save=True, gather=fused)
    elif x.dtype == "bfloat16":
        act, gate, up = swiglu_gemm(rows, wg, wu, 0, wp, hp, route=route, gather=fused), None, None
    else:
        gate = grouped_gemm(rows, wg, route, wp, hp, out_dtype=x.dtype, gather=fused)
        up = grouped_gemm(rows, wu, route, wp, hp, out_dtype=x.dtype, gather=fused)
        act = silu_mul(gate, up)
    down = grouped_gemm(act, wd, route, hp, wp, out_dtype=x.dtype)
    if wp != width:
        down = repitch(down, 1, route["capacity"], wp, route["capacity"], width)
    y = combine_all(down, route, width)
    if not save:
        return y
    # rows: the (padded) token matrix when the products read it through the
    # route's order (gathered), else the expert-major routed copy
    return y, dict(rows=rows, gathered=fused, gate=gate, up=up, act=act, down=down, w_gate=wg, w_up=wu, w_down=wd)


def combine_backward_all(gradient, expert_rows, route, width):
    """(d expert rows [capacity][width], d weights [rows*top_k] fp32) of
    combine_all, one launch for every (token, slot)."""
    d_rows = AMDStorage(expert_rows.size, expert_rows.dtype)
    d_weights = AMDStorage(route["capacity"], "float32")
    if route["capacity"]:
        d_rows.runtime.call("qutai_amd_combine_backward", gradient.ptr, expert_rows.ptr, route["weights"].ptr,
                            route["indices"].ptr, route["locations"].ptr, route["offsets"].ptr, d_rows.ptr,
                            d_weights.ptr, route["rows"], width, route["top_k"], code(expert_rows.dtype))
    return d_rows, d_weights


def combine_backward(gradient, outputs, weights, route, width):
    """Reference-shaped combine backward (cuda_lm.py:544-581): per-expert row
    gradients in the order of ``outputs``, then the weight gradient."""
    if weights is not route["weights"]:
        route = dict(route, weights=weights)
    dtype = outputs[0][1].dtype if outputs else gradient.dtype
    block = AMDStorage(route["capacity"] * width, dtype)
    starts = _host_offsets(route)
    item = 2 if dtype == "bfloat16" else 4
    for expert, values in outputs:
        if values.size:
            block.runtime.copy(block.ptr + starts[expert] * width * item, values.ptr, values.nbytes)
    d_block, d_weights = combine_backward_all(_as_dtype(gradient, dtype), block, route, width)
    grads = []
    for expert, values in outputs:
        part = AMDStorage(values.size, dtype)
        if values.size:
            part.runtime.copy(part.ptr, d_block.ptr + starts[expert] * width * item, values.nbytes)
        grads.append(part)
    return (*grads, d_weights)


def route_gather_backward_all(d_rows, route, width, *, out_dtype=None):
    """Token-row gradient of route_gather_all: the sum over each token's
    slots of its expert-major rows (fp32 sum, one rounding to out_dtype:
    the rows' dtype, or bf16 from fp32 rows)."""
    out_dtype = d_rows.dtype if out_dtype is None else out_dtype
    out = AMDStorage(route["rows"] * width, out_dtype)
    if out.size:
        out.runtime.call("qutai_amd_combine", d_rows.ptr, None, route["indices"].ptr, route["locations"].ptr,
                         route["offsets"].ptr, out.ptr, route["rows"], width, route["top_k"], code(d_rows.dtype),
                         code(out_dtype))
    return out


def routing_backward(gradient, route, auxiliary=False):
    """Gradient of the router logits (cuda_lm.routing_backward,
    cuda_lm.py:452-467): from the routing weights' gradient [rows*top_k], or
    with ``auxiliary`` from the aux loss's scalar gradient."""
    rows, experts = route["rows"], route["experts"]
    g = _as_dtype(gradient, "float32")
    if g.size != (1 if auxiliary else rows * route["top_k"]):
        raise ValueError("routing_backward: gradient size does not match the route")
    out = AMDStorage(rows * experts, "float32")
    if rows:
        out.runtime.call("qutai_amd_route_backward", g.ptr, route["probs"].ptr, route["weights"].ptr,
                         route["indices"].ptr, route["utilization"].ptr, out.ptr, rows, experts, route["top_k"],
                         int(bool(auxiliary)))
    return out


def moe_experts_backward(gradient, route, saved, width, hidden, *, x_dtype, weight_dtype):
    """Backward of moe_experts_forward: (dx, d routing weights, dW_gate,
    dW_up, dW_down).  Every product is one grouped launch over all experts
    (NN for the data gradients, grouped-K TN for the weight gradients); the
    token gradient sums each token's slots in fp32 and rounds once.  Padded
    widths as in the forward; weight gradients are cropped back."""
    wp, hp = _pad8(width), _pad8(hidden)
    experts, capacity = route["experts"], route["capacity"]
    dt = saved["down"].dtype
    d_down, d_weights = combine_backward_all(_as_dtype(gradient, dt), saved["down"], route, width)
    if wp != width:
        d_down = repitch(d_down, 1, capacity, width, capacity, wp)
    d_act = grouped_gemm(d_down, saved["w_down"], route, wp, hp, out_dtype=dt, transpose_right=False)
    dw_down = grouped_gemm_k(d_down, saved["act"], route, wp, hp, out_dtype=weight_dtype)
    d_gate, d_up = silu_mul_backward(d_act, saved["gate"], saved["up"])
    if hp % 64 == 0:  # dGate W_gate + dUp W_up in one accumulator
        d_rows = grouped_gemm_pair(d_gate, d_up, saved["w_gate"], saved["w_up"], route, hp, wp)
    else:
        d_rows = grouped_gemm(d_gate, saved["w_gate"], route, hp, wp, out_dtype="float32", transpose_right=False)
        grouped_gemm(d_up, saved["w_up"], route, hp, wp, out_dtype="float32", transpose_right=False, out=d_rows,
                     accumulate=True)
    gathered = saved.get("gathered", False)
    dw_gate = grouped_gemm_k(d_gate, saved["rows"], route, hp, wp, out_dtype=weight_dtype, gather=gathered)
    dw_up = grouped_gemm_k(d_up, saved["rows"], route, hp, wp, out_dtype=weight_dtype, gather=gathered)
    if (wp, hp) != (width, hidden):
        d_rows = repitch(d_rows, 1, capacity, wp, capacity, width)
        dw_gate, dw_up = (repitch(w, experts, hp, wp, hidden, width) for w in (dw_gate, dw_up))
        dw_down = repitch(dw_down, experts, wp, hp, width, hidden)
    if x_dtype == "bfloat16":  # fp32 slot sums rounded once, straight to bf16
        dx = route_gather_backward_all(d_rows, route, width, out_dtype="bfloat16")
    else:
        dx = _as_dtype(route_gather_backward_all(d_rows, route, width), x_dtype)
    return dx, d_weights, dw_gate, dw_up, dw_down


def _check_attention(q, k, v, batch, time, heads, kv_heads, dim):
    if len({q.dtype, k.dtype, v.dtype}) != 1 or q.dtype not in ("bfloat16", "float32"):
        raise ValueError("attention takes q, k, v of one dtype, bfloat16 or float32")
    if not 0 < dim <= 256 or kv_heads <= 0 or heads % kv_heads:
        raise ValueError("attention needs 0 < head dimension <= 256 and heads divisible by kv_heads")
    if q.size != batch * time * heads * dim or k.size != batch * time * kv_heads * dim or v.size != k.size:
        raise ValueError("q/k/v sizes do not match (batch, time, heads, dim)")


def attention(q, k, v, batch, time, heads, kv_heads, dim, *, causal=True, layout=1, scale=None):
    """Attention forward (cuda_lm.attention, src/qutai/backends/cuda_lm.py:229-275):
    (out, lse float32).  bf16 q/k/v with head dimension 64 run the fused MFMA
    kernel; other head dimensions (<= 256) and float32 storage run the
    one-wave-per-row kernel, as the reference falls back to its warp kernel.
    layout 1 is the lm layout [batch][time][heads][dim], layout 0 the nn
    layout [batch][heads][time][dim].  The score matrix is never stored."""
    _check_attention(q, k, v, batch, time, heads, kv_heads, dim)
    out = AMDStorage(q.size, q.dtype)
    lse = AMDStorage(batch * heads * time, "float32")
    scale = dim ** -0.5 if scale is None else scale
    if q.size:
        out.runtime.call("qutai_amd_attention_fwd", q.ptr, k.ptr, v.ptr, out.ptr, lse.ptr, batch, heads, kv_heads,
                         time, dim, code(q.dtype), layout, float(scale), int(bool(causal)),
                         mfma=q.dtype == "bfloat16" and dim == 64)
    return out, lse


def attention_backward(gradient, q, k, v, out, lse, batch, time, heads, kv_heads, dim, *, causal=True, layout=1,
                       scale=None):
    """(dq, dk, dv) of ``attention`` (cuda_lm.attention_backward,
    src/qutai/backends/cuda_lm.py:278-365): activations and gradient of one
    dtype, float32 lse from the forward (the reference's ValueError rule,
    cuda_lm.py:279-282); deterministic."""
    _check_attention(q, k, v, batch, time, heads, kv_heads, dim)
    if gradient.dtype != q.dtype or out.dtype != q.dtype or lse.dtype != "float32":
        raise ValueError("attention backward needs gradient/out of the activations' dtype and a float32 lse")
    if gradient.size != q.size or out.size != q.size or lse.size != batch * time * heads:
        raise ValueError("gradient/out/lse sizes do not match (batch, time, heads, dim)")
    dq, dk, dv = AMDStorage(q.size, q.dtype), AMDStorage(k.size, k.dtype), AMDStorage(v.size, v.dtype)
    delta = AMDStorage(lse.size, "float32")
    scale = dim ** -0.5 if scale is None else scale
    if q.size:
        runtime = dq.runtime
        need = runtime.lib.qutai_amd_attention_bwd_workspace_size(batch, heads, kv_heads, time, dim, code(q.dtype))
        workspace = AMDStorage((need + 3) // 4, "float32") if need else None
        runtime.call("qutai_amd_attention_bwd", gradient.ptr, q.ptr, k.ptr, v.ptr, out.ptr, lse.ptr, dq.ptr, dk.ptr,
                     dv.ptr, delta.ptr, workspace.ptr if workspace else None, need, batch, heads, kv_heads, time, dim,
                     code(q.dtype), layout, float(scale), int(bool(causal)), mfma=q.dtype == "bfloat16" and dim == 64)
    return dq, dk, dv


# ---- decoder glue (the rest of a Decoder.loss step) ---------------------------------

def _acc_dtype(dtype):
    """Accumulation dtype of the activations (cuda_lm.py:9-11): fp32 for bf16/fp32."""
    if dtype not in ("bfloat16", "float32"):
        raise ValueError("amd lm kernels take bfloat16 or float32 activations")
    return "float32"


def add_into(target, source):
    """target += source, element-wise in target's dtype (cuda_lm.py:64-73)."""
    if target.dtype != source.dtype or target.size != source.size:
        raise ValueError("add_into needs storages of equal dtype and size")
    if target.size:
        target.runtime.call("qutai_amd_add", target.ptr, source.ptr, target.ptr, target.size, code(target.dtype))


def embedding(weight, ids, width, *, out_dtype=None):
    """Rows of the fp32 embedding table for the host token ids
    (cuda_lm.py:77-93), in out_dtype (default the table's)."""
    dtype = out_dtype or weight.dtype
    if _acc_dtype(dtype) != weight.dtype:
        raise ValueError("the embedding table must be in the activations' accumulation dtype")
    if not (isinstance(ids, array) and ids.typecode == "q"):
        ids = array("q", (int(t) for t in ids))
    result = AMDStorage(len(ids) * width, dtype)
    if result.size:
        identifiers = amd.storage(ids, dtype="int64")
        result.runtime.call("qutai_amd_embedding", weight.ptr, identifiers.ptr, result.ptr, len(ids), width,
                            code(dtype))
    return result


def embedding_backward_index(ids):
    """Device index of the table gradient's row sums: the distinct token ids
    ascending, offsets into the rows, and the rows of each token in input
    order (cuda_lm.py:96-123 groups them the same way on the host).  Built
    with C-level sorts and searches; made once per forward, so the backward
    launches without a host transfer."""
    if not (isinstance(ids, array) and ids.typecode == "q"):
        ids = array("q", (int(t) for t in ids))
    order = sorted(range(len(ids)), key=ids.__getitem__)  # stable: input order within a token
    grouped = array("q", map(ids.__getitem__, order))
    tokens = sorted(set(ids))
    offsets = array("q", map(partial(bisect_left, grouped), tokens))
    offsets.append(len(ids))
    return tuple(amd.storage(values, dtype="int64")
                 for values in (array("q", tokens), offsets, array("q", order)))


def embedding_backward(gradient, ids, count, width, *, index=None, out=None):
    """Table gradient [count][width] (fp32): each token's gradient rows summed
    in input order (cuda_lm.py:96-123).  ``index`` is
    ``embedding_backward_index(ids)`` when the caller made it earlier; with
    ``out`` (an fp32 [count][width] storage) the row sums are added into it in
    place and it is returned."""
    if out is None:
        result = amd.full(count * width, 0.0, dtype=_acc_dtype(gradient.dtype))
    elif out.dtype != "float32" or out.size != count * width:
        raise ValueError("embedding_backward accumulates into an fp32 [count][width] storage")
    else:
        result = out
    if len(ids) and width:
        tokens, offsets, positions = embedding_backward_index(ids) if index is None else index
        result.runtime.call("qutai_amd_embedding_backward", gradient.ptr, tokens.ptr, offsets.ptr, positions.ptr,
                            result.ptr, tokens.size, width, code(gradient.dtype), int(out is not None))
    return result


class EmbeddingRowSums(DeferredGradient):
    """The table gradient of an embedding lookup as a deferred contribution:
    dense on demand, or its rows added in place into a gradient the backward
    pass has just made (a tied embedding/head table), which skips filling a
    [count][width] zero buffer and adding two whole tables."""

    device = "amd"
    dtype = "float32"

    def __init__(self, gradient, ids, count, width, index):
        self.gradient, self.ids, self.count, self.width, self.index = gradient, ids, count, width, index
        self.size = count * width

    def materialize(self):
        return embedding_backward(self.gradient, self.ids, self.count, self.width, index=self.index)

    def add_into(self, storage):
        embedding_backward(self.gradient, self.ids, self.count, self.width, index=self.index, out=storage)


def rms_norm(values, weight, width, eps, *, bf16_copy=False):
    """(out, inverse) of RMSNorm over rows of width (cuda_lm.py:126-145); both
    fp32.  With ``bf16_copy`` also out rounded to bf16 (the copy the bf16
    path's products take), written by the same kernel: (out, inverse, copy)."""
    acc = _acc_dtype(values.dtype)
    if weight.dtype != acc or weight.size != width:
        raise ValueError("rms_norm needs an fp32 weight of width values")
    rows = values.size // width
    out, inverse = AMDStorage(values.size, acc), AMDStorage(rows, acc)
    copy = AMDStorage(values.size, "bfloat16") if bf16_copy else None
    if rows:
        out.runtime.call("qutai_amd_rms_norm_bf16", values.ptr, weight.ptr, out.ptr, None if copy is None else copy.ptr,
                         inverse.ptr, rows, width, float(eps), code(values.dtype))
    return (out, inverse, copy) if bf16_copy else (out, inverse)


def rms_norm_backward(gradient, values, weight, inverse, width, residual=None):
    """(dx in the activation dtype, dweight fp32) (cuda_lm.py:148-177).  With
    ``residual`` (fp32 activations only) dx is residual + dx, added as dx is
    stored: one fp32 rounding, the value of a separate add."""
    rows = values.size // width
    g = gradient if gradient.dtype == "float32" else amd.from_storage(gradient, dtype="float32")
    if residual is not None and (values.dtype != "float32" or residual.dtype != "float32"
                                 or residual.size != values.size):
        raise ValueError("the residual gradient must be fp32 of the activation's size")
    dx, dw = AMDStorage(values.size, values.dtype), AMDStorage(width, weight.dtype)
    if rows:
        runtime = get_runtime()
        partial = AMDStorage(runtime.lib.qutai_amd_rms_norm_workspace(rows, width), "float32")
        runtime.call("qutai_amd_rms_norm_backward", g.ptr, values.ptr, weight.ptr, inverse.ptr,
                     None if residual is None else residual.ptr, dx.ptr, dw.ptr, partial.ptr, rows, width,
                     code(values.dtype))
    elif residual is not None:
        dx = residual.copy()
    return dx, dw


def silu(values):
    """x * sigmoid(x) (cuda_lm.py:180-192)."""
    out = AMDStorage(values.size, values.dtype)
    if values.size:
        out.runtime.call("qutai_amd_silu", values.ptr, None, out.ptr, values.size, 0, code(values.dtype))
    return out


def silu_backward(gradient, values):
    """g * s * (1 + x (1 - s)) (cuda_lm.py:195-207)."""
    out = AMDStorage(values.size, values.dtype)
    if values.size:
        out.runtime.call("qutai_amd_silu", values.ptr, gradient.ptr, out.ptr, values.size, 1, code(values.dtype))
    return out


def rope(values, batch, time, heads, dim, theta, offset=0, inverse=False, *, column=0, row=None, out=None,
         out_column=0, out_row=None):
    """Rotary embedding of [batch][time][heads][dim] (cuda_lm.py:210-226).
    ``values`` may be a wider matrix of ``row`` elements per position whose
    columns column .. column + heads*dim are rotated; the result goes to a new
    contiguous block, or into columns out_column .. of ``out`` (``out_row``
    elements per position)."""
    width = heads * dim
    row = width if row is None else row
    positions = batch * time
    if column < 0 or row < width or column + width > row or values.size < positions * row:
        raise ValueError("rope columns outside the source rows")
    if out is None:
        if out_column or out_row not in (None, width):
            raise ValueError("a new rope result is contiguous")
        out, out_row = AMDStorage(positions * width, values.dtype), width
    else:
        out_row = width if out_row is None else out_row
        if out.dtype != values.dtype or out_column < 0 or out_row < width or out_column + width > out_row \
                or out.size < positions * out_row:
            raise ValueError("rope output columns outside the target rows")
    if positions * width:
        item = _TYPES[values.dtype][1]
        out.runtime.call("qutai_amd_rope_rows", values.ptr + column * item, out.ptr + out_column * item, batch, time,
                         heads, dim, float(theta), offset, int(bool(inverse)), row, out_row, code(values.dtype))
    return out


def copy_rows(source, rows, width, *, column=0, row=None, out=None, out_column=0, out_row=None):
    """Columns column .. column + width of the ``rows`` rows of ``source``
    (``row`` elements each) into a new contiguous [rows][width] block, or into
    columns out_column .. of ``out`` (``out_row`` elements per row)."""
    row = width if row is None else row
    if column < 0 or row < width or column + width > row or source.size < rows * row:
        raise ValueError("copied columns outside the source rows")
    if out is None:
        out, out_column, out_row = AMDStorage(rows * width, source.dtype), 0, width
    else:
        out_row = width if out_row is None else out_row
        if out.dtype != source.dtype or out_column < 0 or out_column + width > out_row or out.size < rows * out_row:
            raise ValueError("copied columns outside the target rows")
    amd._copy_strided(source, out, (rows, width), (row, 1), (out_row, 1), source_offset=column,
                      target_offset=out_column)
    return out


def head_rows(values, start, count, width, time):
    """Rows start .. start+count of the prediction positions (cuda_lm.py:584-598)."""
    result = AMDStorage(count * width, values.dtype)
    if result.size:
        result.runtime.call("qutai_amd_head_rows", values.ptr, result.ptr, count, start, width, time, 0,
                            code(values.dtype))
    return result


def head_rows_backward(target, gradient, start, count, width, time):
    """target[prediction rows] += gradient (cuda_lm.py:601-613)."""
    if count * width:
        target.runtime.call("qutai_amd_head_rows", gradient.ptr, target.ptr, count, start, width, time, 1,
                            code(target.dtype))


def prepare_labels(labels):
    """Labels resident on the device as int64 (cuda_lm.py:616-617)."""
    if not (isinstance(labels, array) and labels.typecode == "q"):
        labels = array("q", (int(x) for x in labels))
    return amd.storage(labels, dtype="int64")


def _head_labels(labels, start, rows):
    ids = labels if isinstance(labels, AMDStorage) else prepare_labels(labels)
    if ids.dtype != "int64" or start < 0 or start + rows > ids.size:
        raise ValueError("invalid head label storage or range")
    return ids, ids.ptr + 8 * start


def head_loss(logits, labels, rows, vocab, *, start=0):
    """Summed cross entropy of rows of logits (label -100 ignored), one fp32
    value (cuda_lm.py:629-643)."""
    _, pointer = _head_labels(labels, start, rows)
    values = AMDStorage(rows, _acc_dtype(logits.dtype))
    if rows:
        values.runtime.call("qutai_amd_head_loss", logits.ptr, pointer, values.ptr, rows, vocab, code(logits.dtype))
    return amd.sum_all(values) if rows else amd.full(1, 0.0, dtype=values.dtype)


def head_block_stats(logits, labels, stats, picked, rows, cols, col0, *, first):
    """Fold one vocabulary block [rows][cols] (columns col0 ..) of the logits
    into the per-row running (max, sum exp) pairs ``stats`` ([rows][2] fp32)
    and the label logits ``picked`` ([rows] fp32)."""
    ids, _ = _head_labels(labels, 0, rows)
    if rows:
        logits.runtime.call("qutai_amd_head_block_stats", logits.ptr, ids.ptr, stats.ptr, picked.ptr, rows, cols, col0,
                            int(first), code(logits.dtype))


def head_block_loss(stats, picked, labels, rows):
    """Summed cross entropy of the rows from their folded stats (one fp32 value)."""
    ids, _ = _head_labels(labels, 0, rows)
    values = AMDStorage(rows, "float32")
    if rows:
        values.runtime.call("qutai_amd_head_block_loss", stats.ptr, picked.ptr, ids.ptr, values.ptr, rows)
    return amd.sum_all(values) if rows else amd.full(1, 0.0, dtype="float32")


def head_block_gradient(logits, labels, stats, gradient, rows, cols, col0, count):
    """In place over one vocabulary block: g / count * (softmax - onehot)."""
    ids, _ = _head_labels(labels, 0, rows)
    g = gradient if gradient.dtype == "float32" else amd.from_storage(gradient, dtype="float32")
    if rows:
        logits.runtime.call("qutai_amd_head_block_gradient", logits.ptr, ids.ptr, stats.ptr, g.ptr, rows, cols, col0,
                            1.0 / count, code(logits.dtype))
    return logits


def head_gradient(logits, labels, rows, vocab, gradient, count, *, start=0):
    """In place: logits = g / count * (softmax - onehot) (cuda_lm.py:646-660)."""
    _, pointer = _head_labels(labels, start, rows)
    g = gradient if gradient.dtype == "float32" else amd.from_storage(gradient, dtype="float32")
    if rows:
        logits.runtime.call("qutai_amd_head_gradient", logits.ptr, pointer, g.ptr, rows, vocab, 1.0 / count,
                            code(logits.dtype))
    return logits
