"""LM layers on the GEMM path (src/qutai/lm/layers.py:9-449, contraction parts).

``linear`` / ``Projection`` / ``SwiGLU`` follow the reference call patterns
(weights stored (out, in), ``Y = X W^T`` forward, ``dX = G W`` and
``dW = G^T X`` backward, precision captured in forward and restored in
backward).  ``SparseMoE`` keeps the reference routing semantics but stores
each projection of all experts as one stacked tensor, so the expert
projections run as grouped GEMMs over device-resident row ranges instead of
a Python loop of per-expert GEMMs.  ``attention_products`` is the score /
value product pair of the attention layers (S = Q K^T, P = softmax(S/sqrt D),
O = P V) on the batched GEMM.
"""
from __future__ import annotations

from array import array
from itertools import chain
from math import prod, sqrt

from ..backends import amd, amd_lm
from ..backends.precision import matmul_precision, set_matmul_precision
from ..core.context import is_recording
from ..core.grad import DeferredGradient, owned, record
from ..core.tensor import Tensor


def backend(value):
    device = value if isinstance(value, str) else value.device
    if device == "amd":
        return amd_lm
    raise ValueError("no LM kernels for this device")


def activation_dtype(x, weight):
    """bf16 activations on the GPU with fp32 weights under autocast or bf16
    inputs (src/qutai/lm/layers.py:20-28)."""
    if weight.dtype == "float32" and (matmul_precision() == "bfloat16" or x.dtype == "bfloat16"):
        return "bfloat16"
    return weight.dtype


def _bf16_path(*operands):
    """True when GEMMs of these operands run on the bf16 MFMA path (a bf16
    operand or autocast), where fp32 operands are rounded to bf16 (RNE)."""
    return matmul_precision() == "bfloat16" or any(o.dtype == "bfloat16" for o in operands)


def _bf16(values):
    return values if values.dtype == "bfloat16" else amd.from_storage(values, dtype="bfloat16")


def _bf16_input(x):
    """x's storage rounded to bf16 for the bf16-path products, made once per
    activation: the q, k and v projections of one normalised input share the
    copy (the rounding is the same each time).  Cached only on tensors made
    by a recorded op, whose storage is never written again."""
    if x.dtype == "bfloat16":
        return x.storage
    if getattr(x, "backward_rule", None) is None:
        return _bf16(x.storage)
    cached = getattr(x, "_bf16_input", None)
    if cached is None or cached[0] is not x.storage:
        cached = (x.storage, _bf16(x.storage))
        x._bf16_input = cached
    return cached[1]


def linear(x, weight):
    """Y = X W^T with W stored (out, in) (src/qutai/lm/layers.py:35-74).  On
    the bf16 path the fp32 operands are rounded to bf16 once here, the same
    rounding the GEMM would apply, and the rounded copies serve the backward
    products too."""
    b = backend(x)
    rows = x.size // x.shape[-1]
    out_features, inner = weight.shape
    precision = matmul_precision()
    xs, ws = x.storage, weight.storage
    if _bf16_path(x, weight):
        xs, ws = _bf16_input(x), _bf16(ws)
    values = b.gemm(xs, ws, rows, inner, out_features, transpose_right=True, out_dtype=activation_dtype(x, weight))

    def backward(g):
        with set_matmul_precision(precision):
            dx = None
            if x.requires_grad:
                dx = (ProductGradient(b, g, ws, rows, out_features, inner, precision) if x.dtype == "float32"
                      else b.gemm(g, ws, rows, out_features, inner, out_dtype=x.dtype))
            dw = (owned(b.gemm(g, xs, out_features, rows, inner, transpose_left=True, out_dtype=weight.dtype))
                  if weight.requires_grad else None)
        return dx, dw

    return record(Tensor(values, shape=(*x.shape[:-1], out_features)), (x, weight), backward)


class ProductGradient(DeferredGradient):
    """A Linear's fp32 input gradient dX = G W (rows x inner from G rows x
    cols and W cols x inner), left for the backward pass to place: alone it
    is one GEMM; when it meets another fp32 contribution to the same input
    (the q, k and v projections of one normalised activation) the GEMM adds
    into that gradient in its epilogue, round(old + product) once, the
    value a separate fp32 add of the product gives, without the add's pass
    over three rows x inner arrays."""

    device, dtype = "amd", "float32"

    def __init__(self, b, g, w, rows, cols, inner, precision):
        self.b, self.g, self.w, self.rows, self.cols, self.inner = b, g, w, rows, cols, inner
        self.precision, self.size = precision, rows * inner

    def materialize(self):
        with set_matmul_precision(self.precision):
            return self.b.gemm(self.g, self.w, self.rows, self.cols, self.inner, out_dtype="float32")

    def add_into(self, storage):
        with set_matmul_precision(self.precision):
            self.b.gemm(self.g, self.w, self.rows, self.cols, self.inner, out_dtype="float32", out=storage,
                        accumulate=True)


def residual_add(x, update):
    """x + update cast to x's dtype (src/qutai/lm/layers.py:31-32).  fp32 x
    with a bf16 update (autocast) adds in one pass; the backward is the
    cast's and the add's: the gradient to x, and rounded to bf16 to update."""
    if x.device == "amd" and x.dtype == "float32" and update.dtype == "bfloat16" and x.shape == update.shape:
        return record(Tensor(amd.add_widen(x.storage, update.storage), shape=x.shape), (x, update),
                      lambda g: (g, amd.from_storage(g, dtype="bfloat16")))
    return x + update.to(dtype=x.dtype)


def scaled(x, factor):
    """x * factor as a recorded op (the scalar products of decoder.py:131, 173)."""
    return record(Tensor(amd.scale(x.storage, factor), shape=x.shape), (x,), lambda g: (amd.scale(g, factor),))


def embed(ids, weight, shape):
    """Rows of the (vocab, width) table for host token ids, shape (*shape,
    width) (src/qutai/lm/layers.py:77-85)."""
    b = backend(weight)
    width = weight.shape[1]
    values = b.embedding(weight.storage, ids, width)
    result = record(Tensor(values, shape=(*shape, width)), (weight,))
    if result.requires_grad:
        # the row grouping goes to the device now, with the ids, so that the
        # backward launches without a host transfer (which would wait for
        # every kernel queued before it)
        index = b.embedding_backward_index(ids)
        result.backward_rule = lambda g: (b.EmbeddingRowSums(g, ids, weight.shape[0], width, index),)
    return result


def rms_norm(x, weight, eps):
    """RMSNorm over the last axis, fp32 output (src/qutai/lm/layers.py:88-96).
    Under autocast the following projections round this output to bf16: the
    norm kernel writes that copy too and it becomes the output's cached bf16
    input (_bf16_input), in place of a separate cast pass."""
    b = backend(x)
    width = x.shape[-1]
    copy = None
    if matmul_precision() == "bfloat16":
        out, inverse, copy = b.rms_norm(x.storage, weight.storage, width, eps, bf16_copy=True)
    else:
        out, inverse = b.rms_norm(x.storage, weight.storage, width, eps)

    def backward(g):
        if x.dtype == "float32" and x.requires_grad:
            state = NormBackward(b, g, x.storage, weight.storage, inverse, width)
            return NormInputGradient(state), NormWeightGradient(state)
        dx, dweight = b.rms_norm_backward(g, x.storage, weight.storage, inverse, width)
        return dx, owned(dweight)

    result = record(Tensor(out, shape=x.shape), (x, weight), backward)
    if copy is not None:
        result._bf16_input = (out, copy)
    return result


class NormBackward:
    """One RMSNorm backward kernel call (dx and dweight together), run when
    the pass first asks for either: for dx summed with the residual stream's
    gradient (the norm's input is also the residual connection's), the
    kernel adds that gradient as it stores dx, the fp32 add's value without
    the add's pass over three rows x width arrays."""

    def __init__(self, b, g, x, weight, inverse, width):
        self.args, self.dx, self.dweight = (b, g, x, weight, inverse, width), None, None

    def run(self, residual=None):
        b, g, x, weight, inverse, width = self.args
        self.dx, self.dweight = b.rms_norm_backward(g, x, weight, inverse, width, residual=residual)
        self.args = None
        return self.dx


class NormInputGradient(DeferredGradient):
    device, dtype = "amd", "float32"

    def __init__(self, state):
        self.state, self.size = state, state.args[2].size

    def materialize(self):
        return self.state.run()

    def add_into(self, storage):
        amd_lm.add_into(storage, self.state.run())

    def sum_with(self, existing, in_place):
        return self.state.run(existing)


class NormWeightGradient(DeferredGradient):
    device = "amd"

    def __init__(self, state):
        self.state, self.size, self.dtype = state, state.args[3].size, state.args[3].dtype

    def _get(self):
        if self.state.dweight is None:
            self.state.run()
        return self.state.dweight

    def materialize(self):
        return owned(self._get())

    def add_into(self, storage):
        amd_lm.add_into(storage, self._get())


def rope(x, heads, theta, offset=0):
    """Rotary position embedding of (batch, time, heads*dim); backward is the
    inverse rotation (src/qutai/lm/layers.py:108-116)."""
    b = backend(x)
    batch, time, features = x.shape
    dims = (batch, time, heads, features // heads, theta, offset)
    return record(Tensor(b.rope(x.storage, *dims), shape=x.shape), (x,),
                  lambda g: (b.rope(g, *dims, inverse=True),))


def silu_mul(gate, up):
    """silu(gate) * up as one recorded op (SwiGLU's activation, lm/layers.py:310-311)."""
    b = backend(gate)
    values = b.silu_mul(gate.storage, up.storage)
    return record(Tensor(values, shape=gate.shape), (gate, up),
                  lambda g: b.silu_mul_backward(g, gate.storage, up.storage))


def swiglu(x, w_gate, w_up):
    """silu(x W_gate^T) * (x W_up^T) as one recorded op on the fused bf16 GEMM
    (qutai_amd_gemm_swiglu): the same roundings as ``silu_mul(linear(x,
    w_gate), linear(x, w_up))`` on the bf16 path (x and fp32 weights rounded
    to bf16 once, bf16 gate and up, bf16 silu, one rounding of the product).
    The backward is the unfused one: silu_mul_backward, each projection's
    dX = G W and dW = G^T X, and the two dX summed as autograd sums the
    gradients of a twice-used input (src/qutai/lm/layers.py:35-74, 310-311)."""
    b = backend(x)
    rows = x.size // x.shape[-1]
    hidden, inner = w_gate.shape
    precision = matmul_precision()
    xs, gs, us = _bf16_input(x), _bf16(w_gate.storage), _bf16(w_up.storage)
    act, gate, up = b.swiglu_gemm(xs, gs, us, rows, inner, hidden, save=True)

    def backward(g):
        dgate, dup = b.silu_mul_backward(g, gate, up)
        with set_matmul_precision(precision):
            dx = None
            if x.requires_grad:
                dx = b.gemm(dgate, gs, rows, hidden, inner, out_dtype=x.dtype)
                if x.dtype == "float32":  # round(old + product) once: the fp32 add's value
                    b.gemm(dup, us, rows, hidden, inner, out_dtype=x.dtype, out=dx, accumulate=True)
                else:
                    dx = amd.add(dx, b.gemm(dup, us, rows, hidden, inner, out_dtype=x.dtype))
            dwg = (owned(b.gemm(dgate, xs, hidden, rows, inner, transpose_left=True, out_dtype=w_gate.dtype))
                   if w_gate.requires_grad else None)
            dwu = (owned(b.gemm(dup, xs, hidden, rows, inner, transpose_left=True, out_dtype=w_up.dtype))
                   if w_up.requires_grad else None)
        return dx, dwg, dwu

    return record(Tensor(act, shape=(*x.shape[:-1], hidden)), (x, w_gate, w_up), backward)


def _swiglu_fusable(x, w_gate, w_up):
    """The fused GEMM covers bf16-path products with bf16 activations and
    16-byte rows (inner a multiple of 8)."""
    return (x.device == "amd" and w_gate.dtype == w_up.dtype and w_gate.shape == w_up.shape
            and _bf16_path(x, w_gate, w_up) and activation_dtype(x, w_gate) == "bfloat16"
            and x.shape[-1] % 8 == 0)


class Projection:
    def __init__(self, inputs, outputs, *, device="amd", dtype="float32", seed=None, std=0.02):
        self.weight = Tensor(backend(device).normal(inputs * outputs, std=std, seed=seed, dtype=dtype),
                             shape=(outputs, inputs), requires_grad=True)

    def __call__(self, x):
        return linear(x, self.weight)

    def parameters(self):
        return (self.weight,)


class SwiGLU:
    """down(silu(gate(x)) * up(x)); seeds seed, seed+1, seed+2 (lm/layers.py:291-314)."""

    def __init__(self, width, hidden, *, device="amd", dtype="float32", seed=None, std=0.02):
        self.gate = Projection(width, hidden, device=device, dtype=dtype, seed=seed)
        self.up = Projection(width, hidden, device=device, dtype=dtype, seed=None if seed is None else seed + 1)
        self.down = Projection(hidden, width, device=device, dtype=dtype, seed=None if seed is None else seed + 2,
                               std=std)

    def __call__(self, x):
        if _swiglu_fusable(x, self.gate.weight, self.up.weight):
            return self.down(swiglu(x, self.gate.weight, self.up.weight))
        return self.down(silu_mul(self.gate(x), self.up(x)))

    def parameters(self):
        return (*self.gate.parameters(), *self.up.parameters(), *self.down.parameters())


class SparseMoE:
    """Top-k routed SwiGLU experts (lm/layers.py:353-406).

    Expert e's gate/up weights are ``w_gate[e]`` / ``w_up[e]`` (hidden, width)
    and its down weight ``w_down[e]`` (width, hidden); expert e is initialised
    from seeds seed+1+3e, +1, +2 like the reference's per-expert SwiGLU."""

    def __init__(self, width, hidden, experts, top_k, *, device="amd", dtype="float32", seed=None, std=0.02):
        self.router = Projection(width, experts, device=device, dtype=dtype, seed=seed)
        self.width, self.hidden, self.n_experts, self.top_k = width, hidden, experts, top_k
        b = backend(device)

        def stacked(rows, cols, offset, scale):
            parts = [b.normal(rows * cols, std=scale, seed=None if seed is None else seed + 1 + 3 * e + offset,
                              dtype=dtype) for e in range(experts)]
            block = amd.AMDStorage(experts * rows * cols, dtype)
            item = 2 if dtype == "bfloat16" else 4
            for e, part in enumerate(parts):
                block.runtime.copy(block.ptr + e * rows * cols * item, part.ptr, part.nbytes)
            return Tensor(block, shape=(experts, rows, cols), requires_grad=True)

        self.w_gate = stacked(hidden, width, 0, 0.02)
        self.w_up = stacked(hidden, width, 1, 0.02)
        self.w_down = stacked(width, hidden, 2, std)
        self.utilization = None

    def __call__(self, x):
        """(result, aux) like the reference (lm/layers.py:376-402); every
        expert runs in one grouped launch per projection, forward and
        backward, with no host synchronisation.  ``last_route`` keeps the
        routing arrays of the call."""
        with set_matmul_precision(None):
            scores = self.router(x.to(dtype=self.router.weight.dtype))
        b = backend(x)
        rows = x.size // x.shape[-1]
        route = b.routing(scores.storage, rows, self.n_experts, self.top_k, download_counts=False)
        self.last_route = route
        weights = record(Tensor(route["weights"], shape=(rows, self.top_k)), (scores,),
                         lambda g: (b.routing_backward(g, route),))
        aux = record(Tensor(route["aux"], shape=()), (scores,), lambda g: (b.routing_backward(g, route, True),))
        self.utilization = Tensor(route["utilization"], shape=(self.n_experts,))
        values, saved = b.moe_experts_forward(x.storage, route, self.w_gate.storage, self.w_up.storage,
                                              self.w_down.storage, self.width, self.hidden, save=True)
        if x.dtype != values.dtype:
            values = amd.from_storage(values, dtype=x.dtype)
        weight_dtype = self.w_gate.dtype

        def backward(g):
            dx, dw, dwg, dwu, dwd = b.moe_experts_backward(g, route, saved, self.width, self.hidden,
                                                           x_dtype=x.dtype, weight_dtype=weight_dtype)
            # every one is a storage this backward just made (dx: the routed
            # rows summed back into token order)
            return owned(dx), dw, owned(dwg), owned(dwu), owned(dwd)

        result = record(Tensor(values, shape=x.shape), (x, weights, self.w_gate, self.w_up, self.w_down), backward)
        return result, aux

    @property
    def last_counts(self):
        """Per-expert token counts of the last call (one device read)."""
        route = getattr(self, "last_route", None)
        if route is None:
            return (0,) * self.n_experts
        return tuple(route["count_buffer"].to_array().tolist())

    def parameters(self):
        return (*self.router.parameters(), self.w_gate, self.w_up, self.w_down)


class RMSNorm:
    """Unit-initialised RMSNorm weight (src/qutai/lm/layers.py:275-288)."""

    def __init__(self, width, eps, *, device="amd", dtype="float32"):
        self.weight = Tensor(amd.full(width, 1.0, dtype=dtype), shape=(width,), requires_grad=True)
        self.eps = eps

    def __call__(self, x):
        return rms_norm(x, self.weight, self.eps)

    def parameters(self):
        return (self.weight,)


class GQA:
    """Grouped-query attention block: q/k/v projections (seeds seed..seed+2),
    RoPE on q and k, fused causal attention, out projection (seed+3, std
    0.02/sqrt(2 n_layers)) (src/qutai/lm/layers.py:317-350)."""

    def __init__(self, config, *, device="amd", dtype="float32", seed=None):
        width = config.d_model
        kv_width = config.n_kv_heads * (width // config.n_heads)

        def offset(i):
            return None if seed is None else seed + i

        self.q = Projection(width, width, device=device, dtype=dtype, seed=seed)
        self.k = Projection(width, kv_width, device=device, dtype=dtype, seed=offset(1))
        self.v = Projection(width, kv_width, device=device, dtype=dtype, seed=offset(2))
        self.out = Projection(width, width, device=device, dtype=dtype, seed=offset(3),
                              std=0.02 / sqrt(2 * config.n_layers))
        self.heads, self.kv_heads, self.theta = config.n_heads, config.n_kv_heads, config.rope_theta

    def __call__(self, x):
        weights = (self.q.weight, self.k.weight, self.v.weight)
        if _stacked_qkv(x, *weights):
            return self.out(gqa_attention(x, *weights, self.heads, self.kv_heads, self.theta))
        q = rope(self.q(x), self.heads, self.theta)
        k = rope(self.k(x), self.kv_heads, self.theta)
        return self.out(attention(q, k, self.v(x), self.heads, self.kv_heads))

    def parameters(self):
        return (*self.q.parameters(), *self.k.parameters(), *self.v.parameters(), *self.out.parameters())


class Block:
    """Pre-norm decoder block: x + attn(norm(x)), then x + ffn(norm(x)); the
    FFN is SwiGLU or SparseMoE (seed+4); returns (hidden, aux)
    (src/qutai/lm/layers.py:409-446)."""

    def __init__(self, config, *, device="amd", dtype="float32", seed=None):
        self.attn_norm = RMSNorm(config.d_model, config.norm_eps, device=device, dtype=dtype)
        self.ffn_norm = RMSNorm(config.d_model, config.norm_eps, device=device, dtype=dtype)
        self.attn = GQA(config, device=device, dtype=dtype, seed=seed)
        self.is_moe = config.ffn_type == "moe"
        ffn_seed = None if seed is None else seed + 4
        down_std = 0.02 / sqrt(2 * config.n_layers)
        if self.is_moe:
            self.ffn = SparseMoE(config.d_model, config.d_expert, config.n_experts, config.top_k, device=device,
                                 dtype=dtype, seed=ffn_seed, std=down_std)
        else:
            self.ffn = SwiGLU(config.d_model, config.d_ff, device=device, dtype=dtype, seed=ffn_seed, std=down_std)

    def __call__(self, x):
        x = residual_add(x, self.attn(self.attn_norm(x)))
        if self.is_moe:
            y, aux = self.ffn(self.ffn_norm(x))
        else:
            y = self.ffn(self.ffn_norm(x))
            aux = Tensor(amd.full(1, 0.0, dtype=x.dtype), shape=())
        return residual_add(x, y), aux

    def hidden(self, x):
        return self(x)[0]

    def packed(self, x):
        return pack(*self(x))

    def parameters(self):
        return (*self.attn_norm.parameters(), *self.ffn_norm.parameters(), *self.attn.parameters(),
                *self.ffn.parameters())


def pack(hidden, aux):
    """hidden and its scalar aux loss as one flat tensor, so that a recomputed
    MoE block has one output (src/qutai/lm/layers.py:161-169)."""
    values = amd.concatenate((hidden.storage, aux.to(dtype=hidden.dtype).storage), ((hidden.size,), (1,)))
    size = hidden.size
    return record(Tensor(values, shape=(size + 1,)), (hidden, aux),
                  lambda g: (amd.take(g, 0, size), _cast(amd.take(g, size, 1), aux.dtype)))


def unpack(packed, shape):
    """Inverse of ``pack`` (src/qutai/lm/layers.py:172-191)."""
    size = prod(shape)
    hidden = record(Tensor(amd.take(packed.storage, 0, size), shape=shape), (packed,),
                    lambda g: (amd.concatenate((g, amd.full(1, 0.0, dtype=g.dtype)), ((size,), (1,))),))
    aux = record(Tensor(amd.take(packed.storage, size, 1), shape=()), (packed,),
                 lambda g: (amd.concatenate((amd.full(size, 0.0, dtype=g.dtype), g), ((size,), (1,))),))
    return hidden, aux


def _cast(values, dtype):
    return values if values.dtype == dtype else amd.from_storage(values, dtype=dtype)


def vocab_block(chunk_size, rows, vocab):
    """Vocabulary columns per block of the loss head: the most that keep a
    block's logits within chunk_size x vocab values (the reference's bound
    for one chunk of rows), a multiple of 8 (16-byte rows), at least 8."""
    if rows <= chunk_size:
        return vocab
    return min(vocab, max(8, (chunk_size * vocab // rows) // 8 * 8))


KEEP_LOGITS_BYTES = 2 << 30
KEEP_LOGITS_CHUNKS = 4


def projection_loss(hidden, weight, labels, chunk_size, *, prepared_labels=None, keep_logits=None):
    """Mean next-token cross entropy of hidden (batch, time, width) against
    the tied (vocab, width) weight; labels -100 are ignored
    (src/qutai/lm/layers.py:194-257).  As in the reference at most
    chunk_size x vocab logits exist at once, but the blocks are cut along the
    vocabulary instead of the rows: every block holds all prediction rows
    for a range of vocabulary columns, the forward folds each row's running
    (max, sum exp) over the blocks, and the backward recomputes a block's
    logits, turns them into the softmax gradient and writes that block's rows
    of the weight gradient with one GEMM over all rows (no read-modify-write
    of the whole gradient per chunk), while dX accumulates in fp32.

    With ``keep_logits`` (default: when the rows are at most
    KEEP_LOGITS_CHUNKS x chunk_size -- the caller's chunk still bounds the
    memory, to that factor -- and all rows x vocab logits fit
    KEEP_LOGITS_BYTES) and a backward to follow, the forward's blocks are
    kept and the first backward turns them into the gradient in place instead
    of recomputing them (the same values: the GEMM is deterministic); the
    graph holds them until then, and a second backward over a retained graph
    recomputes.  ``keep_logits=False`` restores the reference's bound of
    chunk_size x vocab logits.  The config-4 head (4096 rows, chunk 1024)
    keeps 268 MB and skips four 137-GFLOP GEMMs."""
    b = backend(hidden)
    _, time, width = hidden.shape
    vocab = weight.shape[0]
    precision = matmul_precision()
    try:  # C-level conversion of integer labels
        targets = array("q", chain.from_iterable(row[1:] for row in labels))
    except TypeError:
        targets = array("q", (int(label) for row in labels for label in row[1:]))
    label_data = b.prepare_labels(targets) if prepared_labels is None else prepared_labels
    rows = len(targets)
    count = max(1, rows - targets.count(-100))
    out_dtype = activation_dtype(hidden, weight)
    hs, ws = hidden.storage, weight.storage
    if _bf16_path(hidden, weight):  # round once, not once per block and product
        hs, ws = _bf16(hs), _bf16(ws)
    block = vocab_block(chunk_size, rows, vocab)
    inputs = b.head_rows(hs, 0, rows, width, time)
    stats = amd.AMDStorage(2 * rows, "float32")
    picked = amd.AMDStorage(rows, "float32")

    def block_logits(c0, cols):
        return b.gemm(inputs, amd.view(ws, c0 * width, cols * width), rows, width, cols, transpose_right=True,
                      out_dtype=out_dtype)

    esize = 2 if out_dtype == "bfloat16" else 4
    if keep_logits is None:
        keep_logits = rows <= KEEP_LOGITS_CHUNKS * chunk_size and rows * vocab * esize <= KEEP_LOGITS_BYTES
    keep = is_recording() and (hidden.requires_grad or weight.requires_grad) and bool(keep_logits)
    kept = {}
    for c0 in range(0, vocab, block):
        cols = min(block, vocab - c0)
        logits = block_logits(c0, cols)
        b.head_block_stats(logits, label_data, stats, picked, rows, cols, c0, first=c0 == 0)
        if keep:
            kept[c0] = logits
    result = amd.scale(_cast(b.head_block_loss(stats, picked, label_data, rows), hidden.dtype), 1 / count)

    def backward(gradient):
        with set_matmul_precision(precision):
            dw = amd.AMDStorage(weight.size, weight.dtype) if weight.requires_grad else None
            part = None  # dX of the prediction rows, fp32, summed over the blocks
            for c0 in range(0, vocab, block):
                cols = min(block, vocab - c0)
                logits = kept.pop(c0, None)  # overwritten in place: a second backward recomputes
                if logits is None:
                    logits = block_logits(c0, cols)
                incoming = b.head_block_gradient(logits, label_data, stats, gradient, rows, cols, c0, count)
                if weight.requires_grad:
                    b.gemm(incoming, inputs, cols, rows, width, transpose_left=True, out_dtype=weight.dtype,
                           out=amd.view(dw, c0 * width, cols * width))
                if hidden.requires_grad:
                    w_block = amd.view(ws, c0 * width, cols * width)
                    if part is None:
                        part = b.gemm(incoming, w_block, rows, cols, width, out_dtype="float32")
                    else:
                        b.gemm(incoming, w_block, rows, cols, width, out_dtype="float32", out=part, accumulate=True)
            dx = None
            if hidden.requires_grad:
                dx = amd.full(hidden.size, 0.0, dtype=hidden.dtype)
                if part is not None:
                    b.head_rows_backward(dx, _cast(part, hidden.dtype), 0, rows, width, time)
            return dx, owned(dw)

    return record(Tensor(result, shape=()), (hidden, weight), backward)


def attention_products(q, k, v, *, scale=None):
    """Score and value products of attention on (groups, T, D) tensors:
    S = Q K^T (NT, no materialised K^T), P = softmax(scale * S) row-wise,
    O = P V (NN); fp32 accumulation in both GEMMs, storage dtype kept
    (src/qutai/nn/layers.py:334-354)."""
    if q.shape != k.shape or q.shape != v.shape or q.ndim != 3:
        raise ValueError("attention_products takes equal (groups, T, D) q, k, v")
    groups, time, dim = q.shape
    scale = 1 / sqrt(dim) if scale is None else scale
    scores = amd.gemm(q.storage, k.storage, time, dim, time, batch=groups, transpose_right=True,
                      out_dtype=q.dtype)
    probs = amd.softmax(scores, (groups * time, time), -1, scale=scale)
    out = amd.gemm(probs, v.storage, time, time, dim, batch=groups, out_dtype=q.dtype)
    return Tensor(out, shape=(groups, time, dim)), Tensor(probs, shape=(groups, time, time))


def attention(q, k, v, heads, kv_heads):
    """Causal grouped-query attention on (batch, time, heads*64) tensors in the
    lm layout (src/qutai/lm/layers.py:119-130): fused forward (the T x T
    scores are never stored) and fused backward recorded for autograd."""
    b = backend(q)
    batch, time, features = q.shape
    dims = (batch, time, heads, kv_heads, features // heads)
    out, lse = b.attention(q.storage, k.storage, v.storage, *dims)
    return record(Tensor(out, shape=q.shape), (q, k, v),
                  lambda g: b.attention_backward(g, q.storage, k.storage, v.storage, out, lse, *dims))


def _stacked_qkv(x, wq, wk, wv):
    """True when GQA's three projections can run as one GEMM: amd tensors on
    the bf16 path with bf16 projection outputs, one weight dtype."""
    if x.device != "amd" or x.ndim != 3 or any(w.device != "amd" or w.ndim != 2 for w in (wq, wk, wv)):
        return False
    if not (wq.dtype == wk.dtype == wv.dtype) or wk.shape != wv.shape:
        return False
    if wq.shape[1] != x.shape[-1] or wk.shape[1] != x.shape[-1]:
        return False
    return _bf16_path(x, wq) and activation_dtype(x, wq) == "bfloat16"


def gqa_attention(x, wq, wk, wv, heads, kv_heads, theta):
    """RoPE(x Wq^T), RoPE(x Wk^T), x Wv^T and causal grouped-query attention
    as one recorded op: GQA up to its out projection (src/qutai/lm/layers.py:
    317-350 with rope 108-116 and attention 119-130) on the bf16 path.  The
    three projections are one GEMM against the stacked weight [Wq; Wk; Wv]
    (dq + 2 dkv rows, cast to bf16 into one block); RoPE reads the q and k
    columns of that product in place and v's columns are copied out.  The
    backward stacks dq, dk, dv the same way, so the input gradient is one GEMM
    over K = dq + 2 dkv and the weight gradients are the row blocks of one
    GEMM.  The forward values are those of the separate projections (every
    output element sums K in the same order whatever the tile); the input
    gradient sums its three terms in one accumulator where the separate
    projections add three rounded products."""
    b = backend(x)
    batch, time, width = x.shape
    rows = batch * time
    dq, dkv = wq.shape[0], wk.shape[0]
    total = dq + 2 * dkv
    head = dq // heads
    precision = matmul_precision()
    xs = _bf16_input(x)
    ws = amd.AMDStorage(total * width, "bfloat16")
    for w, start in ((wq, 0), (wk, dq), (wv, dq + dkv)):
        amd.cast_into(amd.view(ws, start * width, w.size), w.storage)
    qkv = b.gemm(xs, ws, rows, width, total, transpose_right=True, out_dtype="bfloat16")
    q = b.rope(qkv, batch, time, heads, head, theta, row=total)
    k = b.rope(qkv, batch, time, kv_heads, head, theta, column=dq, row=total)
    v = b.copy_rows(qkv, rows, dkv, column=dq + dkv, row=total)
    del qkv
    dims = (batch, time, heads, kv_heads, head)
    out, lse = b.attention(q, k, v, *dims)

    def backward(g):
        with set_matmul_precision(precision):
            gq, gk, gv = b.attention_backward(g, q, k, v, out, lse, *dims)
            d = amd.AMDStorage(rows * total, gq.dtype)
            b.rope(gq, batch, time, heads, head, theta, inverse=True, out=d, out_row=total)
            b.rope(gk, batch, time, kv_heads, head, theta, inverse=True, out=d, out_column=dq, out_row=total)
            b.copy_rows(gv, rows, dkv, out=d, out_column=dq + dkv, out_row=total)
            dx = None
            if x.requires_grad:
                dx = (ProductGradient(b, d, ws, rows, total, width, precision) if x.dtype == "float32"
                      else b.gemm(d, ws, rows, total, width, out_dtype=x.dtype))
            dws = (None, None, None)
            if wq.requires_grad or wk.requires_grad or wv.requires_grad:
                dw = b.gemm(d, xs, total, rows, width, transpose_left=True, out_dtype=wq.dtype)
                dws = tuple(owned(amd.view(dw, start * width, w.size)) if w.requires_grad else None
                            for w, start in ((wq, 0), (wk, dq), (wv, dq + dkv)))
        return (dx, *dws)

    return record(Tensor(out, shape=(batch, time, dq)), (x, wq, wk, wv), backward)


def attention_fused(q, k, v, *, scale=None, causal=False):
    """Score and value products of (groups, T, 64) bf16 tensors in one fused
    pass: O = softmax(scale * Q K^T) V (scale defaults to 1/sqrt(64))."""
    if q.shape != k.shape or q.shape != v.shape or q.ndim != 3:
        raise ValueError("attention_fused takes equal (groups, T, D) q, k, v")
    groups, time, dim = q.shape
    out, _ = backend(q).attention(q.storage, k.storage, v.storage, groups, time, 1, 1, dim, causal=causal,
                                  layout=0, scale=scale)
    return Tensor(out, shape=q.shape)


def parameter_count(layer):
    return sum(prod(p.shape) for p in layer.parameters())
