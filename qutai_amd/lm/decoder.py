"""Decoder-only language model on the MI355X (src/qutai/lm/decoder.py:20-175).

Embedding (tied with the output head), ``n_layers`` pre-norm blocks (GQA
attention with RoPE, SwiGLU or top-k MoE FFN), a final RMSNorm, and the
chunked next-token loss.  Every op runs on the device through the HIP
kernels of ``qutai_amd.backends.amd_lm``: the training step reads nothing
back to the host.

Parameters are fp32; under ``autocast`` (matmul precision bfloat16) the
projections, attention and FFN run on bf16 activations while the residual
stream, norms and parameter gradients stay fp32, as in the reference.  A MoE
block stores each projection of all experts as one (experts, out, in) tensor:
``named_parameters`` names them ``ffn.experts.gate.weight`` etc.; expert e of
the reference's ``ffn.experts.{e}.gate.weight`` is row block e.
"""
from __future__ import annotations

from array import array
from bisect import bisect_left
from itertools import chain

from ..backends import amd
from ..core.context import set_recording
from ..core.tensor import Tensor
from .config import Config
from .layers import Block, Projection, RMSNorm, backend, embed, linear, projection_loss, scaled, unpack
from .recompute import checkpoint


def _int_array(values):
    """int64 array of host ids (C-level conversion; other numbers via int())."""
    values = list(values)
    try:
        return array("q", values)
    except TypeError:
        return array("q", (int(v) for v in values))


class Decoder:
    def __init__(self, config: Config, *, device="amd", dtype=None, seed=None):
        dtype = "float32" if dtype is None else dtype
        if device != "amd":
            raise ValueError("this Decoder runs on the amd device")
        if dtype != "float32":
            raise ValueError("decoder parameters on the amd device are float32 (bf16 activations via autocast)")
        self.config = config
        self.embedding = Projection(config.d_model, config.vocab_size, device=device, dtype=dtype, seed=seed)
        self.blocks = tuple(Block(config, device=device, dtype=dtype, seed=None if seed is None else seed + 1 + 100 * i)
                            for i in range(config.n_layers))
        self.norm = RMSNorm(config.d_model, config.norm_eps, device=device, dtype=dtype)
        self.last_lm_loss = None
        self.last_auxiliary_loss = None

    # ---- parameters (decoder.py:39-90) -------------------------------------------
    def named_parameters(self):
        result = [("embedding.weight", self.embedding.weight)]
        for i, block in enumerate(self.blocks):
            p = f"blocks.{i}."
            result += [(p + "attn_norm.weight", block.attn_norm.weight), (p + "ffn_norm.weight", block.ffn_norm.weight)]
            result += [(p + f"attn.{n}.weight", getattr(block.attn, n).weight) for n in ("q", "k", "v", "out")]
            if block.is_moe:
                result.append((p + "ffn.router.weight", block.ffn.router.weight))
                result += [(p + "ffn.experts.gate.weight", block.ffn.w_gate), (p + "ffn.experts.up.weight", block.ffn.w_up),
                           (p + "ffn.experts.down.weight", block.ffn.w_down)]
            else:
                result += [(p + f"ffn.{n}.weight", getattr(block.ffn, n).weight) for n in ("gate", "up", "down")]
        result.append(("norm.weight", self.norm.weight))
        return tuple(result)

    def parameters(self):
        return tuple(dict.fromkeys(p for _, p in self.named_parameters()))

    def parameter_counts(self):
        return self.config.parameter_counts()

    # ---- forward (decoder.py:92-139) -----------------------------------------------
    def _tokens(self, tokens):
        rows = [row if isinstance(row, (list, tuple)) else list(row) for row in tokens]
        if not rows or any(len(row) != len(rows[0]) for row in rows) or not 1 <= len(rows[0]) <= self.config.max_seq_len:
            raise ValueError("tokens must be a non-empty 2-D batch no longer than max_seq_len")
        ids = _int_array(chain.from_iterable(rows))  # C-level loops: the ids feed every step
        if min(ids) < 0 or max(ids) >= self.config.vocab_size:
            raise ValueError("token id outside the vocabulary")
        return ids, (len(rows), len(rows[0]))

    def hidden(self, tokens, *, train=True):
        with set_recording(train):
            return self._hidden(tokens, train=train)

    def _hidden(self, tokens, *, train=True):
        ids, shape = self._tokens(tokens)
        hidden = embed(ids, self.embedding.weight, shape)
        auxiliary = []
        for block in self.blocks:
            if train and self.config.activation_checkpointing:
                if block.is_moe:
                    hidden, aux = unpack(checkpoint(block.packed, hidden, parameters=block.parameters()),
                                         hidden.shape)
                else:
                    hidden = checkpoint(block.hidden, hidden, parameters=block.parameters())
                    aux = Tensor(amd.full(1, 0.0, dtype=hidden.dtype), shape=())
            else:
                hidden, aux = block(hidden)
            auxiliary.append(aux)
        total = auxiliary[0]
        for value in auxiliary[1:]:
            total = total + value.to(dtype=total.dtype)
        self.last_auxiliary_loss = scaled(total, 1 / self.config.n_layers)
        return self.norm(hidden)

    def __call__(self, tokens, *, train=True):
        """Logits (batch, time, vocab) of the tied head (decoder.py:134-139)."""
        with set_recording(train):
            return linear(self.hidden(tokens, train=train), self.embedding.weight)

    # ---- loss (decoder.py:141-175) -------------------------------------------------
    def loss(self, tokens, labels=None, *, train=True, chunk_size=128):
        if chunk_size <= 0:
            raise ValueError("chunk_size must be positive")
        _, shape = self._tokens(tokens)
        if shape[1] < 2:
            raise ValueError("next-token training needs at least two positions")
        labels = tokens if labels is None else labels
        label_rows = [row if isinstance(row, (list, tuple)) else list(row) for row in labels]
        if len(label_rows) != shape[0] or any(len(row) != shape[1] for row in label_rows):
            raise ValueError("labels must have the shape of tokens")
        ordered = sorted(_int_array(chain.from_iterable(label_rows)))
        first = bisect_left(ordered, -99)  # first label above the ignore id
        if ordered[0] < -100 or ordered[-1] >= self.config.vocab_size or (first < len(ordered) and ordered[first] < 0):
            raise ValueError("labels must be vocabulary ids or -100")
        with set_recording(train):
            prepared = backend(self.embedding.weight).prepare_labels(
                _int_array(chain.from_iterable(row[1:] for row in label_rows)))
            hidden = self.hidden(tokens, train=train)
            self.last_lm_loss = projection_loss(hidden, self.embedding.weight, label_rows, chunk_size,
                                                prepared_labels=prepared)
            aux = self.last_auxiliary_loss.to(dtype=self.last_lm_loss.dtype)
            return self.last_lm_loss + scaled(aux, self.config.aux_loss_coef)

