"""Decoder configuration (src/qutai/lm/config.py:5-71): the same fields,
defaults, validation and parameter-count formula."""
from __future__ import annotations

from dataclasses import asdict, dataclass
from math import isfinite


@dataclass
class Config:
    vocab_size: int = 32768
    n_layers: int = 20
    d_model: int = 1024
    n_heads: int = 16
    n_kv_heads: int = 4
    d_ff: int = 3584
    max_seq_len: int = 1024
    ffn_type: str = "dense"
    n_experts: int = 8
    top_k: int = 2
    d_expert: int = 1792
    rope_theta: float = 10000.0
    norm_eps: float = 1e-06
    aux_loss_coef: float = 0.01
    activation_checkpointing: bool = True

    def __post_init__(self):
        sizes = (self.vocab_size, self.n_layers, self.d_model, self.n_heads, self.n_kv_heads, self.d_ff,
                 self.max_seq_len, self.n_experts, self.d_expert)
        if any(type(v) is not int or v <= 0 for v in sizes):
            raise ValueError("model sizes must be positive integers")
        if self.d_model % self.n_heads or self.n_heads % self.n_kv_heads:
            raise ValueError("d_model must split into n_heads, and n_heads into n_kv_heads groups")
        head = self.d_model // self.n_heads
        if head % 2 or head > 256:
            raise ValueError("the RoPE head width must be even and at most 256")
        if self.ffn_type not in ("dense", "moe") or type(self.top_k) is not int or not 1 <= self.top_k <= self.n_experts:
            raise ValueError("ffn_type must be dense or moe, with 1 <= top_k <= n_experts")
        real = (self.norm_eps, self.rope_theta, self.aux_loss_coef)
        if any(not isinstance(v, (int, float)) or not isfinite(v) for v in real):
            raise ValueError("norm_eps, rope_theta and aux_loss_coef must be finite numbers")
        if self.norm_eps <= 0 or self.rope_theta <= 0 or self.aux_loss_coef < 0:
            raise ValueError("norm_eps and rope_theta must be positive, aux_loss_coef non-negative")

    def to_dict(self):
        return asdict(self)

    def parameter_counts(self):
        d = self.d_model
        kv_width = self.n_kv_heads * (d // self.n_heads)
        shared = self.vocab_size * d + d  # tied embedding / head and the final norm
        per_attention = 2 * d * d + 2 * d * kv_width + 2 * d  # q, out, k, v and the two norms
        if self.ffn_type == "dense":
            total = shared + self.n_layers * (per_attention + 3 * d * self.d_ff)
            return {"total_parameters": total, "active_parameters": total}
        expert = 3 * d * self.d_expert
        base = shared + self.n_layers * (per_attention + d * self.n_experts)
        return {"total_parameters": base + self.n_layers * self.n_experts * expert,
                "active_parameters": base + self.n_layers * self.top_k * expert}
