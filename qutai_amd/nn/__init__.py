from .layers import Attention, Linear, MultiHeadAttention, causal_mask, softmax

__all__ = ["Attention", "Linear", "MultiHeadAttention", "causal_mask", "softmax"]
