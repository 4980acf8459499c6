from .cache import KVCache
from .layers import Attention, Linear, MultiHeadAttention, causal_mask, softmax

__all__ = ["Attention", "KVCache", "Linear", "MultiHeadAttention", "causal_mask", "softmax"]
