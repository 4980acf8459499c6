from .layers import Projection, SparseMoE, SwiGLU, attention_products, linear

__all__ = ["Projection", "SparseMoE", "SwiGLU", "attention_products", "linear"]
