from .config import Config
from .decoder import Decoder
from .layers import GQA, Block, Projection, RMSNorm, SparseMoE, SwiGLU, attention_products, linear, projection_loss
from .precision import autocast
from .recompute import checkpoint

__all__ = ["Block", "Config", "Decoder", "GQA", "autocast", "Projection", "RMSNorm", "SparseMoE", "SwiGLU", "attention_products",
           "checkpoint", "linear", "projection_loss"]
