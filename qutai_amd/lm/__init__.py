from .config import Config
from .decoder import Decoder
from .layers import GQA, Block, Projection, RMSNorm, SparseMoE, SwiGLU, attention_products, linear, projection_loss
from .layers import rope, silu_mul
from .precision import autocast
from .recompute import checkpoint as activation_checkpoint
from .checkpoint import checkpoint_metadata, load_checkpoint, load_weights, save_checkpoint, save_weights

__all__ = ["Block", "Config", "Decoder", "GQA", "Projection", "RMSNorm", "SparseMoE", "SwiGLU", "activation_checkpoint",
           "attention_products", "autocast", "checkpoint_metadata", "linear", "load_checkpoint", "load_weights",
           "projection_loss", "rope", "save_checkpoint", "save_weights", "silu_mul"]
