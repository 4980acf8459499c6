from .layers import Linear

__all__ = ["Linear"]
