from .linalg import matmul

__all__ = ["matmul"]
