from .transformer import MultiheadAttention

__all__ = ["MultiheadAttention"]
