"""The attention path's torch.nn-style surface: functional SDPA and MultiheadAttention."""

from . import functional
from .modules.transformer import MultiheadAttention

__all__ = ["functional", "MultiheadAttention"]
