"""gguf_train_amd - MI355X (gfx950) attention for GGUF_train's operator API.

The product is libgt_attn.so (hand-written HIP kernels behind the reference's C ABI,
include/gt_attn.h).  This package is its Python host: the ctypes loader (_C), the
PyTorch <-> handle bridge (_bridge), FlashAttentionFn, scaled_dot_product_attention and
MultiheadAttention with the reference's signatures, and the GGUF Q8_0 codec.
"""

from . import _C
from ._bridge import QuantizedTensor
from ._functions import FlashAttentionDropoutFn, FlashAttentionFn, RoPEFn
from ._ops import (attention_dropout_mask, attention_weights_dropout, dequantize, flash_attention,
                   flash_attention_backward, flash_attention_dropout, flash_attention_dropout_backward,
                   flash_attention_lse, flash_attention_rope, flash_attention_train, quantize, rope)
from . import nn
from .kv_cache import KVCache

__all__ = [
    "_C",
    "QuantizedTensor",
    "FlashAttentionFn",
    "FlashAttentionDropoutFn",
    "RoPEFn",
    "rope",
    "flash_attention",
    "flash_attention_lse",
    "flash_attention_train",
    "flash_attention_rope",
    "flash_attention_backward",
    "flash_attention_dropout",
    "flash_attention_dropout_backward",
    "attention_weights_dropout",
    "attention_dropout_mask",
    "quantize",
    "dequantize",
    "nn",
    "KVCache",
]
