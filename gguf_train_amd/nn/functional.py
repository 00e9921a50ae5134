"""`scaled_dot_product_attention` with the reference's signature and semantics
(gguf_train/nn/functional.py:724-767).

- scale defaults to 1/sqrt(D) (computed in Python double, handed to C as float32);
- attn_mask: bool True = may attend, float = added to the scores; it is checked against the
  attention weights (B, H, L, S) from the right and reshaped to 4-D;
- is_causal masks s > l (top-left aligned);
- dropout_p == 0 runs the fused native kernel through FlashAttentionFn; dropout_p > 0 runs the
  fused native dropout kernels through FlashAttentionDropoutFn (the reference composes matmul,
  softmax, dropout, matmul; here the dropout decisions come from a counter-based generator
  seeded from torch's default generator, and a row with nothing to attend to yields 0 as on the
  dropout_p == 0 path, where the reference's -1e9 fill would average V);
- inside autocast, q/k/v (and a float mask) are cast to the autocast dtype
  (gguf_train/_tensor.py:261-283, gguf_train/amp.py:8-10);
- k/v may be QuantizedTensor (GGUF Q8_0); they are read as their dequantized values and carry
  no gradient.
"""

from __future__ import annotations

import math

import torch

from .._bridge import QuantizedTensor
from .._functions import FlashAttentionDropoutFn, FlashAttentionFn, RoPEFn, draw_dropout_seed
from .. import _ops


def _autocast_lower(*ts):
    """Casts floating-point operands to the active autocast dtype (the reference's
    _AUTOCAST_LOWER policy); returns them unchanged outside autocast."""
    out = []
    for t in ts:
        if isinstance(t, torch.Tensor) and t.is_floating_point():
            dev = t.device.type
            if torch.is_autocast_enabled(dev):
                t = t.to(torch.get_autocast_dtype(dev))
        out.append(t)
    return out


def scaled_dot_product_attention(
    query,
    key,
    value,
    attn_mask=None,
    dropout_p: float = 0.0,
    is_causal: bool = False,
    scale: float | None = None,
    enable_gqa: bool = False,
):
    (enable_gqa,)  # GQA follows from the head counts, as in the reference
    query, key, value, attn_mask = _autocast_lower(query, key, value, attn_mask)
    sc = (1.0 / math.sqrt(query.shape[-1])) if scale is None else float(scale)
    if attn_mask is not None:
        if query.ndim == 4 and key.ndim == 4:
            want = (query.shape[0], query.shape[1], query.shape[2], key.shape[2])
            if attn_mask.ndim > 4 or any(m != 1 and m != w for m, w in zip(reversed(attn_mask.shape), reversed(want))):
                raise RuntimeError(
                    f"scaled_dot_product_attention: attn_mask of shape {list(attn_mask.shape)} cannot be broadcast "
                    f"to the attention weights {list(want)}"
                )
            if attn_mask.ndim != 4:
                attn_mask = attn_mask.reshape((1,) * (4 - attn_mask.ndim) + tuple(attn_mask.shape))
    quantized = isinstance(key, QuantizedTensor) or isinstance(value, QuantizedTensor)
    with torch.autocast(query.device.type, enabled=False):
        if quantized:
            if dropout_p != 0.0:
                raise RuntimeError("scaled_dot_product_attention: dropout is not supported with q8_0 key/value")
            return _ops.flash_attention(query, key, value, attn_mask, sc, is_causal)
        if dropout_p == 0.0:
            return FlashAttentionFn.apply(query, key, value, attn_mask, sc, is_causal)
        # dropout (the reference composes it, gguf_train/nn/functional.py:750-767): fused forward
        # and backward drawing the decisions from a seed of torch's generator
        out, _ = FlashAttentionDropoutFn.apply(query, key, value, attn_mask, sc, is_causal, float(dropout_p),
                                               draw_dropout_seed())
        return out


def rope(input, positions, n_dims: int | None = None, mode: int = 0, n_ctx_orig: int = 0, freq_base: float = 10000.0,
         freq_scale: float = 1.0):
    """Rotary position embedding with the reference's signature (gguf_train/nn/functional.py:770-772):
    input (batch, heads, seq_len, head_dim) or (heads, seq_len, head_dim), positions 1-D (the first
    seq_len are used); n_dims defaults to head_dim; mode 0 NORMAL, 2 NeoX."""
    nd = input.shape[-1] if n_dims is None else int(n_dims)
    return RoPEFn.apply(input, positions, nd, int(mode), int(n_ctx_orig), float(freq_base), float(freq_scale))
