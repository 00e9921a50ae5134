"""Autograd Functions of the attention path.

`RoPEFn` keeps the reference's RoPEFn (gguf_train/_functions.py:1906-1919): forward(ctx, x,
pos, n_dims, mode, n_ctx_orig, freq_base, freq_scale) saves the positions and calls the native
gt_rope; the backward calls gt_rope_backward (the inverse rotation) and returns (gx, None x 6).

`FlashAttentionFn` keeps the reference's signature and behaviour
(gguf_train/_functions.py:1922-1965): forward(ctx, q, k, v, mask, scale, is_causal) saves
its inputs, sets ctx.scale (1/sqrt(D) when None) and ctx.is_causal, and calls the native
gt_flash_attention; the backward returns (dq, dk, dv, None, None, None) with a GQA group's
gradients summed into its kv head.  The reference's Python backward composition
(matmul/softmax over full (B,H,L,S) intermediates) is replaced by the native recompute-based
gt_flash_attention_backward, which works from the saved output and log-sum-exp.

`FlashAttentionDropoutFn` replaces the reference's dropout composition in
scaled_dot_product_attention (gguf_train/nn/functional.py:750-767), which builds the scores,
softmax, a rand_like mask and two matmuls out of differentiable ops: one fused forward and one
fused backward whose dropout decisions come from Philox4x32-10 keyed by a 64-bit seed drawn
from torch's default CPU generator at the forward (so torch.manual_seed, fork_rng and
checkpoint's RNG-state replay reproduce the same decisions); it returns the output and the
non-differentiable log-sum-exp, from which MultiheadAttention recomputes the dropped weights.

The Function subclasses torch.autograd.Function, whose engine - like the reference engine
(gguf_train/_autograd_engine.py:325-326) - casts each gradient to its input's dtype.
"""

from __future__ import annotations

import math

import torch

from . import _ops


class RoPEFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, pos, n_dims, mode, n_ctx_orig, freq_base, freq_scale):
        ctx.args = (int(n_dims), int(mode), int(n_ctx_orig), float(freq_base), float(freq_scale))
        ctx.save_for_backward(pos)
        return _ops.rope(x, pos, *ctx.args)

    @staticmethod
    def backward(ctx, grad_out):
        if grad_out is None:
            return (None,) * 7
        (pos,) = ctx.saved_tensors
        gx = _ops.rope(grad_out, pos, *ctx.args, backward=True)
        return (gx, None, None, None, None, None, None)


class FlashAttentionFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, mask, scale, is_causal):
        ctx.scale = float(scale) if scale is not None else (1.0 / math.sqrt(q.shape[-1]))
        ctx.is_causal = bool(is_causal)
        if any(ctx.needs_input_grad[:3]):
            # the unrounded float32 output (float16/bfloat16 inputs) makes rowsum(dO * O) exact
            out, lse, out32 = _ops.flash_attention_train(q, k, v, mask, ctx.scale, ctx.is_causal)
            ctx.save_for_backward(q, k, v, mask, out if out32 is None else out32, lse)
        else:
            out = _ops.flash_attention(q, k, v, mask, ctx.scale, ctx.is_causal)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        if grad_out is None:
            return (None,) * 6
        q, k, v, mask, out, lse = ctx.saved_tensors
        dq, dk, dv = _ops.flash_attention_backward(grad_out, q, k, v, mask, out, lse, ctx.scale, ctx.is_causal)
        return (dq, dk, dv, None, None, None)


class FlashAttentionLseFn(torch.autograd.Function):
    """FlashAttentionFn that also returns the per-row log-sum-exp (B, H, L) of the same forward
    pass (not differentiable), for callers that need both - MultiheadAttention with
    need_weights=True recomputes the explicit weights from it - without a second forward."""

    @staticmethod
    def forward(ctx, q, k, v, mask, scale, is_causal):
        ctx.scale = float(scale) if scale is not None else (1.0 / math.sqrt(q.shape[-1]))
        ctx.is_causal = bool(is_causal)
        out, lse, out32 = _ops.flash_attention_train(q, k, v, mask, ctx.scale, ctx.is_causal)
        ctx.save_for_backward(q, k, v, mask, out if out32 is None else out32, lse)
        ctx.mark_non_differentiable(lse)
        return out, lse

    @staticmethod
    def backward(ctx, grad_out, grad_lse):
        if grad_out is None:
            return (None,) * 6
        q, k, v, mask, out, lse = ctx.saved_tensors
        dq, dk, dv = _ops.flash_attention_backward(grad_out, q, k, v, mask, out, lse, ctx.scale, ctx.is_causal)
        return (dq, dk, dv, None, None, None)


def draw_dropout_seed() -> int:
    """A 64-bit Philox key from torch's default CPU generator (advances its state)."""
    return int(torch.randint(-(2 ** 63), 2 ** 63 - 1, (), dtype=torch.int64).item()) & 0xFFFFFFFFFFFFFFFF


class FlashAttentionDropoutFn(torch.autograd.Function):
    """Attention with dropout of the probabilities: (out, lse), lse not differentiable."""

    @staticmethod
    def forward(ctx, q, k, v, mask, scale, is_causal, dropout_p, seed):
        ctx.scale = float(scale) if scale is not None else (1.0 / math.sqrt(q.shape[-1]))
        ctx.is_causal = bool(is_causal)
        ctx.dropout = (float(dropout_p), int(seed))
        out, lse, out32 = _ops.flash_attention_dropout(q, k, v, mask, ctx.scale, ctx.is_causal, *ctx.dropout)
        ctx.save_for_backward(q, k, v, mask, out if out32 is None else out32, lse)
        ctx.mark_non_differentiable(lse)
        return out, lse

    @staticmethod
    def backward(ctx, grad_out, grad_lse):
        if grad_out is None:
            return (None,) * 8
        q, k, v, mask, out, lse = ctx.saved_tensors
        dq, dk, dv = _ops.flash_attention_dropout_backward(grad_out, q, k, v, mask, out, lse, ctx.scale,
                                                           ctx.is_causal, *ctx.dropout)
        return (dq, dk, dv, None, None, None, None, None)
