"""MultiheadAttention with the reference's constructor, forward signature and mask conventions
(gguf_train/nn/modules/transformer.py:21-191).

- packed in-projection (`in_proj_weight` (3E, E)) when kdim == vdim == embed_dim, separate
  q/k/v projection weights otherwise; xavier-uniform init, zero biases;
- query/key/value: batched 3-D ((L, B, E), or (B, L, E) with batch_first) or unbatched 2-D;
- boolean attn_mask / key_padding_mask: True marks a position that must NOT be attended to and
  becomes -1e9 in the scores' dtype (-inf in float16, where a row whose every key is blocked
  then gives 0; autocast lowers the mask with q/k/v, so it behaves the same); float masks are
  added; a 2-D attn_mask is (L, S), a 3-D one (B*H, L, S);
- need_weights=False runs the fused attention kernel (scaled_dot_product_attention);
  need_weights=True returns the softmax weights too (averaged over heads by default): the fused
  kernel gives the output and its log-sum-exp, the native gt_attention_weights recomputes the
  weights from them (the reference composes them with ggml ops, transformer.py:153-166).  The
  causal mask excludes future keys rather than adding -1e9 (the same weights unless every
  visible key of a row is masked out); gradients flow through the output, not the returned
  weights; with dropout in training the fused dropout kernels run and the returned weights are
  the dropped ones the output was formed with (gt_attention_weights_dropout, same decisions).

The projections are plain GEMMs (torch.nn.functional.linear); the attention itself is the
native kernel.
"""

from __future__ import annotations

import math

import torch
from torch import nn

from ... import _ops
from ..._functions import FlashAttentionDropoutFn, FlashAttentionLseFn, draw_dropout_seed
from .. import functional as F


class MultiheadAttention(nn.Module):
    def __init__(
        self,
        embed_dim: int,
        num_heads: int,
        dropout: float = 0.0,
        bias: bool = True,
        add_bias_kv: bool = False,
        add_zero_attn: bool = False,
        kdim: int | None = None,
        vdim: int | None = None,
        batch_first: bool = False,
        device=None,
        dtype=None,
    ) -> None:
        super().__init__()
        (add_bias_kv, add_zero_attn)  # accepted and ignored, as in the reference
        self.embed_dim = int(embed_dim)
        self.num_heads = int(num_heads)
        self.head_dim = self.embed_dim // self.num_heads
        assert self.head_dim * self.num_heads == self.embed_dim, "embed_dim must be divisible by num_heads"
        self.dropout = float(dropout)
        self.batch_first = bool(batch_first)
        self.kdim = self.embed_dim if kdim is None else int(kdim)
        self.vdim = self.embed_dim if vdim is None else int(vdim)
        fk = {"device": device, "dtype": dtype or torch.get_default_dtype()}
        self._qkv_same = self.kdim == self.embed_dim and self.vdim == self.embed_dim
        if self._qkv_same:
            self.in_proj_weight = nn.Parameter(torch.empty((3 * self.embed_dim, self.embed_dim), **fk))
            self.register_parameter("q_proj_weight", None)
            self.register_parameter("k_proj_weight", None)
            self.register_parameter("v_proj_weight", None)
            nn.init.xavier_uniform_(self.in_proj_weight)
        else:
            self.register_parameter("in_proj_weight", None)
            self.q_proj_weight = nn.Parameter(torch.empty((self.embed_dim, self.embed_dim), **fk))
            self.k_proj_weight = nn.Parameter(torch.empty((self.embed_dim, self.kdim), **fk))
            self.v_proj_weight = nn.Parameter(torch.empty((self.embed_dim, self.vdim), **fk))
            nn.init.xavier_uniform_(self.q_proj_weight)
            nn.init.xavier_uniform_(self.k_proj_weight)
            nn.init.xavier_uniform_(self.v_proj_weight)
        if bias:
            self.in_proj_bias = nn.Parameter(torch.zeros((3 * self.embed_dim,), **fk))
        else:
            self.register_parameter("in_proj_bias", None)
        self.out_proj = nn.Linear(self.embed_dim, self.embed_dim, bias=bias, **fk)

    def forward(
        self,
        query,
        key,
        value,
        key_padding_mask=None,
        need_weights: bool = True,
        attn_mask=None,
        average_attn_weights: bool = True,
        is_causal: bool = False,
    ):
        is_batched = query.ndim == 3
        if not is_batched:
            if query.ndim != 2 or key.ndim != 2 or value.ndim != 2:
                raise RuntimeError(
                    "MultiheadAttention: query, key and value must all be 3-D (batched) or all 2-D (unbatched), "
                    f"got {query.ndim}-D, {key.ndim}-D and {value.ndim}-D"
                )
            batch_dim = 0 if self.batch_first else 1
            query, key, value = query.unsqueeze(batch_dim), key.unsqueeze(batch_dim), value.unsqueeze(batch_dim)
            if key_padding_mask is not None:
                if key_padding_mask.ndim != 1:
                    raise RuntimeError(
                        "MultiheadAttention: key_padding_mask of an unbatched input must be 1-D (S), "
                        f"got {list(key_padding_mask.shape)}"
                    )
                key_padding_mask = key_padding_mask.unsqueeze(0)
        elif key.ndim != 3 or value.ndim != 3:
            raise RuntimeError(
                "MultiheadAttention: query, key and value must all be 3-D (batched) or all 2-D (unbatched), "
                f"got {query.ndim}-D, {key.ndim}-D and {value.ndim}-D"
            )
        if not self.batch_first:
            query, key, value = query.transpose(0, 1), key.transpose(0, 1), value.transpose(0, 1)

        B, L, E = query.shape
        S = key.shape[1]
        H, D = self.num_heads, self.head_dim
        if self._qkv_same:
            wq, wk, wv = self.in_proj_weight.chunk(3, dim=0)
        else:
            wq, wk, wv = self.q_proj_weight, self.k_proj_weight, self.v_proj_weight
        if self.in_proj_bias is not None:
            bq, bk, bv = self.in_proj_bias.chunk(3, dim=0)
        else:
            bq = bk = bv = None
        # (B, L, H, D) memory viewed as (B, H, L, D): the kernels read these strides directly
        q = torch.nn.functional.linear(query, wq, bq).reshape(B, L, H, D).transpose(1, 2)
        k = torch.nn.functional.linear(key, wk, bk).reshape(B, S, H, D).transpose(1, 2)
        v = torch.nn.functional.linear(value, wv, bv).reshape(B, S, H, D).transpose(1, 2)

        mask = None
        if attn_mask is not None:
            if attn_mask.ndim == 2:
                if tuple(attn_mask.shape) != (L, S):
                    raise RuntimeError(
                        f"MultiheadAttention: the 2D attn_mask has shape {list(attn_mask.shape)}, expected {[L, S]}"
                    )
                mask = self._additive_mask(attn_mask, q.dtype, "attn_mask").reshape(1, 1, L, S)
            elif attn_mask.ndim == 3:
                if tuple(attn_mask.shape) != (B * H, L, S):
                    raise RuntimeError(
                        f"MultiheadAttention: the 3D attn_mask has shape {list(attn_mask.shape)}, "
                        f"expected {[B * H, L, S]}"
                    )
                mask = self._additive_mask(attn_mask, q.dtype, "attn_mask").reshape(B, H, L, S)
            else:
                raise RuntimeError(f"MultiheadAttention: attn_mask must be 2D or 3D, got {attn_mask.ndim}D")
        if key_padding_mask is not None:
            if tuple(key_padding_mask.shape) != (B, S):
                raise RuntimeError(
                    f"MultiheadAttention: key_padding_mask has shape {list(key_padding_mask.shape)}, expected {[B, S]}"
                )
            km = self._additive_mask(key_padding_mask, q.dtype, "key_padding_mask").reshape(B, 1, 1, S)
            mask = km if mask is None else (mask + km)

        scale = 1.0 / math.sqrt(D)
        if not need_weights:
            attn_out = F.scaled_dot_product_attention(
                q, k, v, attn_mask=mask, dropout_p=self.dropout if self.training else 0.0, is_causal=is_causal,
                scale=scale,
            )
            attn_weights = None
        elif self.dropout > 0.0 and self.training:
            # dropout on the explicit weights (the reference composes it, transformer.py:153-166):
            # the fused dropout forward, and the weights it multiplied V by, recomputed from its
            # log-sum-exp with the same dropout decisions
            seed = draw_dropout_seed()
            attn_out, lse = FlashAttentionDropoutFn.apply(q, k, v, mask, scale, is_causal, float(self.dropout), seed)
            with torch.no_grad():
                attn_weights = _ops.attention_weights_dropout(q.detach(), k.detach(), mask, lse, scale, is_causal,
                                                              average_attn_weights, float(self.dropout), seed)
        else:
            # native: the fused forward gives the output and the log-sum-exp, from which the
            # weights are recomputed (gt_attention_weights); gradients flow through the output
            # one forward pass gives both (with its backward residuals when grads are needed)
            needs_grad = torch.is_grad_enabled() and any(t.requires_grad for t in (q, k, v))
            if needs_grad:
                attn_out, lse = FlashAttentionLseFn.apply(q, k, v, mask, scale, is_causal)
            else:
                attn_out, lse = _ops.flash_attention_lse(q, k, v, mask, scale, is_causal)
            with torch.no_grad():
                attn_weights = _ops.attention_weights(q.detach(), k.detach(), mask, lse, scale, is_causal,
                                                      average_attn_weights)

        out = attn_out.transpose(1, 2).reshape(B, L, E)
        out = self.out_proj(out)
        if not self.batch_first:
            out = out.transpose(0, 1)
        if not is_batched:
            out = out.squeeze(1 if not self.batch_first else 0)
            if attn_weights is not None:
                attn_weights = attn_weights.squeeze(0)
        return out, attn_weights

    @staticmethod
    def _additive_mask(mask, dtype, name: str):
        """torch.nn convention: True in a boolean mask blocks the position (-1e9); a float mask
        is added as it is."""
        if mask.dtype == torch.bool:
            # in the scores' dtype, as the reference (transformer.py:187-188): -1e9 is -inf in
            # float16, so a float16 row whose every key is blocked gives 0 (the rule for a row
            # with nothing visible), with or without autocast (which lowers the mask as well)
            # (-1e9 rounded to `dtype` as a cast rounds it: -inf for float16)
            fill = torch.tensor(-1e9, dtype=torch.float64).to(dtype).item()
            return torch.zeros(mask.shape, dtype=dtype, device=mask.device).masked_fill(mask, fill)
        if not mask.is_floating_point():
            raise RuntimeError(f"MultiheadAttention: {name} must be a boolean or floating point tensor, got {mask.dtype}")
        return mask if mask.dtype == dtype else mask.to(dtype)
