"""Thin Python calls of the native attention and Q8_0 entry points on PyTorch tensors."""

from __future__ import annotations

import ctypes

import torch

from . import _C
from ._bridge import QuantizedTensor, adopt, adopt_quantized, bind_stream, borrow

_GT_DTYPE = {torch.float32: _C.GT_F32, torch.float16: _C.GT_F16, torch.bfloat16: _C.GT_BF16,
             torch.float64: _C.GT_F64}


def _device_of(*ts) -> torch.device:
    for t in ts:
        if t is not None:
            return t.device
    return torch.device("cpu")


def flash_attention(q, k, v, mask=None, scale: float = 0.0, is_causal: bool = False) -> torch.Tensor:
    """gt_flash_attention (csrc/gguf_train.h:311) on PyTorch tensors."""
    bind_stream(_device_of(q))
    hq, hk, hv = borrow(q), borrow(k), borrow(v)
    hm = borrow(mask) if mask is not None else None
    ptr = _C.lib.gt_flash_attention(hq.ptr, hk.ptr, hv.ptr, hm.ptr if hm else None, ctypes.c_float(scale),
                                    1 if is_causal else 0)
    return adopt(ptr, "flash_attention")


def flash_attention_lse(q, k, v, mask=None, scale: float = 0.0, is_causal: bool = False):
    """Forward that also returns the per-row log-sum-exp (B, H, L) needed by the backward."""
    bind_stream(_device_of(q))
    hq, hk, hv = borrow(q), borrow(k), borrow(v)
    hm = borrow(mask) if mask is not None else None
    po, pl = ctypes.c_void_p(), ctypes.c_void_p()
    rc = _C.lib.gt_flash_attention_lse(hq.ptr, hk.ptr, hv.ptr, hm.ptr if hm else None, ctypes.c_float(scale),
                                       1 if is_causal else 0, ctypes.byref(po), ctypes.byref(pl))
    _C.check_rc(rc, "flash_attention")
    return adopt(po.value, "flash_attention"), adopt(pl.value, "flash_attention")


def flash_attention_train(q, k, v, mask=None, scale: float = 0.0, is_causal: bool = False):
    """Training forward: (out, lse, out32) where out32 is the float32 output before rounding
    (None for float32/float64 inputs, whose `out` is already exact)."""
    bind_stream(_device_of(q))
    hq, hk, hv = borrow(q), borrow(k), borrow(v)
    hm = borrow(mask) if mask is not None else None
    po, pl, p32 = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
    rc = _C.lib.gt_flash_attention_train(hq.ptr, hk.ptr, hv.ptr, hm.ptr if hm else None, ctypes.c_float(scale),
                                         1 if is_causal else 0, ctypes.byref(po), ctypes.byref(pl), ctypes.byref(p32))
    _C.check_rc(rc, "flash_attention")
    out32 = adopt(p32.value, "flash_attention") if p32.value else None
    return adopt(po.value, "flash_attention"), adopt(pl.value, "flash_attention"), out32


def flash_attention_backward(dout, q, k, v, mask, out, lse, scale: float, is_causal: bool):
    """Native recompute-based backward: (dq, dk, dv) in float32 (float64 for float64 inputs)."""
    bind_stream(_device_of(q))
    hg, hq, hk, hv = borrow(dout), borrow(q), borrow(k), borrow(v)
    hm = borrow(mask) if mask is not None else None
    ho = borrow(out) if out is not None else None
    hl = borrow(lse) if lse is not None else None
    pq, pk, pv = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
    rc = _C.lib.gt_flash_attention_backward(hg.ptr, hq.ptr, hk.ptr, hv.ptr, hm.ptr if hm else None,
                                            ho.ptr if ho else None, hl.ptr if hl else None, ctypes.c_float(scale),
                                            1 if is_causal else 0, ctypes.byref(pq), ctypes.byref(pk),
                                            ctypes.byref(pv))
    _C.check_rc(rc, "flash_attention_backward")
    return (adopt(pq.value, "flash_attention_backward"), adopt(pk.value, "flash_attention_backward"),
            adopt(pv.value, "flash_attention_backward"))


def flash_attention_dropout(q, k, v, mask, scale: float, is_causal: bool, p: float, seed: int, offset: int = 0):
    """Training forward with dropout of the probabilities: (out, lse, out32) as
    flash_attention_train; decisions from Philox4x32-10 keyed by (seed, offset)."""
    bind_stream(_device_of(q))
    hq, hk, hv = borrow(q), borrow(k), borrow(v)
    hm = borrow(mask) if mask is not None else None
    po, pl, p32 = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
    rc = _C.lib.gt_flash_attention_dropout(hq.ptr, hk.ptr, hv.ptr, hm.ptr if hm else None, ctypes.c_float(scale),
                                           1 if is_causal else 0, float(p), _u64(seed), _u64(offset),
                                           ctypes.byref(po), ctypes.byref(pl), ctypes.byref(p32))
    _C.check_rc(rc, "flash_attention_dropout")
    out32 = adopt(p32.value, "flash_attention_dropout") if p32.value else None
    return adopt(po.value, "flash_attention_dropout"), adopt(pl.value, "flash_attention_dropout"), out32


def flash_attention_dropout_backward(dout, q, k, v, mask, out, lse, scale: float, is_causal: bool, p: float,
                                     seed: int, offset: int = 0):
    """Backward of flash_attention_dropout with the same (p, seed, offset): (dq, dk, dv)."""
    bind_stream(_device_of(q))
    hg, hq, hk, hv = borrow(dout), borrow(q), borrow(k), borrow(v)
    hm = borrow(mask) if mask is not None else None
    ho = borrow(out) if out is not None else None
    hl = borrow(lse) if lse is not None else None
    pq, pk, pv = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
    rc = _C.lib.gt_flash_attention_dropout_backward(hg.ptr, hq.ptr, hk.ptr, hv.ptr, hm.ptr if hm else None,
                                                    ho.ptr if ho else None, hl.ptr if hl else None,
                                                    ctypes.c_float(scale), 1 if is_causal else 0, float(p), _u64(seed),
                                                    _u64(offset), ctypes.byref(pq), ctypes.byref(pk), ctypes.byref(pv))
    _C.check_rc(rc, "flash_attention_dropout_backward")
    who = "flash_attention_dropout_backward"
    return adopt(pq.value, who), adopt(pk.value, who), adopt(pv.value, who)


def attention_weights_dropout(q, k, mask, lse, scale: float, is_causal: bool, average_heads: bool, p: float,
                              seed: int, offset: int = 0):
    """The weights flash_attention_dropout multiplied V by (after dropout; averaged over the heads
    when asked)."""
    bind_stream(_device_of(q))
    hq, hk, hl = borrow(q), borrow(k), borrow(lse)
    hm = borrow(mask) if mask is not None else None
    ptr = _C.lib.gt_attention_weights_dropout(hq.ptr, hk.ptr, hm.ptr if hm else None, hl.ptr, ctypes.c_float(scale),
                                              1 if is_causal else 0, 1 if average_heads else 0, float(p), _u64(seed),
                                              _u64(offset))
    return adopt(ptr, "attention_weights_dropout")


def attention_dropout_mask(shape, p: float, seed: int, offset: int = 0, device=None) -> torch.Tensor:
    """The dropout decisions (B,H,L,S) bool (True = kept) of (p, seed, offset) on a HIP device."""
    dev = torch.device("cuda") if device is None else torch.device(device)
    index = dev.index if dev.index is not None else (torch.cuda.current_device() if torch.cuda.is_available() else 0)
    if torch.cuda.is_available():
        bind_stream(torch.device("cuda", index))
    B, H, L, S = (int(x) for x in shape)
    ptr = _C.lib.gt_attention_dropout_mask(B, H, L, S, float(p), _u64(seed), _u64(offset), index)
    return adopt(ptr, "attention_dropout_mask")


def _u64(x: int) -> int:
    return int(x) & 0xFFFFFFFFFFFFFFFF


def attention_weights(q, k, mask, lse, scale: float = 0.0, is_causal: bool = False, average_heads: bool = False):
    """gt_attention_weights: softmax(q.k^T*scale + mask) (causal-masked), recomputed from the
    forward's log-sum-exp `lse`; (B,H,L,S), or (B,L,S) averaged over the heads."""
    bind_stream(_device_of(q))
    hq, hk, hl = borrow(q), borrow(k), borrow(lse)
    hm = borrow(mask) if mask is not None else None
    ptr = _C.lib.gt_attention_weights(hq.ptr, hk.ptr, hm.ptr if hm else None, hl.ptr, ctypes.c_float(scale),
                                      1 if is_causal else 0, 1 if average_heads else 0)
    return adopt(ptr, "attention_weights")


def rope(x, pos, n_dims: int, mode: int = 0, n_ctx_orig: int = 0, freq_base: float = 10000.0,
         freq_scale: float = 1.0, backward: bool = False) -> torch.Tensor:
    """gt_rope / gt_rope_backward (csrc/gguf_train.h:309-310) on PyTorch tensors."""
    bind_stream(_device_of(x))
    hx, hp = borrow(x), borrow(pos)
    fn = _C.lib.gt_rope_backward if backward else _C.lib.gt_rope
    ptr = fn(hx.ptr, hp.ptr, int(n_dims), int(mode), int(n_ctx_orig), ctypes.c_float(freq_base),
             ctypes.c_float(freq_scale))
    return adopt(ptr, "rope")


def flash_attention_rope(q, k, v, pos, mask=None, scale: float = 0.0, is_causal: bool = False, n_dims=None,
                         mode: int = 0, freq_base: float = 10000.0, freq_scale: float = 1.0) -> torch.Tensor:
    """gt_flash_attention_rope: attention of rope(q, pos) and rope(k, pos), the query rotation fused
    into the prefill kernel where it runs (no autograd; forward only)."""
    bind_stream(_device_of(q))
    hq, hk, hv, hp = borrow(q), borrow(k), borrow(v), borrow(pos)
    hm = borrow(mask) if mask is not None else None
    nd = q.shape[-1] if n_dims is None else int(n_dims)
    ptr = _C.lib.gt_flash_attention_rope(hq.ptr, hk.ptr, hv.ptr, hm.ptr if hm else None, ctypes.c_float(scale),
                                         1 if is_causal else 0, hp.ptr, nd, int(mode), ctypes.c_float(freq_base),
                                         ctypes.c_float(freq_scale))
    return adopt(ptr, "flash_attention_rope")


def quantize(t: torch.Tensor, qtype: str = "q8_0") -> QuantizedTensor:
    """gt_quantize (csrc/gguf_train.h:381); rows of last-dim length, GGUF Q8_0 blocks."""
    if qtype != "q8_0":
        raise ValueError(f"unsupported quantization type {qtype!r} (only 'q8_0')")
    bind_stream(t.device)
    h = borrow(t)
    ptr = _C.lib.gt_quantize(h.ptr, _C.GT_Q8_0 - _C.GT_Q_BASE)
    return adopt_quantized(ptr, t.shape, "quantize")


def dequantize(qt: QuantizedTensor, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """gt_dequantize (csrc/gguf_train.h:382): y = float(qs) * float(d), then `dtype`."""
    if dtype not in _GT_DTYPE:
        raise ValueError(f"unsupported dequantize dtype {dtype}")
    bind_stream(qt.device)
    h = borrow(qt)
    ptr = _C.lib.gt_dequantize(h.ptr, _GT_DTYPE[dtype])
    return adopt(ptr, "dequantize")
