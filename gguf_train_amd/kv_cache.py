"""A key/value cache for decoding, on the device.

The reference decodes through llama.cpp's context (LlamaContext.forward_logits / clear_kv,
gguf_train/llama/__init__.py:174-190, csrc/llama_bridge.cpp:245-296): tokens are fed at
positions that continue what the context holds, the context has a fixed size (n_ctx) and
clear_kv() empties it.  KVCache keeps that behaviour for attention: `batch` sequences of
n_head_kv heads, room for `capacity` tokens each, stored in HBM as float16 / bfloat16 /
float32 or GGUF Q8_0 (each appended row quantized exactly as `quantize` does).  Attention
over the cache runs the library's kernels with each sequence's own length:
split-K decode for one query row (straight from the Q8_0 blocks for a Q8_0 cache), the MFMA
prefill kernel for several.
"""

from __future__ import annotations

import ctypes

import torch

from . import _C
from ._bridge import adopt, adopt_quantized, bind_stream, borrow

_CACHE_DTYPES = {torch.float32: _C.GT_F32, torch.float16: _C.GT_F16, torch.bfloat16: _C.GT_BF16, "q8_0": _C.GT_Q8_0}


class KVCache:
    def __init__(self, batch: int, n_head_kv: int, capacity: int, head_dim: int, dtype=torch.float16,
                 device: str | torch.device = "cuda") -> None:
        if dtype not in _CACHE_DTYPES:
            raise ValueError(f"unsupported cache dtype {dtype!r} (float32, float16, bfloat16 or 'q8_0')")
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("the KV cache lives in device memory: pass a cuda device")
        self.dtype = dtype
        self.batch, self.n_head_kv, self.head_dim = int(batch), int(n_head_kv), int(head_dim)
        bind_stream(self.device)
        index = self.device.index if self.device.index is not None else torch.cuda.current_device()
        self._ptr = _C.check_ptr(_C.lib.gt_kv_cache_create(self.batch, self.n_head_kv, int(capacity), self.head_dim,
                                                           _CACHE_DTYPES[dtype], int(index)), "kv_cache")

    def __del__(self, _free=_C.lib.gt_kv_cache_free):
        ptr = getattr(self, "_ptr", None)
        if ptr:
            _free(ptr)
            self._ptr = None

    @property
    def capacity(self) -> int:
        return int(_C.lib.gt_kv_cache_capacity(self._ptr))

    def n_ctx(self) -> int:
        """The number of tokens a sequence can hold (LlamaContext.n_ctx)."""
        return self.capacity

    def length(self, seq: int = 0) -> int:
        n = int(_C.lib.gt_kv_cache_length(self._ptr, int(seq)))
        if n < 0:
            raise IndexError(_C.last_error())
        return n

    @property
    def lengths(self) -> list[int]:
        return [self.length(b) for b in range(self.batch)]

    def clear(self, seq: int | None = None) -> None:
        """Empties one sequence, or all of them (LlamaContext.clear_kv)."""
        bind_stream(self.device)
        _C.check_rc(_C.lib.gt_kv_cache_clear(self._ptr, -1 if seq is None else int(seq)), "kv_cache")

    clear_kv = clear

    def append(self, k: torch.Tensor, v: torch.Tensor, pos_offset: int | None = None, rope: dict | None = None) -> None:
        """Appends k, v (batch, n_head_kv, T, head_dim) to every sequence: float tensors, or Q8_0
        `QuantizedTensor`s (e.g. read from a GGUF file), whose blocks a Q8_0 cache stores as they
        are.  With pos_offset the positions must continue what each sequence holds, as
        forward_logits(pos_offset=...).  `rope` (keys n_dims, mode, freq_base, freq_scale, as
        nn.functional.rope) rotates each key row at its cache position on the way in; the cache
        then holds what rope() of the keys followed by append() would store."""
        bind_stream(self.device)
        hk, hv = borrow(k), borrow(v)
        off = -1 if pos_offset is None else int(pos_offset)
        if rope is None:
            rc = _C.lib.gt_kv_cache_append(self._ptr, hk.ptr, hv.ptr, off)
        else:
            r = dict(rope)
            unknown = set(r) - {"n_dims", "mode", "freq_base", "freq_scale"}
            if unknown:
                raise TypeError(f"unknown rope arguments {sorted(unknown)}")
            rc = _C.lib.gt_kv_cache_append_rope(self._ptr, hk.ptr, hv.ptr, off, int(r.get("n_dims", self.head_dim)),
                                                int(r.get("mode", 0)), ctypes.c_float(r.get("freq_base", 10000.0)),
                                                ctypes.c_float(r.get("freq_scale", 1.0)))
        _C.check_rc(rc, "kv_cache")

    def attention(self, q: torch.Tensor, scale: float | None = None, is_causal: bool = True) -> torch.Tensor:
        """Attention of q (batch, H, L, head_dim) whose rows are the last L tokens of each
        sequence, over what each sequence holds; causal: a token sees itself and earlier ones."""
        bind_stream(self.device)
        hq = borrow(q)
        ptr = _C.lib.gt_kv_cache_attention(self._ptr, hq.ptr, ctypes.c_float(0.0 if scale is None else scale),
                                           1 if is_causal else 0)
        return adopt(ptr, "kv_cache")

    def keys(self):
        """The key storage (batch, n_head_kv, capacity, head_dim), shared, not copied."""
        return self._storage(_C.lib.gt_kv_cache_keys)

    def values(self):
        return self._storage(_C.lib.gt_kv_cache_values)

    def _storage(self, fn):
        ptr = fn(self._ptr)
        if self.dtype == "q8_0":
            return adopt_quantized(ptr, (self.batch, self.n_head_kv, self.capacity, self.head_dim), "kv_cache")
        return adopt(ptr, "kv_cache")
