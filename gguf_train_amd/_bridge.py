"""Moves PyTorch tensors across the C ABI without copies.

Inputs are lent to the library as borrowed handles (gt_tensor_from_device_ptr for HIP
memory, gt_tensor_from_external for host memory); results come back as library-owned
handles and are adopted by PyTorch through DLPack (gt_tensor_to_dlpack), so the memory the
kernels wrote is the memory the caller reads.  Every native call is made on the caller's
current PyTorch stream (gt_set_stream), which keeps the library ordered with PyTorch work.

PyTorch is plumbing here: device memory and streams.  No attention math happens in PyTorch.
"""

from __future__ import annotations

import ctypes
import itertools
from dataclasses import dataclass

import torch

from . import _C

TORCH_TO_GT = {
    torch.float32: _C.GT_F32,
    torch.float16: _C.GT_F16,
    torch.bfloat16: _C.GT_BF16,
    torch.float64: _C.GT_F64,
    torch.int8: _C.GT_I8,
    torch.uint8: _C.GT_U8,
    torch.int16: _C.GT_I16,
    torch.int32: _C.GT_I32,
    torch.int64: _C.GT_I64,
    torch.bool: _C.GT_BOOL,
}
GT_TO_TORCH = {v: k for k, v in TORCH_TO_GT.items()}

_tokens = itertools.count(1)

_PyCapsule_New = ctypes.pythonapi.PyCapsule_New
_PyCapsule_New.restype = ctypes.py_object
_PyCapsule_New.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_void_p]
_DLTENSOR = b"dltensor"


@dataclass
class QuantizedTensor:
    """A GGUF Q8_0 tensor: `data` holds the ggml blocks (fp16 d + 32 int8, 34 bytes per 32
    values along the flattened logical shape) as a uint8 tensor; `shape` is the logical shape.
    Mirrors the reference's quantized Tensor (dtype code 108, gguf_train/_dtype.py:85)."""

    data: torch.Tensor
    shape: tuple
    gt_dtype: int = _C.GT_Q8_0

    @property
    def device(self) -> torch.device:
        return self.data.device

    @property
    def ndim(self) -> int:
        return len(self.shape)

    def numel(self) -> int:
        n = 1
        for s in self.shape:
            n *= int(s)
        return n


class Handle:
    """Owns one gt_tensor* and frees it when dropped; `keep` pins borrowed memory."""

    __slots__ = ("ptr", "keep")

    def __init__(self, ptr: int, keep=None):
        self.ptr = ptr
        self.keep = keep

    def release(self) -> int:
        p, self.ptr = self.ptr, 0
        return p

    def __del__(self, _free=_C.lib.gt_tensor_free):
        if self.ptr:
            _free(self.ptr)
            self.ptr = 0


def _i64(vals) -> ctypes.Array:
    vals = [int(v) for v in vals]
    return (ctypes.c_int64 * max(len(vals), 1))(*vals)


def bind_stream(device: torch.device) -> None:
    """Makes the library enqueue on PyTorch's current stream of `device`."""
    if device.type == "cuda":
        _C.lib.gt_set_stream(ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream))
    else:
        _C.lib.gt_set_stream(None)


_released_buf = (ctypes.c_uint64 * 1024)()


def _drain_released() -> None:
    """Borrowed memory stays pinned by `Handle.keep`, so the release tokens the library queues
    carry no information here; drop them so the queue does not grow."""
    while _C.lib.gt_external_released(_released_buf, 1024) == 1024:
        pass


def borrow(t) -> Handle:
    """A handle on the memory of a PyTorch tensor (or QuantizedTensor), without a copy."""
    if next(_tokens) % 512 == 0:
        _drain_released()
    if isinstance(t, QuantizedTensor):
        d = t.data
        if not d.is_cuda:
            nb = d.numel()
            ptr = _C.lib.gt_tensor_from_data(len(t.shape), _i64(t.shape), _C.GT_Q8_0, _C.GT_DEV_CPU, 0,
                                             ctypes.c_void_p(d.contiguous().data_ptr()), nb)
            return Handle(_C.check_ptr(ptr, "borrow"))
        if not d.is_contiguous() or d.dtype != torch.uint8:
            raise ValueError("QuantizedTensor.data must be a contiguous uint8 tensor")
        strides = []
        acc = 1
        for s in reversed(t.shape):
            strides.append(acc)
            acc *= int(s)
        strides.reverse()
        ptr = _C.lib.gt_tensor_from_device_ptr(len(t.shape), _i64(t.shape), _i64(strides), _C.GT_Q8_0,
                                               d.device.index or 0, ctypes.c_void_p(d.data_ptr()), next(_tokens))
        return Handle(_C.check_ptr(ptr, "borrow"), keep=d)
    if t.dtype not in TORCH_TO_GT:
        raise TypeError(f"dtype {t.dtype} is not supported by libgt_attn")
    code = TORCH_TO_GT[t.dtype]
    if t.numel() == 0:
        # nothing to lend: an empty library tensor of the same shape and device
        dev_type = _C.GT_DEV_CUDA if t.is_cuda else _C.GT_DEV_CPU
        ptr = _C.lib.gt_tensor_empty(t.ndim, _i64(t.shape), code, dev_type, (t.device.index or 0) if t.is_cuda else 0)
        return Handle(_C.check_ptr(ptr, "borrow"))
    shape, strides = _i64(t.shape), _i64(t.stride())
    if t.is_cuda:
        ptr = _C.lib.gt_tensor_from_device_ptr(t.ndim, shape, strides, code, t.device.index or 0,
                                               ctypes.c_void_p(t.data_ptr()), next(_tokens))
    else:
        ptr = _C.lib.gt_tensor_from_external(t.ndim, shape, strides, code, ctypes.c_void_p(t.data_ptr()),
                                             next(_tokens))
    return Handle(_C.check_ptr(ptr, "borrow"), keep=t)


def adopt(ptr: int, ctx: str = "") -> torch.Tensor:
    """Turns a library-owned result handle into a PyTorch tensor (zero-copy, via DLPack)."""
    _C.check_ptr(ptr, ctx)
    try:
        dl = _C.lib.gt_tensor_to_dlpack(ptr)
        _C.check_ptr(dl, ctx)
    finally:
        _C.lib.gt_tensor_free(ptr)
    capsule = _PyCapsule_New(dl, _DLTENSOR, None)
    return torch.utils.dlpack.from_dlpack(capsule)


def adopt_quantized(ptr: int, shape, ctx: str = "") -> QuantizedTensor:
    return QuantizedTensor(adopt(ptr, ctx), tuple(int(s) for s in shape))
