"""GGUF files: metadata and tensors, on the host or straight into GPU memory.

The read side of the reference's `gguf_train.gguf` (gguf_train/gguf/__init__.py:69-266) over
libgt_attn's own GGUF reader (gt_gguf_*).  `GGUFFile(path, dequantize, device)` reads every
tensor at open, as the reference does; `device="cuda"` streams each one from the file into HBM
(gt_gguf_get_tensor_device) instead of building a host copy first.  Q8_0 tensors that are not
dequantized come back as `QuantizedTensor` (the 34-byte ggml blocks), which the attention entry
points accept as k / v.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch

from . import _C
from ._bridge import QuantizedTensor, adopt, adopt_quantized, bind_stream

# enum gguf_type
_UINT8, _INT8, _UINT16, _INT16, _UINT32, _INT32, _FLOAT32, _BOOL, _STRING, _ARRAY, _UINT64, _INT64, _FLOAT64 = range(13)
_INT_TYPES = frozenset((_UINT8, _INT8, _UINT16, _INT16, _UINT32, _INT32, _UINT64, _INT64))
_FLOAT_TYPES = frozenset((_FLOAT32, _FLOAT64))
_ARRAY_CTYPES = {
    _UINT8: ctypes.c_uint8,
    _INT8: ctypes.c_int8,
    _UINT16: ctypes.c_uint16,
    _INT16: ctypes.c_int16,
    _UINT32: ctypes.c_uint32,
    _INT32: ctypes.c_int32,
    _FLOAT32: ctypes.c_float,
    _BOOL: ctypes.c_int8,
    _UINT64: ctypes.c_uint64,
    _INT64: ctypes.c_int64,
    _FLOAT64: ctypes.c_double,
}

# Keys under these prefixes carry the real shape and dtype of tensors GGUF cannot describe; they
# are applied to the tensors and are not metadata (gguf_train/gguf/__init__.py:31-33).
_RESERVED_PREFIXES = ("gguf_train.shape.", "gguf_train.dtype.")


def _kv_scalar(handle: int, i: int, ktype: int):
    lib = _C.lib
    n = int(lib.gt_gguf_kv_val_str(handle, i, None, 0))
    if n < 0:
        raise RuntimeError(f"GGUF metadata entry {i} cannot be read")
    buf = ctypes.create_string_buffer(n + 1)
    lib.gt_gguf_kv_val_str(handle, i, buf, n + 1)
    text = buf.value.decode("utf-8", errors="replace")
    if ktype in _INT_TYPES:
        return int(text)
    if ktype in _FLOAT_TYPES:
        return float(text)
    if ktype == _BOOL:
        return text == "true"
    return text


def _kv_array(handle: int, i: int) -> list:
    lib = _C.lib
    etype = int(lib.gt_gguf_kv_arr_type(handle, i))
    n = int(lib.gt_gguf_kv_arr_n(handle, i))
    if n <= 0:
        return []
    if etype == _STRING:
        return [(lib.gt_gguf_kv_arr_str(handle, i, j) or b"").decode("utf-8", errors="replace") for j in range(n)]
    ctype = _ARRAY_CTYPES.get(etype)
    data = lib.gt_gguf_kv_arr_data(handle, i)
    if ctype is None or not data:
        raise RuntimeError(f"GGUF metadata entry {i} is an array of an unknown element type ({etype})")
    values = ctypes.cast(data, ctypes.POINTER(ctype * n)).contents[:]
    return [bool(v) for v in values] if etype == _BOOL else values


def _device_index(device) -> int | None:
    if device is None:
        return None
    dev = torch.device(device)
    if dev.type == "cpu":
        return None
    if dev.type != "cuda":
        raise ValueError(f"device {device!r}: only 'cpu' and HIP ('cuda') devices are supported")
    return dev.index if dev.index is not None else torch.cuda.current_device()


def _shape_of(ptr: int) -> tuple:
    nd = int(_C.lib.gt_tensor_ndim(ptr))
    buf = (ctypes.c_int64 * max(nd, 1))()
    _C.lib.gt_tensor_shape(ptr, buf)
    return tuple(int(buf[i]) for i in range(nd))


def _adopt_any(ptr: int, ctx: str):
    _C.check_ptr(ptr, ctx)
    if int(_C.lib.gt_tensor_dtype(ptr)) == _C.GT_Q8_0:
        return adopt_quantized(ptr, _shape_of(ptr), ctx)
    return adopt(ptr, ctx)


class GGUFFile:
    """Opened GGUF archive exposing metadata KV pairs and tensors (gguf_train/gguf/__init__.py:69).

    ``metadata`` maps keys to ``int``, ``float``, ``bool`` or ``str`` values, and to lists of
    those for GGUF arrays.  ``device`` (None / "cpu", or a HIP device) is where the tensors are
    placed; on a HIP device they are read from the file straight into device memory.
    """

    def __init__(self, path: str | Path, dequantize: bool = False, device=None) -> None:
        self.path = str(path)
        dev = _device_index(device)
        self._handle = _C.check_ptr(_C.lib.gt_gguf_open(self.path.encode("utf-8")), f"open GGUF {self.path}")
        try:
            self.metadata: dict[str, object] = {}
            for i in range(int(_C.lib.gt_gguf_n_kv(self._handle))):
                k_raw = _C.lib.gt_gguf_kv_key(self._handle, i)
                key = k_raw.decode("utf-8", errors="replace") if k_raw else f"kv_{i}"
                if key.startswith(_RESERVED_PREFIXES):
                    continue
                ktype = int(_C.lib.gt_gguf_kv_type(self._handle, i))
                self.metadata[key] = _kv_array(self._handle, i) if ktype == _ARRAY else _kv_scalar(self._handle, i, ktype)

            self.tensors: dict[str, torch.Tensor | QuantizedTensor] = {}
            if dev is not None:
                bind_stream(torch.device("cuda", dev))
            for i in range(int(_C.lib.gt_gguf_n_tensors(self._handle))):
                t_raw = _C.lib.gt_gguf_tensor_name(self._handle, i)
                name = t_raw.decode("utf-8", errors="replace")
                deq = 1 if dequantize else 0
                if dev is None:
                    ptr = _C.lib.gt_gguf_get_tensor(self._handle, t_raw, deq)
                else:
                    ptr = _C.lib.gt_gguf_get_tensor_device(self._handle, t_raw, deq, dev)
                self.tensors[name] = _adopt_any(ptr, f"read tensor {name}")
        finally:
            self.close()

    def __getitem__(self, key: str):
        return self.tensors[key]

    def __contains__(self, key: object) -> bool:
        return key in self.tensors

    def __iter__(self):
        return iter(self.tensors)

    def __len__(self) -> int:
        return len(self.tensors)

    def keys(self):
        return self.tensors.keys()

    def values(self):
        return self.tensors.values()

    def items(self):
        return self.tensors.items()

    def get(self, key: str, default=None):
        return self.tensors.get(key, default)

    def close(self) -> None:
        if getattr(self, "_handle", 0):
            _C.lib.gt_gguf_close(self._handle)
            self._handle = 0


def load_gguf(path: str | Path, dequantize: bool = False, return_metadata: bool = False, device=None):
    """Load tensors and metadata from a .gguf file (gguf_train/gguf/__init__.py:133-138)."""
    gf = GGUFFile(path, dequantize=dequantize, device=device)
    if return_metadata:
        return gf.tensors, gf.metadata
    return gf


def _dtype_name(v) -> str:
    if isinstance(v, QuantizedTensor):
        return "q8_0"
    return str(v.dtype).replace("torch.", "")


def inspect_gguf(path: str | Path) -> dict:
    """Metadata and tensor shapes/dtypes of a .gguf file (gguf_train/gguf/__init__.py:258-266)."""
    gf = load_gguf(path, dequantize=False)
    return {
        "path": str(path),
        "n_tensors": len(gf.tensors),
        "metadata": gf.metadata,
        "tensors": {k: {"shape": tuple(v.shape), "dtype": _dtype_name(v)} for k, v in gf.tensors.items()},
    }


__all__ = ["GGUFFile", "load_gguf", "inspect_gguf"]
