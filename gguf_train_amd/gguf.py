"""GGUF files: metadata and tensors, on the host or straight into GPU memory.

A Python front end over libgt_attn's own GGUF reader (the gt_gguf_* entry points).  What a
caller sees is the read side of the reference's `gguf_train.gguf`
(gguf_train/gguf/__init__.py:69-138 and 258-266): `GGUFFile` reads the metadata and every
tensor when it is opened and closes the file; it is a read-only mapping of tensor names to
tensors with `.metadata` (int / float / bool / str values, lists for GGUF arrays; the
reserved `gguf_train.shape.` / `gguf_train.dtype.` keys are applied to the tensors and left
out); `load_gguf` and `inspect_gguf` keep their signatures and results.  Added here: a
`device` argument - on a HIP device each tensor is streamed from the file into device memory
(gt_gguf_get_tensor_device) instead of going through a host copy - and Q8_0 tensors that are
not dequantized come back as `QuantizedTensor` (the 34-byte ggml blocks), which the attention
entry points accept as k / v.
"""

from __future__ import annotations

import contextlib
import ctypes
import enum
from collections.abc import Mapping
from pathlib import Path

import numpy as np
import torch

from . import _C
from ._bridge import QuantizedTensor, adopt, adopt_quantized, bind_stream


class ValueType(enum.IntEnum):
    """GGUF metadata value types (the numbering of the GGUF file format)."""

    UINT8 = 0
    INT8 = 1
    UINT16 = 2
    INT16 = 3
    UINT32 = 4
    INT32 = 5
    FLOAT32 = 6
    BOOL = 7
    STRING = 8
    ARRAY = 9
    UINT64 = 10
    INT64 = 11
    FLOAT64 = 12


# Element layout of numeric arrays in the reader's buffers (little-endian, as in the file).
_NUMPY_ELEMENT = {
    ValueType.UINT8: np.dtype("<u1"), ValueType.INT8: np.dtype("<i1"),
    ValueType.UINT16: np.dtype("<u2"), ValueType.INT16: np.dtype("<i2"),
    ValueType.UINT32: np.dtype("<u4"), ValueType.INT32: np.dtype("<i4"),
    ValueType.UINT64: np.dtype("<u8"), ValueType.INT64: np.dtype("<i8"),
    ValueType.FLOAT32: np.dtype("<f4"), ValueType.FLOAT64: np.dtype("<f8"),
    ValueType.BOOL: np.dtype("<i1"),
}

# How the reader's text form of a scalar becomes a Python value.
_PARSE_SCALAR = {t: int for t in (ValueType.UINT8, ValueType.INT8, ValueType.UINT16, ValueType.INT16,
                                  ValueType.UINT32, ValueType.INT32, ValueType.UINT64, ValueType.INT64)}
_PARSE_SCALAR.update({ValueType.FLOAT32: float, ValueType.FLOAT64: float, ValueType.BOOL: lambda s: s == "true"})

# Keys that record the real shape / dtype of a tensor GGUF cannot describe; the reader applies
# them to the tensors, so they are not metadata.
RESERVED_KEY_PREFIXES = ("gguf_train.shape.", "gguf_train.dtype.")


def _text(raw: bytes | None) -> str:
    return (raw or b"").decode("utf-8", errors="replace")


class _Entries:
    """Decodes the metadata entries of an open reader handle into Python values."""

    def __init__(self, handle: int):
        self.handle = handle
        self.lib = _C.lib

    def __len__(self) -> int:
        return int(self.lib.gt_gguf_n_kv(self.handle))

    def key(self, i: int) -> str:
        raw = self.lib.gt_gguf_kv_key(self.handle, i)
        return _text(raw) if raw else f"kv_{i}"

    def value(self, i: int):
        kind = int(self.lib.gt_gguf_kv_type(self.handle, i))
        if kind == ValueType.ARRAY:
            return self._array(i)
        # scalars come as text: ask for the length, then for the characters
        n = int(self.lib.gt_gguf_kv_val_str(self.handle, i, None, 0))
        if n < 0:
            raise RuntimeError(f"GGUF metadata entry {i} cannot be read")
        buf = ctypes.create_string_buffer(n + 1)
        self.lib.gt_gguf_kv_val_str(self.handle, i, buf, n + 1)
        parse = _PARSE_SCALAR.get(kind, str)
        return parse(_text(buf.value))

    def _array(self, i: int) -> list:
        kind = int(self.lib.gt_gguf_kv_arr_type(self.handle, i))
        n = int(self.lib.gt_gguf_kv_arr_n(self.handle, i))
        if n <= 0:
            return []
        if kind == ValueType.STRING:
            return [_text(self.lib.gt_gguf_kv_arr_str(self.handle, i, j)) for j in range(n)]
        element = _NUMPY_ELEMENT.get(kind)
        addr = self.lib.gt_gguf_kv_arr_data(self.handle, i)
        if element is None or not addr:
            raise RuntimeError(f"GGUF metadata entry {i} is an array of an unknown element type ({kind})")
        values = np.frombuffer(ctypes.string_at(addr, n * element.itemsize), dtype=element)
        return values.astype(bool).tolist() if kind == ValueType.BOOL else values.tolist()

    def as_dict(self) -> dict:
        out = {}
        for i in range(len(self)):
            key = self.key(i)
            if not key.startswith(RESERVED_KEY_PREFIXES):
                out[key] = self.value(i)
        return out


def _hip_device(device) -> int | None:
    """The HIP device index for `device`, or None for the host."""
    if device is None:
        return None
    dev = torch.device(device)
    if dev.type == "cpu":
        return None
    if dev.type != "cuda":
        raise ValueError(f"device {device!r}: only 'cpu' and HIP ('cuda') devices are supported")
    return torch.cuda.current_device() if dev.index is None else dev.index


def _result(ptr: int, what: str):
    """A tensor handle from the reader as a torch tensor, or a QuantizedTensor for Q8_0 blocks."""
    _C.check_ptr(ptr, what)
    if int(_C.lib.gt_tensor_dtype(ptr)) != _C.GT_Q8_0:
        return adopt(ptr, what)
    nd = int(_C.lib.gt_tensor_ndim(ptr))
    dims = (ctypes.c_int64 * max(nd, 1))()
    _C.lib.gt_tensor_shape(ptr, dims)
    return adopt_quantized(ptr, tuple(dims[:nd]), what)


@contextlib.contextmanager
def _reader(path: str):
    handle = _C.check_ptr(_C.lib.gt_gguf_open(path.encode("utf-8")), f"open GGUF {path}")
    try:
        yield handle
    finally:
        _C.lib.gt_gguf_close(handle)


class GGUFFile(Mapping):
    """A GGUF file read into memory: a mapping of tensor names to tensors, plus `metadata`.

    Everything is read when the object is built and the file is closed again.  `dequantize`
    turns quantized tensors into float32; `device` (None / "cpu", or a HIP device) is where
    the tensors are placed - on a HIP device they go from the file straight to device memory.
    """

    def __init__(self, path: str | Path, dequantize: bool = False, device=None) -> None:
        self.path = str(path)
        hip = _hip_device(device)
        with _reader(self.path) as handle:
            self.metadata: dict[str, object] = _Entries(handle).as_dict()
            if hip is not None:
                bind_stream(torch.device("cuda", hip))
            flag = 1 if dequantize else 0
            self.tensors: dict[str, torch.Tensor | QuantizedTensor] = {}
            for i in range(int(_C.lib.gt_gguf_n_tensors(handle))):
                raw = _C.lib.gt_gguf_tensor_name(handle, i)
                name = _text(raw)
                ptr = (_C.lib.gt_gguf_get_tensor(handle, raw, flag) if hip is None
                       else _C.lib.gt_gguf_get_tensor_device(handle, raw, flag, hip))
                self.tensors[name] = _result(ptr, f"read tensor {name}")

    def __getitem__(self, name: str):
        return self.tensors[name]

    def __iter__(self):
        return iter(self.tensors)

    def __len__(self) -> int:
        return len(self.tensors)

    def close(self) -> None:
        """Nothing to release: the file was closed once it had been read."""

    # Identity equality and hashing, as the reference's GGUFFile (a plain class,
    # gguf_train/gguf/__init__.py:69): Mapping would compare the tensor dicts (ambiguous for
    # multi-element tensors) and make instances unhashable.
    __eq__ = object.__eq__
    __hash__ = object.__hash__


def load_gguf(path: str | Path, dequantize: bool = False, return_metadata: bool = False, device=None):
    """The tensors of a .gguf file: the GGUFFile, or (tensors, metadata) with return_metadata."""
    f = GGUFFile(path, dequantize=dequantize, device=device)
    return (f.tensors, f.metadata) if return_metadata else f


def inspect_gguf(path: str | Path) -> dict:
    """Path, tensor count, metadata, and the shape and dtype of every tensor of a .gguf file."""
    f = GGUFFile(path, dequantize=False)

    def describe(t) -> dict:
        dtype = "q8_0" if isinstance(t, QuantizedTensor) else str(t.dtype).replace("torch.", "")
        return {"shape": tuple(t.shape), "dtype": dtype}

    return {"path": str(path), "n_tensors": len(f), "metadata": f.metadata,
            "tensors": {name: describe(t) for name, t in f.items()}}


__all__ = ["GGUFFile", "ValueType", "load_gguf", "inspect_gguf"]
