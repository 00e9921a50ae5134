"""Builds GGUF files byte by byte for the reader tests, from the published format:

    "GGUF" | u32 version | u64 n_tensors | u64 n_kv
    n_kv x      (string key, u32 value type, value)         arrays: u32 elem type, u64 n, elements
    n_tensors x (string name, u32 n_dims, u64 ne[n_dims], u32 ggml type, u64 offset)
    zero padding to the alignment, then each tensor's bytes padded to the alignment

Strings are a u64 length and UTF-8 bytes.  The builder writes what it is told, so tests can
also make files a reader must refuse.
"""

from __future__ import annotations

import struct
from pathlib import Path

# value types (enum gguf_type)
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_PACK = {U8: "B", I8: "b", U16: "H", I16: "h", U32: "I", I32: "i", F32: "f", BOOL: "?", U64: "Q", I64: "q",
         F64: "d"}

# tensor types (enum ggml_type)
T_F32, T_F16, T_Q4_0, T_Q8_0, T_I8, T_I16, T_I32, T_I64, T_F64, T_BF16 = 0, 1, 2, 8, 24, 25, 26, 27, 28, 30


def _str(s) -> bytes:
    b = s if isinstance(s, bytes) else s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _val(vtype: int, v) -> bytes:
    return _str(v) if vtype == STRING else struct.pack("<" + _PACK[vtype], v)


class GGUFBuilder:
    def __init__(self, version: int = 3, alignment: int = 32):
        self.version = version
        self.alignment = alignment
        self.kvs: list[bytes] = []
        self.tensors: list[tuple] = []  # (name, ne, ggml type, data, offset or None)

    def kv(self, key: str, vtype: int, value, elem: int | None = None) -> "GGUFBuilder":
        body = _str(key) + struct.pack("<I", vtype)
        if vtype == ARRAY:
            body += struct.pack("<IQ", elem, len(value)) + b"".join(_val(elem, x) for x in value)
        else:
            body += _val(vtype, value)
        self.kvs.append(body)
        return self

    def tensor(self, name: str, ne, ttype: int, data: bytes, offset: int | None = None) -> "GGUFBuilder":
        self.tensors.append((name, list(ne), ttype, bytes(data), offset))
        return self

    def _pad(self, n: int) -> int:
        return (-n) % self.alignment

    def to_bytes(self, truncate: int = 0) -> bytes:
        infos, blobs, off = [], [], 0
        for name, ne, ttype, data, forced in self.tensors:
            infos.append(_str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", d) for d in ne)
                         + struct.pack("<IQ", ttype, off if forced is None else forced))
            blobs.append(data + bytes(self._pad(len(data))))
            off += len(blobs[-1])
        head = b"GGUF" + struct.pack("<IQQ", self.version, len(self.tensors), len(self.kvs))
        head += b"".join(self.kvs) + b"".join(infos)
        head += bytes(self._pad(len(head)))
        out = head + b"".join(blobs)
        return out[: len(out) - truncate] if truncate else out

    def write(self, path, truncate: int = 0) -> Path:
        path = Path(path)
        path.write_bytes(self.to_bytes(truncate))
        return path
