"""A small GGUF (v3) writer for the loader tests: key/values of every value
type, tensors as raw ggml-layout bytes (F32, F16, Q8_0 blocks, I32), the
data section aligned as the format specifies.  Test helper only."""
from __future__ import annotations

import struct

import numpy as np

GGUF_MAGIC = b"GGUF"
# GGUF value types
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q",
           I64: "<q", F64: "<d"}
# ggml types
T_F32, T_F16, T_Q8_0, T_I32 = 0, 1, 8, 26


def _str(s: str | bytes) -> bytes:
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def _value(vtype: int, v) -> bytes:
    if vtype == STRING:
        return _str(v)
    if vtype == ARRAY:
        etype, items = v
        out = struct.pack("<IQ", etype, len(items))
        return out + b"".join(_value(etype, x) for x in items)
    return struct.pack(_SCALAR[vtype], v)


class GgufFile:
    """kv: list of (key, vtype, value); tensors: list of (name, ggml_type, ne, raw bytes)."""

    def __init__(self, alignment: int = 32, version: int = 3):
        self.alignment, self.version = alignment, version
        self.kv: list = []
        self.tensors: list = []

    def add_kv(self, key: str, vtype: int, value):
        self.kv.append((key, vtype, value))

    def add_tensor(self, name: str, gtype: int, ne, raw: bytes):
        self.tensors.append((name, gtype, list(ne), bytes(raw)))

    def bytes(self, offsets=None, n_dims_override=None) -> bytes:
        head = GGUF_MAGIC + struct.pack("<IQQ", self.version, len(self.tensors), len(self.kv))
        for key, vtype, value in self.kv:
            head += _str(key) + struct.pack("<I", vtype) + _value(vtype, value)
        data = b""
        infos = b""
        for i, (name, gtype, ne, raw) in enumerate(self.tensors):
            pad = (-len(data)) % self.alignment
            data += b"\0" * pad
            off = len(data) if offsets is None else offsets[i]
            nd = len(ne) if n_dims_override is None else n_dims_override
            infos += _str(name) + struct.pack("<I", nd) + b"".join(struct.pack("<Q", d) for d in ne)
            infos += struct.pack("<IQ", gtype, off)
            data += raw
        head += infos
        head += b"\0" * ((-len(head)) % self.alignment)
        return head + data

    def write(self, path, **kw):
        with open(path, "wb") as f:
            f.write(self.bytes(**kw))


def table_f32(a: np.ndarray):
    """(T_F32, ne, bytes) of a 2-D float32 array [rows, cols] (ggml ne = (cols, rows))."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    return T_F32, [a.shape[1], a.shape[0]], a.tobytes()


def table_f16(a: np.ndarray):
    a = np.ascontiguousarray(a, dtype=np.float16)
    return T_F16, [a.shape[1], a.shape[0]], a.tobytes()


def table_q8_0(q: np.ndarray, cols: int):
    """q: uint8 [rows, cols/32*34] Q8_0 blocks."""
    q = np.ascontiguousarray(q, dtype=np.uint8)
    return T_Q8_0, [cols, q.shape[0]], q.tobytes()
