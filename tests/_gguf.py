"""GGUF byte builders for tests, in the layout internal/gguf/gguf.go:292-354
reads (magic, version, tensor and key counts, keys, tensor table, data at
32-byte alignment): `build` is the general form and `one` a single-tensor
file with raw dimensions, type and offset (the shapes gguf_test.go and
hostile_test.go feed the reader)."""
from __future__ import annotations

import struct

import numpy as np

F32, F16, Q8_0, BF16 = 0, 1, 8, 30
T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STR, T_ARR, T_U64, T_I64, T_F64 = range(13)
_SCALAR = {T_U8: "<B", T_I8: "<b", T_U16: "<H", T_I16: "<h", T_U32: "<I", T_I32: "<i", T_F32: "<f",
           T_BOOL: "<?", T_U64: "<Q", T_I64: "<q", T_F64: "<d"}


def gstr(s) -> bytes:
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def gval(t: int, v, et: int | None = None) -> bytes:
    """A value of type t (without its type tag); arrays give (et, items)."""
    if t == T_STR:
        return gstr(v)
    if t == T_ARR:
        return struct.pack("<IQ", et, len(v)) + b"".join(gval(et, x) for x in v)
    return struct.pack(_SCALAR[t], v)


def kv(key: str, t: int, v, et: int | None = None) -> bytes:
    return gstr(key) + struct.pack("<I", t) + gval(t, v, et)


def build(kvs: list, tensors: list, version: int = 3, align: int = 32) -> bytes:
    """kvs: encoded key-value entries (kv(...)); tensors: (name, dims, type,
    data bytes), laid out at `align`-byte offsets."""
    b = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kvs)) + b"".join(kvs)
    off = 0
    for name, dims, typ, data in tensors:
        b += gstr(name) + struct.pack("<I", len(dims)) + struct.pack(f"<{len(dims)}Q", *dims)
        b += struct.pack("<IQ", typ, off)
        off += len(data)
        off += (align - off % align) % align
    b += bytes((align - len(b) % align) % align)
    for _, _, _, data in tensors:
        b += bytes(data)
        b += bytes((align - len(b) % align) % align)
    return b


def one(kvb: bytes, nkv: int, dims: list, typ: int, off: int, pad: int) -> bytes:
    """One tensor named "t" with raw dims, type and offset, then `pad` data
    bytes (hostile_test.go's builder)."""
    b = b"GGUF" + struct.pack("<IQQ", 3, 1, nkv) + kvb
    b += struct.pack("<Q", 1) + b"t" + struct.pack("<I", len(dims))
    b += b"".join(struct.pack("<Q", d % (1 << 64)) for d in dims)
    b += struct.pack("<IQ", typ, off % (1 << 64))
    b += bytes((32 - len(b) % 32) % 32)
    return b + bytes(pad)


def f16_bytes(v) -> bytes:
    return np.asarray(v, np.float32).astype(np.float16).tobytes()


def q8_block(d: float, q) -> bytes:
    return np.float16(d).tobytes() + np.asarray(q, np.int8).tobytes()
