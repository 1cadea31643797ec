"""Host mirror of gorelaxor's internal/gguf over libgrx.so.

Names, argument meaning and errors follow the reference package
(github.com/xattribution/gorelaxor, internal/gguf/gguf.go):

    f = Open(path)            # gguf.go:57-113; Parse(b), ReadMeta(path)
    f.Version, f.Names(), f.Keys(), f.Has(name), f.Tensors[name].Dims/.Type
    f.Int(key, d), f.Float(key, d), f.Bool(key, d), f.String(key, d)
    f.Strings(key), f.Floats(key), f.Ints(key)
    f.Float32(name)           # any tensor widened to float32
    f.Weight(name)            # a Q8_0 tensor straight to its device tiles

Parsing, settings and Float32 run on the host and need no GPU; Weight packs
on the GPU.  Errors raise GrxError with the reference's message.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import _lib
from .kern import Context, Weight as KernWeight, default_context

TypeF32, TypeF16, TypeQ8_0, TypeBF16 = 0, 1, 8, 30


@dataclass
class Tensor:
    """gguf.Tensor: Dims in GGUF order (Dims[0] the row length)."""
    Name: str
    Dims: list
    Type: int

    def Elems(self) -> int:
        n = 1
        for d in self.Dims:
            n *= d
        return n


class File:
    def __init__(self, handle):
        self.handle = handle
        L = _lib.lib()
        self.Version = L.grx_gguf_version(handle)
        self._names = [L.grx_gguf_tensor_name(handle, i).decode() for i in range(L.grx_gguf_n_tensors(handle))]
        self.Tensors = {}
        for n in self._names:
            t, nd = C.c_int(), C.c_int()
            dims = (C.c_int64 * 4)()
            _lib.call("grx_gguf_tensor_info", handle, n.encode(), C.byref(t), C.byref(nd), dims)
            self.Tensors[n] = Tensor(n, [int(dims[i]) for i in range(nd.value)], t.value)

    def Names(self) -> list:
        return list(self._names)

    def Keys(self) -> list:
        L = _lib.lib()
        return [L.grx_gguf_key(self.handle, i).decode("utf-8", "replace") for i in range(L.grx_gguf_n_keys(self.handle))]

    def Has(self, name: str) -> bool:
        return bool(_lib.lib().grx_gguf_has(self.handle, name.encode()))

    def Int(self, key: str, default: int) -> int:
        return int(_lib.lib().grx_gguf_int(self.handle, key.encode(), default))

    def Float(self, key: str, default: float) -> float:
        return float(_lib.lib().grx_gguf_float(self.handle, key.encode(), default))

    def Bool(self, key: str, default: bool) -> bool:
        return bool(_lib.lib().grx_gguf_bool(self.handle, key.encode(), int(default)))

    def String(self, key: str, default: str) -> str:
        s = _lib.lib().grx_gguf_string(self.handle, key.encode(), None)
        return default if s is None else s.decode("utf-8", "replace")

    def _len(self, key: str) -> int:
        return max(0, int(_lib.lib().grx_gguf_array_len(self.handle, key.encode())))

    def Strings(self, key: str) -> list:
        L = _lib.lib()
        return [L.grx_gguf_array_string(self.handle, key.encode(), i).decode("utf-8", "replace")
                for i in range(self._len(key))]

    def Floats(self, key: str) -> np.ndarray:
        L = _lib.lib()
        return np.array([L.grx_gguf_array_float(self.handle, key.encode(), i) for i in range(self._len(key))],
                        np.float32)

    def Ints(self, key: str) -> list:
        L = _lib.lib()
        return [int(L.grx_gguf_array_int(self.handle, key.encode(), i)) for i in range(self._len(key))]

    def Float32(self, name: str) -> np.ndarray:
        t = self.Tensors.get(name)
        n = t.Elems() if t else 0
        out = np.zeros(n, np.float32)
        _lib.call("grx_gguf_float32", self.handle, name.encode(), out.ctypes.data_as(C.c_void_p), n)
        return out

    def WeightShape(self, name: str) -> tuple:
        r, c = C.c_int64(), C.c_int64()
        _lib.call("grx_gguf_weight_shape", self.handle, name.encode(), C.byref(r), C.byref(c))
        return r.value, c.value

    def Weight(self, name: str, ctx: Context | None = None) -> KernWeight:
        """File.Weight of a Q8_0 tensor, packed into HBM from the file."""
        ctx = ctx or default_context()
        h = C.c_void_p()
        _lib.call("grx_gguf_weight_q8", ctx.handle, self.handle, name.encode(), C.byref(h))
        L = _lib.lib()
        return KernWeight(h, L.grx_weight_rows(h), L.grx_weight_cols(h), ctx)

    def close(self):
        if self.handle:
            _lib.call("grx_gguf_close", self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def Open(path) -> File:
    h = C.c_void_p()
    _lib.call("grx_gguf_open", str(path).encode(), C.byref(h))
    return File(h)


def Parse(b) -> File:
    buf = np.frombuffer(bytes(b), np.uint8)
    h = C.c_void_p()
    _lib.call("grx_gguf_parse", buf.ctypes.data_as(C.c_void_p) if buf.size else None, buf.size, C.byref(h))
    return File(h)


def ReadMeta(path) -> File:
    h = C.c_void_p()
    _lib.call("grx_gguf_read_meta", str(path).encode(), C.byref(h))
    return File(h)
