"""Host driver of the FastConformer encoder on the GPU.

Mirrors Model.encode of gorelaxor's conformer package (github.com/
xattribution/gorelaxor, conformer/encoder.go:432-489): tensors bound by the
names conformer/model.go:370-422 reads, log-mel features in Mel.Compute's
[mels][frames] layout, a batch of utterances of one frame count at once.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from .kern import Context, default_context


def frames_out(frames: int) -> int:
    """Encoder frames for `frames` mel frames (three stride-2 halvings)."""
    for _ in range(3):
        frames = (frames - 1) // 2 + 1
    return frames


class ConformerEncoder:
    def __init__(self, hp: dict, tensors: dict | None = None, ctx: Context | None = None):
        self.ctx = ctx or default_context()
        self.hp = dict(hp)
        h = _lib.ConformerHParams(d=hp["d"], heads=hp["heads"], layers=hp["layers"], dff=hp["dff"],
                                  conv_kernel=hp["conv_kernel"], sub_channels=hp["sub_channels"],
                                  n_mels=hp["n_mels"], xscaling=int(bool(hp.get("xscaling", True))),
                                  conv_ln=int(hp.get("conv_norm", "batch_norm") == "layer_norm"))
        out = C.c_void_p()
        _lib.call("grx_conformer_create", self.ctx.handle, C.byref(h), C.byref(out))
        self.handle = out
        if tensors:
            for name, arr in tensors.items():
                self.set_tensor(name, arr)

    @classmethod
    def from_gguf(cls, path: str, ctx: Context | None = None) -> "ConformerEncoder":
        """The encoder of a FastConformer GGUF file (conformer.Load,
        conformer/model.go:163-422): Q8_0 linear weights go to the device as
        stored."""
        self = cls.__new__(cls)
        self.handle = None
        self.ctx = ctx or default_context()
        h = _lib.ConformerHParams()
        out = C.c_void_p()
        _lib.call("grx_conformer_load_gguf", self.ctx.handle, str(path).encode(), C.byref(h), C.byref(out))
        self.handle = out
        self.hp = {k: getattr(h, k) for k in ("d", "heads", "layers", "dff", "conv_kernel", "sub_channels",
                                              "n_mels")}
        self.hp["xscaling"] = bool(h.xscaling)
        self.hp["conv_norm"] = "layer_norm" if h.conv_ln else "batch_norm"
        return self

    def set_tensor(self, name: str, arr: np.ndarray) -> None:
        a = np.ascontiguousarray(arr)
        _lib.call("grx_conformer_set_tensor", self.handle, name.encode(), a.ctypes.data_as(C.c_void_p), a.nbytes)

    def encode(self, mel: np.ndarray, valid) -> tuple[np.ndarray, np.ndarray]:
        """mel [batch][n_mels][frames] (or [n_mels][frames]) and the valid
        frames of each: (out [batch][T][d], lens [batch])."""
        mel = np.ascontiguousarray(mel, np.float32)
        if mel.ndim == 2:
            mel = mel[None]
        batch, nm, frames = mel.shape
        assert nm == self.hp["n_mels"]
        v = np.ascontiguousarray(np.broadcast_to(np.asarray(valid, np.int32), (batch,)))
        T = frames_out(frames)
        out = np.zeros((batch, T, self.hp["d"]), np.float32)
        lens = np.zeros(batch, np.int32)
        _lib.call("grx_conformer_encode", self.handle, mel.ctypes.data_as(C.c_void_p), batch, frames,
                  v.ctypes.data_as(C.c_void_p), out.ctypes.data_as(C.c_void_p), lens.ctypes.data_as(C.c_void_p))
        return out, lens

    def encode_dev(self, mel_ptr: int, batch: int, frames: int, valid, out_ptr: int) -> None:
        """The encode with mel and out in device memory (pointers)."""
        v = np.ascontiguousarray(np.broadcast_to(np.asarray(valid, np.int32), (batch,)))
        _lib.call("grx_conformer_encode_dev", self.handle, C.c_void_p(mel_ptr), batch, frames,
                  v.ctypes.data_as(C.c_void_p), C.c_void_p(out_ptr))

    def close(self):
        if self.handle:
            _lib.call("grx_conformer_destroy", self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
