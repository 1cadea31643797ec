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


def frames_out(frames: int, causal: bool = False) -> int:
    """Encoder frames for `frames` mel frames (three stride-2 halvings,
    subOut of conformer/encoder.go:33-38: a causal pre-encoder pads two
    before and one after)."""
    for _ in range(3):
        frames = frames // 2 + 1 if causal else (frames - 1) // 2 + 1
    return frames


def stream_geom(hp: dict, right: int) -> dict:
    """newGeom (conformer/stream.go:23-69): a cache-aware model's chunking
    for right context `right`: chunks of 8*(right+1) mel frames (the first
    1+8*right) led by the 9 frames before them, whose first 2 encoder rows
    are dropped; attention over `left` earlier rows."""
    if hp.get("att_style", "regular") != "chunked_limited":
        raise ValueError("conformer: this model can't stream")
    left = -1
    choices = hp.get("context_choices") or []
    for lc, rc in choices:
        if rc == right:
            left = lc
    if not choices and right == hp.get("att_right", -1):
        left = hp.get("att_left", -1)
    if left < 0:
        raise ValueError(f"conformer: the model wasn't trained for a right context of {right}")
    sub = hp.get("subsampling", 8)
    cache = hp.get("pre_encode_cache", -1)
    cache = sub + 1 if cache < 0 else cache
    drop = hp.get("drop_extra", -1)
    drop = 1 + (cache - 1) // sub if drop < 0 else drop
    first = hp.get("sampling_frames_first", -1)
    first = 1 if first < 0 else first
    chunk = right + 1
    return dict(right=right, chunk=chunk, left=left, left_chunks=left // chunk, mel_first=first + sub * right,
                mel_next=sub * chunk, mel_cache=cache, drop=drop, sample_first=first, sub=sub)


def mel_chunks(mel: np.ndarray, g: dict, final: bool = True):
    """The chunks melChunker.chunks (conformer/stream.go:187-226) cuts from
    mel frames [n_mels][frames] that are all there: (frames [n_mels][nf]
    (the cache frames, zero before the first, then the chunk), length,
    first) for each, a last short chunk when final (a remainder shorter
    than the sampling frames is dropped)."""
    nm, avail = mel.shape
    out, buf, n = [], 0, 0
    while buf < avail:
        size, need = (g["mel_next"], g["sub"]) if n else (g["mel_first"], g["sample_first"])
        if not final and buf + size > avail:
            break
        k = min(size, avail - buf)
        if k < need:
            break
        cache = g["mel_cache"] if n else 0
        ch = np.zeros((nm, cache + k), np.float32)
        lo = buf - cache
        src = mel[:, max(lo, 0):buf + k]
        ch[:, ch.shape[1] - src.shape[1]:] = src
        out.append((ch, cache + k, n == 0))
        buf += size
        n += 1
    return out


def _hparams(hp: dict) -> "_lib.ConformerHParams":
    """grx_conformer_hparams from HParams-named settings (conformer/
    model.go:15-44): att_style "regular" or "chunked_limited", the limits -1
    where there are none, causal_sub as readEncoder defaults it."""
    chunked = hp.get("att_style", "regular") == "chunked_limited"
    h = _lib.ConformerHParams(d=hp["d"], heads=hp["heads"], layers=hp["layers"], dff=hp["dff"],
                              conv_kernel=hp["conv_kernel"], sub_channels=hp["sub_channels"],
                              n_mels=hp["n_mels"], xscaling=int(bool(hp.get("xscaling", True))),
                              conv_ln=int(hp.get("conv_norm", "batch_norm") == "layer_norm"),
                              att_chunked=int(chunked), att_left=hp.get("att_left", -1),
                              att_right=hp.get("att_right", -1), conv_left=hp.get("conv_left", -1),
                              conv_right=hp.get("conv_right", -1),
                              causal_sub=int(bool(hp.get("causal_sub", chunked))),
                              pre_encode_cache=hp.get("pre_encode_cache", -1), drop_extra=hp.get("drop_extra", -1),
                              sampling_frames_first=hp.get("sampling_frames_first", -1))
    choices = list(hp.get("context_choices") or [])
    if len(choices) > 8:
        raise ValueError("at most 8 attention context choices")
    h.n_context_choices = len(choices)
    for i, (lc, rc) in enumerate(choices):
        h.context_choices[i][0], h.context_choices[i][1] = lc, rc
    return h


class ConformerEncoder:
    def __init__(self, hp: dict, tensors: dict | None = None, ctx: Context | None = None):
        self.ctx = ctx or default_context()
        self.hp = dict(hp)
        h = _hparams(hp)
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
                                              "n_mels", "att_left", "att_right", "conv_left", "conv_right",
                                              "pre_encode_cache", "drop_extra", "sampling_frames_first")}
        self.hp["xscaling"] = bool(h.xscaling)
        self.hp["conv_norm"] = "layer_norm" if h.conv_ln else "batch_norm"
        self.hp["att_style"] = "chunked_limited" if h.att_chunked else "regular"
        self.hp["causal_sub"] = bool(h.causal_sub)
        self.hp["context_choices"] = [(h.context_choices[i][0], h.context_choices[i][1])
                                      for i in range(h.n_context_choices)]
        return self

    @property
    def causal(self) -> bool:
        return bool(self.hp.get("causal_sub", self.hp.get("att_style", "regular") == "chunked_limited"))

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
        T = frames_out(frames, self.causal)
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


class ConformerStream:
    """Cache-aware streaming (conformer/stream.go:23-88, 241-307) of `batch`
    streams stepped together: each step takes one chunk per stream as the
    reference's chunker cuts them (mel_chunks) and returns each stream's
    encoder rows for it.  Right context `right` is one of the model's
    trained choices."""

    def __init__(self, enc: ConformerEncoder, right: int, batch: int = 1):
        self.enc = enc
        self.batch = batch
        out = C.c_void_p()
        _lib.call("grx_conformer_stream_create", enc.handle, right, batch, C.byref(out))
        self.handle = out
        g = _lib.ConformerStreamGeom()
        _lib.call("grx_conformer_stream_geometry", self.handle, C.byref(g))
        self.geom = {k: getattr(g, k) for k, _ in _lib.ConformerStreamGeom._fields_}
        self.geom["sub"] = 8

    def step(self, mel: np.ndarray, length) -> list[np.ndarray]:
        """mel [batch][n_mels][nf] (or [n_mels][nf] for one stream), length
        the real frames of each: each stream's rows [L][d]."""
        mel = np.ascontiguousarray(mel, np.float32)
        if mel.ndim == 2:
            mel = mel[None]
        batch, nm, nf = mel.shape
        assert batch == self.batch and nm == self.enc.hp["n_mels"]
        ln = np.ascontiguousarray(np.broadcast_to(np.asarray(length, np.int32), (batch,)))
        d, chunk = self.enc.hp["d"], self.geom["chunk"]
        out = np.zeros((batch, chunk, d), np.float32)
        lens = np.zeros(batch, np.int32)
        _lib.call("grx_conformer_stream_step", self.handle, mel.ctypes.data_as(C.c_void_p), nf,
                  ln.ctypes.data_as(C.c_void_p), out.ctypes.data_as(C.c_void_p), lens.ctypes.data_as(C.c_void_p))
        return [out[b, :lens[b]] for b in range(batch)]

    def step_dev(self, mel_ptr: int, nf: int, length, out_ptr: int) -> np.ndarray:
        """The step with mel [batch][n_mels][nf] and out [batch][chunk][d] in
        device memory: the rows of each stream."""
        ln = np.ascontiguousarray(np.broadcast_to(np.asarray(length, np.int32), (self.batch,)))
        lens = np.zeros(self.batch, np.int32)
        _lib.call("grx_conformer_stream_step_dev", self.handle, C.c_void_p(mel_ptr), nf,
                  ln.ctypes.data_as(C.c_void_p), C.c_void_p(out_ptr), lens.ctypes.data_as(C.c_void_p))
        return lens

    def close(self):
        if self.handle:
            _lib.call("grx_conformer_stream_destroy", self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
