"""Host driver of the whisper-shaped Q8_0 text decoder on the GPU.

Mirrors the decoder side of gorelaxor's whisper package (github.com/
xattribution/gorelaxor, whisper/decoder.go, whisper/transcribe.go): tensors
bound by their ggml names (Model.bind, whisper/model.go:376-401), the
encoder output turned into cross-attention keys and values once
(whisper/encoder.go:120-143), then decode / greedy steps that stay on the
device.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from .kern import Context, default_context


class WhisperDecoder:
    """One decode session, or `streams` (2, 4 or 8) independent sessions
    stepping together with shared weights (each its own encoder output)."""

    def __init__(self, hp: dict, tensors: dict | None = None, ctx: Context | None = None, streams: int = 1):
        self.ctx = ctx or default_context()
        self.hp = dict(hp)
        self.streams = streams
        h = _lib.WhisperHParams(**{k: int(hp[k]) for k in ("n_vocab", "n_text_ctx", "n_state", "n_head",
                                                          "n_layer", "n_audio_ctx")})
        out = C.c_void_p()
        _lib.call("grx_whisper_create_streams", self.ctx.handle, C.byref(h), streams, C.byref(out))
        self.handle = out
        if tensors:
            for name, arr in tensors.items():
                self.set_tensor(name, arr)

    @classmethod
    def from_ggml(cls, path: str, ctx: Context | None = None, streams: int = 1) -> "WhisperDecoder":
        """A decoder from a whisper.cpp (ggml) model file (whisper.Load,
        whisper/model.go:93-225): Q8_0 matrices go to the device as stored."""
        self = cls.__new__(cls)
        self.handle = None
        self.ctx = ctx or default_context()
        self.streams = streams
        h = _lib.WhisperHParams()
        out = C.c_void_p()
        _lib.call("grx_whisper_load_ggml", self.ctx.handle, str(path).encode(), streams, C.byref(h), C.byref(out))
        self.handle = out
        self.hp = {k: int(getattr(h, k)) for k in ("n_vocab", "n_text_ctx", "n_state", "n_head", "n_layer",
                                                   "n_audio_ctx")}
        return self

    def set_tensor(self, name: str, arr: np.ndarray) -> None:
        a = np.ascontiguousarray(arr)
        _lib.call("grx_whisper_set_tensor", self.handle, name.encode(), a.ctypes.data_as(C.c_void_p), a.nbytes)

    def set_encoder_output(self, enc: np.ndarray) -> None:
        e = np.ascontiguousarray(enc, np.float32)
        _lib.call("grx_whisper_set_encoder_output", self.handle, e.ctypes.data_as(C.c_void_p),
                  e.size // self.hp["n_state"])

    def set_encoder_output_stream(self, stream: int, enc: np.ndarray) -> None:
        e = np.ascontiguousarray(enc, np.float32)
        _lib.call("grx_whisper_set_encoder_output_stream", self.handle, stream, e.ctypes.data_as(C.c_void_p),
                  e.size // self.hp["n_state"])

    def greedy_streams(self, prompts, n_steps: int) -> np.ndarray:
        """Greedy decoding of every stream: prompts [streams][n_prompt] ->
        tokens [streams][n_steps + 1]."""
        p = np.ascontiguousarray(prompts, np.int32).reshape(self.streams, -1)
        out = np.zeros((self.streams, n_steps + 1), np.int32)
        _lib.call("grx_whisper_greedy_streams", self.handle, p.ctypes.data_as(C.c_void_p), p.shape[1], n_steps,
                  out.ctypes.data_as(C.c_void_p))
        return out

    def reset(self) -> None:
        _lib.call("grx_whisper_reset", self.handle)

    @property
    def pos(self) -> int:
        return _lib.lib().grx_whisper_pos(self.handle)

    def decode(self, tokens, want_logits: bool = True):
        """Model.decode of the tokens after the cached positions: (logits of
        the last, its argmax)."""
        t = np.ascontiguousarray(tokens, np.int32)
        lg = np.zeros(self.hp["n_vocab"], np.float32) if want_logits else None
        nxt = np.zeros(1, np.int32)
        _lib.call("grx_whisper_decode", self.handle, t.ctypes.data_as(C.c_void_p), t.size,
                  None if lg is None else lg.ctypes.data_as(C.c_void_p), nxt.ctypes.data_as(C.c_void_p))
        return lg, int(nxt[0])

    def greedy(self, prompt, n_steps: int) -> np.ndarray:
        p = np.ascontiguousarray(prompt, np.int32)
        out = np.zeros(n_steps + 1, np.int32)
        _lib.call("grx_whisper_greedy", self.handle, p.ctypes.data_as(C.c_void_p), p.size, n_steps,
                  out.ctypes.data_as(C.c_void_p))
        return out

    def close(self):
        if self.handle:
            _lib.call("grx_whisper_destroy", self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
