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


def special_tokens(n_vocab: int) -> dict:
    """The special token ids of a vocabulary of n_vocab (newVocab, whisper/
    vocab.go:20-45): English models from eot 50256; multilingual ones
    (n_vocab >= 51865) one later, with n_vocab - 51766 languages after sot and
    the task and timestamp tokens moved by the language count past 98."""
    v = dict(eot=50256, sot=50257, translate=50357, transcribe=50358, solm=50359, prev=50360, nosp=50361,
             no_timestamps=50362, beg=50363, n_lang=0)
    if n_vocab >= 51865:
        n_lang = n_vocab - 51765 - 1
        dt = n_lang - 98
        v["eot"] += 1
        v["sot"] += 1
        for k in ("translate", "transcribe", "solm", "prev", "nosp", "no_timestamps", "beg"):
            v[k] += dt
        v["n_lang"] = n_lang
    return v


class Rules:
    """grx_whisper_rules from a dict of special tokens plus the suppress
    list (vocab.suppressed()), the " " token (-1 if none) and the model's
    audio context."""

    def __init__(self, specials: dict, suppress=(), space: int = -1, n_audio_ctx: int = 1500,
                 max_initial_ts: float = 1.0):
        self.suppress = np.ascontiguousarray(suppress, np.int32)
        self.c = _lib.WhisperRules(**{k: int(specials[k]) for k in (
            "eot", "sot", "translate", "transcribe", "solm", "prev", "nosp", "no_timestamps", "beg", "n_lang")},
            space=space, n_suppress=self.suppress.size, n_audio_ctx=n_audio_ctx, max_initial_ts=max_initial_ts)
        self.c.suppress = self.suppress.ctypes.data_as(C.POINTER(C.c_int32))


def _seq(tokens=(), has_ts: bool = False, seek_delta: int = 0):
    t = list(tokens)
    return _lib.WhisperSeq(n_tokens=len(t), last=t[-1] if t else 0, penult=t[-2] if len(t) > 1 else 0,
                           has_ts=int(has_ts), seek_delta=seek_delta)


def _tok(t) -> dict:
    return dict(id=t.id, tid=t.tid, p=t.p, plog=t.plog, force_ts=bool(t.force_ts))


def sample_logits(logits: np.ndarray, rules: Rules, tokens=(), has_ts: bool = False, seek_delta: int = 0,
                  temp: float = 0.0, r: float = 0.0, ctx: Context | None = None) -> dict:
    """session.process + session.sample (whisper/transcribe.go:370-494) on
    the GPU over one row of logits: {id, tid, p, plog, force_ts}."""
    ctx = ctx or default_context()
    lg = np.ascontiguousarray(logits, np.float32)
    out = _lib.WhisperToken()
    seq = _seq(tokens, has_ts, seek_delta)
    _lib.call("grx_whisper_sample_logits", ctx.handle, lg.ctypes.data_as(C.c_void_p), lg.size, C.byref(rules.c),
              C.byref(seq), temp, r, C.byref(out))
    return _tok(out)


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

    def rules_loop(self, rules: "Rules", seek: int, seek_end: int, n_max: int, temp: float = 0.0, r=None,
                   delta_min: int = 10, win_frames: int = 3000):
        """One window's decode loop on the device after a decoded prompt
        (whisper/transcribe.go:207-260): tokens (dicts of id, tid, p, plog,
        force_ts) and the sequence's state (n_tokens, done, failed,
        result_len, seek_delta, has_ts)."""
        draws = None
        if temp > 0:
            draws = np.ascontiguousarray(r, np.float32)
            if draws.size < n_max:
                raise ValueError(f"{n_max} draws needed, {draws.size} given")
        lp = _lib.WhisperLoop(seek=seek, seek_end=seek_end, delta_min=delta_min, win_frames=win_frames, n_max=n_max,
                              temp=temp, r=None if draws is None else draws.ctypes.data_as(C.POINTER(C.c_float)))
        out = (_lib.WhisperToken * max(n_max, 1))()
        res = _lib.WhisperLoopResult()
        _lib.call("grx_whisper_rules_loop", self.handle, C.byref(rules.c), C.byref(lp), out, C.byref(res))
        toks = [_tok(out[k]) for k in range(res.n_tokens)]
        return toks, {k: getattr(res, k) for k in ("n_tokens", "done", "failed", "result_len", "seek_delta", "has_ts")}

    def copy_stream(self, dst: int, src: int) -> None:
        """kvCache.copyFrom (whisper/decoder.go:22-28): stream dst's cache,
        next token and token record become stream src's."""
        _lib.call("grx_whisper_stream_copy", self.handle, dst, src)

    def share_encoder_output(self, dst: int, src: int) -> None:
        """Stream dst takes stream src's cross keys and values."""
        _lib.call("grx_whisper_share_encoder_output", self.handle, dst, src)

    def steps(self, n_steps: int) -> np.ndarray:
        """n_steps greedy steps of every stream from the current position,
        each fed its last choice: tokens [streams][n_steps]."""
        out = np.zeros((self.streams, n_steps), np.int32)
        _lib.call("grx_whisper_steps", self.handle, n_steps, out.ctypes.data_as(C.c_void_p))
        return out

    def logits(self, stream: int = 0) -> np.ndarray:
        """Stream `stream`'s logits of the last step."""
        out = np.zeros(self.hp["n_vocab"], np.float32)
        _lib.call("grx_whisper_logits", self.handle, stream, out.ctypes.data_as(C.c_void_p))
        return out

    def sample(self, rules: Rules, tokens=(), has_ts: bool = False, seek_delta: int = 0, temp: float = 0.0,
               r: float = 0.0, stream: int = 0) -> dict:
        """The token rules and sampler over stream `stream`'s last logits,
        which stay on the device."""
        out = _lib.WhisperToken()
        seq = _seq(tokens, has_ts, seek_delta)
        _lib.call("grx_whisper_sample", self.handle, stream, C.byref(rules.c), C.byref(seq), temp, r, C.byref(out))
        return _tok(out)

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
