"""Host driver of the RNN-T / TDT greedy decoder on the GPU.

Mirrors conformer/rnnt.go of gorelaxor (github.com/xattribution/gorelaxor):
Token (rnnt.go:10-15), DecoderState / NewDecoderState (rnnt.go:19-33) and
Model.Decode (rnnt.go:111-173), over the decoder tensors named as
conformer/model.go:306-315 reads them.  The whole greedy loop runs on the
device; the host sees the tokens when Decode returns.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import _lib
from .kern import Context, default_context

JOINT_ACTS = {"relu": 0, "sigmoid": 1, "tanh": 2}


@dataclass
class Token:
    """One emitted subword (rnnt.go:10-15)."""
    ID: int
    Frame: int
    Duration: int
    P: float


class DecoderState:
    """The prediction network's memory between Decode calls (h and c per
    layer in device memory, and the last emitted token)."""

    def __init__(self, dec: "TransducerDecoder"):
        self._dec = dec
        out = C.c_void_p()
        _lib.call("grx_rnnt_state_create", dec.handle, C.byref(out))
        self.handle = out

    def read(self):
        """(h [layers][H], c [layers][H], last)."""
        L, H = self._dec.hp["pred_layers"], self._dec.hp["pred_hidden"]
        h, c = np.zeros((L, H), np.float32), np.zeros((L, H), np.float32)
        last = C.c_int()
        _lib.call("grx_rnnt_state_read", self.handle, h.ctypes.data_as(C.c_void_p), c.ctypes.data_as(C.c_void_p),
                  C.byref(last))
        return h, c, last.value

    def write(self, h: np.ndarray, c: np.ndarray, last: int) -> None:
        h, c = np.ascontiguousarray(h, np.float32), np.ascontiguousarray(c, np.float32)
        _lib.call("grx_rnnt_state_write", self.handle, h.ctypes.data_as(C.c_void_p), c.ctypes.data_as(C.c_void_p),
                  int(last))

    def close(self):
        if self.handle:
            _lib.call("grx_rnnt_state_destroy", self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class TransducerDecoder:
    """hp: d (encoder width), pred_hidden, pred_layers, pred_vocab (tokens
    plus blank), joint_hidden, joint_act ("relu" / "sigmoid" / "tanh"),
    head_kind ("rnnt" / "tdt"), durations and max_symbols (TDT), blank (-1:
    pred_vocab - 1)."""

    def __init__(self, hp: dict, tensors: dict | None = None, ctx: Context | None = None):
        self.ctx = ctx or default_context()
        self.hp = dict(hp)
        tdt = hp.get("head_kind", "rnnt") == "tdt"
        if hp.get("head_kind", "rnnt") not in ("rnnt", "tdt"):
            raise ValueError(f"conformer: {hp['head_kind']!r} models are not supported (only RNN-T and TDT)")
        durs = list(hp.get("durations", [])) if tdt else []
        h = _lib.RnntHParams(d=hp["d"], pred_hidden=hp["pred_hidden"], pred_layers=hp["pred_layers"],
                             pred_vocab=hp["pred_vocab"], joint_hidden=hp["joint_hidden"],
                             joint_act=JOINT_ACTS[hp.get("joint_act", "relu")], tdt=int(tdt), n_durations=len(durs),
                             max_symbols=hp.get("max_symbols", 10), blank=hp.get("blank", -1))
        for i, v in enumerate(durs[:16]):
            h.durations[i] = v
        if len(durs) > 16:
            h.n_durations = len(durs)
        out = C.c_void_p()
        self.handle = None
        _lib.call("grx_rnnt_create", self.ctx.handle, C.byref(h), C.byref(out))
        self.handle = out
        if tensors:
            for name, arr in tensors.items():
                self.set_tensor(name, arr)

    @classmethod
    def from_gguf(cls, path: str, ctx: Context | None = None) -> "TransducerDecoder":
        """The transducer head of a FastConformer GGUF file (conformer/
        model.go:191-235, 306-315): Q8_0 matrices go to the device as
        stored."""
        self = cls.__new__(cls)
        self.handle = None
        self.ctx = ctx or default_context()
        h = _lib.RnntHParams()
        out = C.c_void_p()
        _lib.call("grx_rnnt_load_gguf", self.ctx.handle, str(path).encode(), C.byref(h), C.byref(out))
        self.handle = out
        acts = {v: k for k, v in JOINT_ACTS.items()}
        self.hp = dict(d=h.d, pred_hidden=h.pred_hidden, pred_layers=h.pred_layers, pred_vocab=h.pred_vocab,
                       joint_hidden=h.joint_hidden, joint_act=acts[h.joint_act],
                       head_kind="tdt" if h.tdt else "rnnt", blank=h.blank, max_symbols=h.max_symbols,
                       durations=[h.durations[i] for i in range(h.n_durations)])
        return self

    def set_tensor(self, name: str, arr: np.ndarray) -> None:
        a = np.ascontiguousarray(arr)
        _lib.call("grx_rnnt_set_tensor", self.handle, name.encode(), a.ctypes.data_as(C.c_void_p), a.nbytes)

    def new_state(self) -> DecoderState:
        """NewDecoderState (rnnt.go:26-33)."""
        return DecoderState(self)

    def _run(self, ptr, T: int, on_dev: bool, st: DecoderState | None, frame_offset: int) -> list[Token]:
        cap = 16 * T + 1024
        out = (_lib.RnntToken * cap)()
        n = C.c_int()
        _lib.call("grx_rnnt_decode", self.handle, ptr, T, int(on_dev), st.handle if st else None, frame_offset,
                  C.cast(out, C.c_void_p), cap, C.byref(n))
        return [Token(out[i].id, out[i].frame, out[i].duration, float(np.float32(out[i].p))) for i in range(n.value)]

    def decode(self, enc: np.ndarray, st: DecoderState | None = None, frame_offset: int = 0) -> list[Token]:
        """Model.Decode of encoder output enc [T][d], continuing from st (None
        starts fresh)."""
        enc = np.ascontiguousarray(enc, np.float32)
        T = enc.size // self.hp["d"]
        return self._run(enc.ctypes.data_as(C.c_void_p), T, False, st, frame_offset)

    def decode_dev(self, enc_ptr: int, T: int, st: DecoderState | None = None, frame_offset: int = 0) -> list[Token]:
        """The same with the encoder output in device memory (a pointer)."""
        return self._run(C.c_void_p(enc_ptr), T, True, st, frame_offset)

    def close(self):
        if self.handle:
            _lib.call("grx_rnnt_destroy", self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
