"""Host driver of the pocket-TTS flow-LM transformer on the GPU.

Mirrors flowLM.text/run/step of gorelaxor's pockettts package (github.com/
xattribution/gorelaxor, pockettts/lm.go:164-195): tensors bound by the names
pockettts/model.go reads, the text prefix run at once, then frames that stay
on the device (teacher-forced latents; the flow head is not part of this).
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from .kern import Context, default_context


class PocketState:
    """The flow LM's transformer state on the device (tstate, pockettts/
    nn.go:113-126): each layer's rotated keys and values for `positions`
    positions.  A Voice (pockettts/voice.go:13-24) is one; seeding an LM
    with it (PocketLM.set_state) leaves it unchanged."""

    def __init__(self, handle, n_layer: int, d: int):
        self.handle = handle
        self.n_layer, self.d = n_layer, d

    @property
    def positions(self) -> int:
        return _lib.lib().grx_pocket_state_positions(self.handle)

    def read(self):
        """(k, v): host copies, [n_layer][positions][d] each."""
        n = self.positions
        k = np.zeros((self.n_layer, n, self.d), np.float32)
        v = np.zeros((self.n_layer, n, self.d), np.float32)
        _lib.call("grx_pocket_state_read", self.handle, k.ctypes.data_as(C.c_void_p), v.ctypes.data_as(C.c_void_p))
        return k, v

    def close(self):
        if self.handle:
            _lib.call("grx_pocket_state_destroy", self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class PocketLM:
    def __init__(self, hp: dict, tensors: dict | None = None, ctx: Context | None = None):
        self.ctx = ctx or default_context()
        self.hp = dict(hp)
        h = _lib.PocketHParams(d=hp["d"], heads=hp["heads"], ff=hp["ff"], n_layer=hp["n_layer"],
                               max_pos=hp["max_pos"], ldim=hp["ldim"], period=float(hp.get("period", 1e4)))
        out = C.c_void_p()
        _lib.call("grx_pocket_create", self.ctx.handle, C.byref(h), C.byref(out))
        self.handle = out
        if tensors:
            for name, arr in tensors.items():
                self.set_tensor(name, arr)

    @classmethod
    def from_gguf(cls, path: str, max_pos: int, ctx: Context | None = None) -> "PocketLM":
        """The flow LM of a Pocket TTS GGUF file (pockettts.Load, pockettts/
        model.go:201-250): Q8_0 transformer matrices go to the device as
        stored."""
        self = cls.__new__(cls)
        self.handle = None
        self.ctx = ctx or default_context()
        h = _lib.PocketHParams()
        out = C.c_void_p()
        _lib.call("grx_pocket_load_gguf", self.ctx.handle, str(path).encode(), max_pos, C.byref(h), C.byref(out))
        self.handle = out
        self.hp = {k: getattr(h, k) for k in ("d", "heads", "ff", "n_layer", "max_pos", "ldim", "period")}
        return self

    def set_tensor(self, name: str, arr: np.ndarray) -> None:
        a = np.ascontiguousarray(arr)
        _lib.call("grx_pocket_set_tensor", self.handle, name.encode(), a.ctypes.data_as(C.c_void_p), a.nbytes)

    def flow_init(self, dim: int, depth: int, decode_steps: int) -> None:
        """Declare the flow head (pockettts.flow.dim, flow.depth,
        decode_steps); its flow.* tensors then bind by name."""
        _lib.call("grx_pocket_flow_init", self.handle, dim, depth, decode_steps)

    def speak(self, noise: np.ndarray, first_latent=None):
        """speakChunk's frame loop on the device: one frame per noise row
        (ldim values each), each fed the previous frame's sampled latent
        (the first: first_latent, or bos).  Returns (latents [n][ldim], eos [n])."""
        ld = self.hp["ldim"]
        noise = np.ascontiguousarray(noise, np.float32).reshape(-1, ld)
        n = noise.shape[0]
        lat = np.zeros((n, ld), np.float32)
        eos = np.zeros(n, np.float32)
        fl = None if first_latent is None else np.ascontiguousarray(first_latent, np.float32)
        _lib.call("grx_pocket_speak", self.handle, None if fl is None else fl.ctypes.data_as(C.c_void_p),
                  noise.ctypes.data_as(C.c_void_p), n, lat.ctypes.data_as(C.c_void_p),
                  eos.ctypes.data_as(C.c_void_p))
        return lat, eos

    def reset(self) -> None:
        _lib.call("grx_pocket_reset", self.handle)

    def make_state(self, k: np.ndarray, v: np.ndarray) -> PocketState:
        """A state from keys and values [n_layer][positions][d] (rotated keys,
        as the caches hold them)."""
        d, nl = self.hp["d"], self.hp["n_layer"]
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        if k.shape != v.shape or k.size % (d * nl) != 0:
            raise ValueError(f"keys {k.shape} and values {v.shape} are not [{nl}][positions][{d}]")
        out = C.c_void_p()
        _lib.call("grx_pocket_state_create", self.handle, k.ctypes.data_as(C.c_void_p), v.ctypes.data_as(C.c_void_p),
                  k.size // (d * nl), C.byref(out))
        return PocketState(out, nl, d)

    def load_voice(self, path: str) -> PocketState:
        """Model.LoadVoice (pockettts/voice.go:26-64): a voice file made for
        the model file this LM was loaded from."""
        out = C.c_void_p()
        _lib.call("grx_pocket_load_voice_gguf", self.handle, str(path).encode(), C.byref(out))
        return PocketState(out, self.hp["n_layer"], self.hp["d"])

    def state(self) -> PocketState:
        """The LM's positions so far, copied into a new state."""
        out = C.c_void_p()
        _lib.call("grx_pocket_state_save", self.handle, C.byref(out))
        return PocketState(out, self.hp["n_layer"], self.hp["d"])

    def set_state(self, st: PocketState) -> None:
        """tstate.clone into the LM (speakChunk, pockettts/speak.go:117): the
        caches take the state's positions, the next position its count."""
        _lib.call("grx_pocket_set_state", self.handle, st.handle)

    @property
    def pos(self) -> int:
        return _lib.lib().grx_pocket_pos(self.handle)

    def run(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        T = x.size // self.hp["d"]
        out = np.zeros(self.hp["d"], np.float32)
        _lib.call("grx_pocket_run", self.handle, x.ctypes.data_as(C.c_void_p), T, out.ctypes.data_as(C.c_void_p))
        return out

    def frames(self, latents: np.ndarray | None, n: int | None = None):
        """n steps fed latents[k] (None: bos every frame): (outputs [n][d], eos [n])."""
        if latents is not None:
            latents = np.ascontiguousarray(latents, np.float32)
            n = latents.size // self.hp["ldim"]
        outs = np.zeros((n, self.hp["d"]), np.float32)
        eos = np.zeros(n, np.float32)
        _lib.call("grx_pocket_frames", self.handle,
                  None if latents is None else latents.ctypes.data_as(C.c_void_p), n,
                  outs.ctypes.data_as(C.c_void_p), eos.ctypes.data_as(C.c_void_p))
        return outs, eos

    def close(self):
        if self.handle:
            _lib.call("grx_pocket_destroy", self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
