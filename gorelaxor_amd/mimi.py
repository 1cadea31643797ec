"""Host driver of pocket-TTS's Mimi decoder on the GPU (latents to audio).

Mirrors mimiDecoder of pockettts/mimi.go (github.com/xattribution/gorelaxor):
decState / newState (mimi.go:110-119) and decode (mimi.go:122-152), over the
tensors named as pockettts/model.go reads them.  Each decoder holds one
stream's state (caches, carried rows, position) in device memory.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from .kern import Context, default_context


class MimiDecoder:
    """hp: d, heads, ff, n_layer, context, ldim, up_s, period, ratios,
    nf, k, res_k, last_k, dil_base, compress, n_res (the settings of
    pockettts.Load, pockettts/model.go:280-308); max_latents bounds the
    latents one decode call takes."""

    def __init__(self, hp: dict, tensors: dict | None = None, max_latents: int = 4, ctx: Context | None = None):
        self.ctx = ctx or default_context()
        self.hp = dict(hp)
        r = list(hp["ratios"])
        h = _lib.MimiHParams(d=hp["d"], heads=hp["heads"], ff=hp["ff"], layers=hp["n_layer"], context=hp["context"],
                             ldim=hp["ldim"], upsample=hp["up_s"], period=float(hp["period"]), n_ratios=len(r),
                             n_filters=hp["nf"], kernel_size=hp["k"], residual_kernel_size=hp["res_k"],
                             last_kernel_size=hp["last_k"], dilation_base=hp["dil_base"], compress=hp["compress"],
                             n_residual=hp["n_res"], max_latents=max_latents)
        for i, v in enumerate(r[:8]):
            h.ratios[i] = v
        out = C.c_void_p()
        self.handle = None
        _lib.call("grx_mimi_create", self.ctx.handle, C.byref(h), C.byref(out))
        self.handle = out
        self.max_latents = max_latents
        self.samples_per_latent = _lib.lib().grx_mimi_samples_per_latent(self.handle)
        if tensors:
            for name, arr in tensors.items():
                self.set_tensor(name, arr)

    @classmethod
    def from_gguf(cls, path, max_latents: int = 4, ctx: Context | None = None) -> "MimiDecoder":
        """The Mimi decoder of a Pocket TTS GGUF file (grx_mimi_load_gguf:
        the Mimi part of pockettts.Load, pockettts/model.go:201-213,
        280-308), its settings in .hp."""
        self = cls.__new__(cls)
        self.ctx = ctx or default_context()
        self.handle = None
        h = _lib.MimiHParams()
        out = C.c_void_p()
        _lib.call("grx_mimi_load_gguf", self.ctx.handle, str(path).encode(), max_latents, C.byref(h), C.byref(out))
        self.handle = out
        self.hp = dict(d=h.d, heads=h.heads, ff=h.ff, n_layer=h.layers, context=h.context, ldim=h.ldim,
                       up_s=h.upsample, period=h.period, ratios=tuple(h.ratios[i] for i in range(h.n_ratios)),
                       nf=h.n_filters, k=h.kernel_size, res_k=h.residual_kernel_size, last_k=h.last_kernel_size,
                       dil_base=h.dilation_base, compress=h.compress, n_res=h.n_residual)
        self.max_latents = max_latents
        self.samples_per_latent = _lib.lib().grx_mimi_samples_per_latent(self.handle)
        return self

    def set_tensor(self, name: str, arr: np.ndarray) -> None:
        """A matrix as ggml Q8_0 rows (uint8) or float32, a vector float32."""
        a = np.ascontiguousarray(arr)
        _lib.call("grx_mimi_set_tensor", self.handle, name.encode(), a.ctypes.data_as(C.c_void_p), a.nbytes)

    def reset(self) -> None:
        """A fresh decState (mimi.go:112-119)."""
        _lib.call("grx_mimi_reset", self.handle)

    def decode(self, lat: np.ndarray) -> np.ndarray:
        """decode (mimi.go:122-152): latents [n][ldim] (scaled back by the
        flow LM's mean and std) -> n * samples_per_latent samples."""
        lat = np.ascontiguousarray(np.atleast_2d(lat), np.float32)
        n = lat.shape[0]
        out = np.zeros(n * self.samples_per_latent, np.float32)
        _lib.call("grx_mimi_decode", self.handle, lat.ctypes.data_as(C.c_void_p), n, out.ctypes.data_as(C.c_void_p))
        return out

    def decode_dev(self, lat_ptr: int, n: int, out_ptr: int) -> None:
        """decode on device buffers, enqueued on the context's stream."""
        _lib.call("grx_mimi_decode_dev", self.handle, C.c_void_p(lat_ptr), n, C.c_void_p(out_ptr))

    def close(self):
        if self.handle:
            _lib.call("grx_mimi_destroy", self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
