"""Host mirror of gorelaxor's internal/kern Q8_0 API over libgrx.so.

Names, argument meaning and error behaviour follow the reference package
(github.com/xattribution/gorelaxor, internal/kern/kern.go):

    w = NewQ8(rows, cols, q8_bytes)      # kern.go:74-84, errors as there
    w.Pack(threads); w.DropRows()        # kern.go:86-103 (packing is done at NewQ8)
    w.Row(dst, j); w.Float32(); w.Bytes()
    MatMul(dst, ldc, x, lda, m, w, bias, threads)   # kern.go:183-196
    Linear(dst, x, m, w, bias, threads)             # kern.go:198-201
    w.ToQ8() on an F32 matrix -> Q8_0 bytes          # kern.go:136-170

Host arrays are numpy float32/uint8.  The reference panics on a buffer too
short for the shape (its bounds probes, kernels_amd64.go:45-49); this mirror
raises IndexError in the same cases, and GrxError for library errors.
The product always runs on the GPU: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import threading

import numpy as np

from . import _lib
from ._lib import GrxError

QK = 32
Q8Bytes = 34

F32, F16, Q8_0 = 0, 1, 2

_ctx_lock = threading.Lock()
_ctxs: dict[int, "Context"] = {}


class Context:
    """A device and its stream (grx_ctx)."""

    def __init__(self, device: int = 0):
        h = C.c_void_p()
        _lib.call("grx_ctx_create", device, C.byref(h))
        self.handle = h
        self.device = device

    def sync(self):
        _lib.call("grx_ctx_sync", self.handle)

    @property
    def stream(self) -> int:
        return _lib.lib().grx_ctx_stream(self.handle) or 0

    def close(self):
        if self.handle:
            _lib.call("grx_ctx_destroy", self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def default_context(device: int = 0) -> Context:
    with _ctx_lock:
        c = _ctxs.get(device)
        if c is None:
            c = _ctxs[device] = Context(device)
        return c


def device_count() -> int:
    return _lib.lib().grx_device_count()


def _ptr(a):
    if a is None:
        return None
    if isinstance(a, np.ndarray):
        return a.ctypes.data_as(C.c_void_p)
    return C.c_void_p(int(a.data_ptr()))  # a device tensor


class Weight:
    """A Q8_0 matrix of Rows x Cols in HBM (kern.Weight, kern.go:38-50)."""

    def __init__(self, handle, rows: int, cols: int, ctx: Context):
        self.handle = handle
        self.Rows, self.Cols, self.Type = rows, cols, Q8_0
        self.ctx = ctx

    def Pack(self, threads: int = 1) -> None:
        """Packing happens once at NewQ8 (grx_weight_q8_create)."""

    def DropRows(self) -> None:
        """The host rows are never kept; nothing to drop."""

    def Row(self, dst: np.ndarray, j: int) -> None:
        if dst.dtype != np.float32 or dst.size < self.Cols:
            raise IndexError("kern: Row destination shorter than Cols")
        _lib.call("grx_weight_row", self.ctx.handle, self.handle, j, _ptr(dst))

    def Float32(self) -> np.ndarray:
        out = np.zeros(self.Rows * self.Cols, np.float32)
        _lib.call("grx_weight_float32", self.ctx.handle, self.handle, _ptr(out))
        return out

    def Bytes(self) -> int:
        return int(_lib.lib().grx_weight_bytes(self.handle))

    def close(self):
        if self.handle:
            _lib.call("grx_weight_destroy", self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def NewQ8(rows: int, cols: int, b, ctx: Context | None = None) -> Weight:
    """kern.NewQ8 (kern.go:74-84): rows x cols values as Q8_0 blocks."""
    ctx = ctx or default_context()
    buf = np.ascontiguousarray(np.frombuffer(bytes(b), np.uint8) if not isinstance(b, np.ndarray) else b,
                               dtype=np.uint8)
    h = C.c_void_p()
    _lib.call("grx_weight_q8_create", ctx.handle, rows, cols, _ptr(buf), buf.size, C.byref(h))
    return Weight(h, rows, cols, ctx)


def LinearFloat(dst: np.ndarray, x: np.ndarray, w: Weight, bias=None) -> None:
    """kern.Linear of one row on a weight that keeps its rows (the float
    route, kern.go:185-196 -> gemvRows): dot4q8avx by groups of four rows,
    dotQ8Go for the last partial group, then the bias."""
    if x.dtype != np.float32 or x.size < w.Cols or dst.dtype != np.float32 or dst.size < w.Rows:
        raise IndexError("kern: Linear buffers shorter than the weight")
    if bias is not None and (bias.dtype != np.float32 or bias.size < w.Rows):
        raise IndexError("kern: bias shorter than Rows")
    _lib.call("grx_linear_q8_float", w.ctx.handle, _ptr(dst), _ptr(x), w.handle, _ptr(bias))


def LinearF32(dst: np.ndarray, x: np.ndarray, w: np.ndarray, rows: int, cols: int, bias=None,
              ctx: Context | None = None) -> None:
    """kern.Linear of one row on a float32 weight (gemvRows: dotF32x4 by
    groups of four rows, dotF32Go for the rest, then the bias)."""
    ctx = ctx or default_context()
    w = np.ascontiguousarray(w, np.float32)
    if w.size < rows * cols or x.size < cols or dst.size < rows:
        raise IndexError("kern: Linear buffers shorter than the weight")
    _lib.call("grx_linear_f32", ctx.handle, _ptr(dst), _ptr(np.ascontiguousarray(x, np.float32)), _ptr(w), rows,
              cols, _ptr(None if bias is None else np.ascontiguousarray(bias, np.float32)))


def ToQ8(v: np.ndarray, rows: int, cols: int, ctx: Context | None = None) -> np.ndarray:
    """Weight.ToQ8 of an F32 matrix (kern.go:136-170) on the GPU: the Q8_0 bytes."""
    ctx = ctx or default_context()
    v = np.ascontiguousarray(v, np.float32)
    if v.size < rows * cols:
        raise IndexError("kern: ToQ8 input shorter than rows*cols")
    out = np.zeros(rows * cols // QK * Q8Bytes, np.uint8)
    _lib.call("grx_to_q8", ctx.handle, rows, cols, _ptr(v), _ptr(out))
    return out


def MatMul(dst: np.ndarray, ldc: int, x: np.ndarray, lda: int, m: int, w: Weight, bias=None,
           threads: int = 1) -> None:
    """kern.MatMul (kern.go:183-196): dst[m][ldc] = x[m][lda] . W^T + bias."""
    if m == 0 or w.Rows == 0:
        return
    if x.dtype != np.float32 or dst.dtype != np.float32:
        raise TypeError("kern: MatMul takes float32 arrays")
    if x.size < (m - 1) * lda + w.Cols or dst.size < (m - 1) * ldc + w.Rows:
        raise IndexError("kern: MatMul buffer shorter than the shape")
    if bias is not None and (bias.dtype != np.float32 or bias.size < w.Rows):
        raise IndexError("kern: MatMul bias shorter than Rows")
    _lib.call("grx_matmul_q8", w.ctx.handle, _ptr(dst), ldc, _ptr(np.ascontiguousarray(x)), lda, m,
              w.handle, _ptr(bias))


def Linear(dst: np.ndarray, x: np.ndarray, m: int, w: Weight, bias=None, threads: int = 1) -> None:
    """kern.Linear (kern.go:198-201)."""
    MatMul(dst, w.Rows, x, w.Cols, m, w, bias, threads)


# ---- device-pointer forms (torch tensors on the GPU) ----

def matmul_dev(dst, x, m: int, w: Weight, bias=None, ldc: int | None = None, lda: int | None = None,
               ctx: Context | None = None) -> None:
    ctx = ctx or w.ctx
    _lib.call("grx_matmul_q8_dev", ctx.handle, _ptr(dst), ldc or w.Rows, _ptr(x), lda or w.Cols, m,
              w.handle, _ptr(bias))


def matmul_dev_noalloc(dst, x, m: int, w: Weight, bias=None, ldc: int | None = None, lda: int | None = None,
                       ctx: Context | None = None) -> None:
    """matmul_dev with no allocation (grx_matmul_q8_dev_noalloc): the
    library's fixed per-GPU scratch holds the rounded activations."""
    ctx = ctx or w.ctx
    _lib.call("grx_matmul_q8_dev_noalloc", ctx.handle, _ptr(dst), ldc or w.Rows, _ptr(x), lda or w.Cols, m,
              w.handle, _ptr(bias))


def quant_act_dev(q, sc, x, m: int, k: int, lda: int | None = None, ctx: Context | None = None) -> None:
    ctx = ctx or default_context()
    _lib.call("grx_quant_act_dev", ctx.handle, _ptr(q), _ptr(sc), _ptr(x), lda or k, m, k)


def matmul_prequant_dev(dst, q, sc, m: int, w: Weight, bias=None, ldc: int | None = None,
                        ctx: Context | None = None) -> None:
    ctx = ctx or w.ctx
    _lib.call("grx_matmul_q8_prequant_dev", ctx.handle, _ptr(dst), ldc or w.Rows, _ptr(q), _ptr(sc), m,
              w.handle, _ptr(bias))


def block_dots_dev(s, q, m: int, w: Weight, ctx: Context | None = None) -> None:
    ctx = ctx or w.ctx
    _lib.call("grx_block_dots_dev", ctx.handle, _ptr(s), _ptr(q), m, w.handle)


# the elementwise float kernels of grx_vec_dev
VEC_EXPF, VEC_EXP8, VEC_GELU = 0, 1, 2


def vec_dev(fn: int, y, x, n: int, ctx: Context | None = None) -> None:
    ctx = ctx or default_context()
    _lib.call("grx_vec_dev", ctx.handle, fn, _ptr(y), _ptr(x), n)


# grx_layernorm_dev: forms, kernel forms and flags
LN_KERN, LN_F64 = 0, 1
LN_BLOCK, LN_WAVE = 0, 1
LN_TREE_ONLY = 1


def layernorm_dev(form: int, impl: int, y, x, rows: int, n: int, w=None, b=None, eps: float = 1e-5,
                  flags: int = 0, ctx: Context | None = None) -> None:
    """The path's LayerNorms on device rows (kern's layerNorm, internal/
    kern/mathx.go:55-75, or pockettts', nn.go:27-49) through the kernels'
    own code, for parity checks."""
    ctx = ctx or default_context()
    _lib.call("grx_layernorm_dev", ctx.handle, form, impl, flags, _ptr(y), _ptr(x), rows, n,
              _ptr(w) if w is not None else None, _ptr(b) if b is not None else None, float(eps))


def set_tune(name: str, value: int) -> None:
    """Override one of the library's kernel choices (grx_debug_tune: GEMM_MIN_M,
    GEMM_KERNEL, GEMM_NS, GEMM_KB, GEMV_WAVES, GEMV1, CONF_ATTN_RQ, FUSE_LN,
    FUSE_XSCORES, WAVE_VALUES, ARGMAX_ATOMIC, NO_GRAPH, GEMM_STAGE_A, GEMV_MX, GEMV1_ROWS,
    FUSE_SELF_ATTN, CONF_DW, CONF_FUSE, CONF_ATTN_G8, CONF_ATTN_THREADS); -1 hands it back.
    The reference's tests switch kernels the same way (setInt, internal/kern/
    kernels_amd64.go:190-200)."""
    _lib.call("grx_debug_tune", name.encode(), int(value))


class tuned:
    """Context manager: the kernel choices given as keywords for the block,
    handed back to the library afterwards."""

    def __init__(self, **choices):
        self.choices = {k: int(v) for k, v in choices.items()}

    def __enter__(self):
        for k, v in self.choices.items():
            set_tune(k, v)
        return self

    def __exit__(self, *exc):
        for k in self.choices:
            set_tune(k, -1)
        return False


__all__ = ["QK", "Q8Bytes", "F32", "F16", "Q8_0", "Context", "default_context", "device_count", "Weight",
           "NewQ8", "ToQ8", "MatMul", "Linear", "LinearFloat", "LinearF32", "matmul_dev", "matmul_dev_noalloc",
           "quant_act_dev", "matmul_prequant_dev",
           "block_dots_dev", "vec_dev", "VEC_EXPF", "VEC_EXP8", "VEC_GELU", "layernorm_dev", "LN_KERN", "LN_F64",
           "LN_BLOCK", "LN_WAVE", "LN_TREE_ONLY", "GrxError", "set_tune", "tuned"]
