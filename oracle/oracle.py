"""numpy front end of the C oracle (oracle/grx_oracle.c).

TEST INFRASTRUCTURE ONLY: loaded by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg as the checker of the HIP product.

Each wrapper names the reference function (file:line in the Go module
github.com/xattribution/gorelaxor) the C restatement follows.
"""
from __future__ import annotations

import contextlib
import ctypes as C
import math
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "liboracle.so")
VNNI_PATH = os.path.join(HERE, "_build", "libgrx_vnni.so")

QK = 32
Q8_BYTES = 34


def build(force: bool = False) -> str:
    """Compile the oracle (and the VNNI baseline) with its Makefile (gcc,
    no GPU needed)."""
    if force or not os.path.exists(LIB_PATH) or not os.path.exists(VNNI_PATH):
        subprocess.run(["make", "-s", "-C", HERE, "-B" if force else "all"], check=True)
    return LIB_PATH


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")


def _declare(L):
    L.orc_set_q8_product.argtypes = [C.c_void_p]
    L.orc_set_q8_product.restype = None
    L.orc_f16_to_f32.argtypes = [C.c_uint16]
    L.orc_f16_to_f32.restype = C.c_float
    L.orc_f32_to_f16.argtypes = [C.c_float]
    L.orc_f32_to_f16.restype = C.c_uint16
    L.orc_quant_q8.argtypes = [_f32p, C.c_size_t, _u8p]
    L.orc_dequant_q8.argtypes = [_f32p, _u8p, C.c_int]
    L.orc_quant_u8.argtypes = [_u8p, _f32p, _f32p, C.c_int]
    L.orc_quant_act_i8.argtypes = [_i8p, _f32p, _f32p, C.c_int]
    L.orc_block_dots.argtypes = [_i32p, _i8p, C.c_int, _u8p, C.c_int, C.c_int]
    L.orc_matmul_q8_int.argtypes = [_f32p, C.c_int, _f32p, C.c_int, C.c_int, _u8p, C.c_int,
                                    C.c_int, C.c_void_p, C.c_int]
    L.orc_matmul_q8_int_prequant.argtypes = [_f32p, C.c_int, _i8p, _f32p, C.c_int, _u8p,
                                             C.c_int, C.c_int, C.c_void_p]
    L.orc_matmul_q8_float.argtypes = [_f32p, C.c_int, _f32p, C.c_int, C.c_int, _u8p, C.c_int,
                                      C.c_int, C.c_void_p]
    L.orc_expf.argtypes = [C.c_float]
    L.orc_expf.restype = C.c_float
    L.orc_exp8.argtypes = [C.c_float]
    L.orc_exp8.restype = C.c_float
    L.orc_expsub.argtypes = [_f32p, C.c_int, C.c_float]
    L.orc_expsub.restype = C.c_float
    L.orc_softmax.argtypes = [_f32p, C.c_int]
    L.orc_gelu_vec.argtypes = [_f32p, C.c_int]
    L.orc_silu_vec.argtypes = [_f32p, C.c_int]
    L.orc_axpy.argtypes = [_f32p, _f32p, C.c_int, C.c_float]
    L.orc_layernorm.argtypes = [_f32p, _f32p, C.c_int, C.c_int, _f32p, _f32p]
    L.orc_layernorm_f64.argtypes = [_f32p, _f32p, C.c_int, C.c_int, C.c_void_p, C.c_void_p,
                                    C.c_double]
    L.orc_dot_f32_go.argtypes = [_f32p, _f32p, C.c_int]
    L.orc_dot_f32_go.restype = C.c_float
    L.orc_dot_f32_x4.argtypes = [_f32p, _f32p, C.c_int, C.c_int, _f32p]
    L.orc_argmax.argtypes = [_f32p, C.c_int]
    L.orc_argmax.restype = C.c_int
    L.orc_whisper_cross_kv.argtypes = [C.c_void_p, _f32p]
    L.orc_whisper_decode.argtypes = [C.c_void_p, _i32p, C.c_int, C.c_void_p]
    L.orc_whisper_decode.restype = C.c_int
    L.orc_whisper_greedy.argtypes = [C.c_void_p, _i32p, C.c_int, C.c_int, _i32p]
    L.orc_matmul_f32.argtypes = [_f32p, C.c_int, _f32p, C.c_int, _f32p, C.c_int, C.c_int, C.c_int, C.c_int,
                                 C.c_void_p]
    L.orc_rope_freqs.argtypes = [_f32p, C.c_int, C.c_double]
    L.orc_apply_rope.argtypes = [_f32p, C.c_int, _f32p, C.c_int, C.c_int]
    L.orc_ptts_forward.argtypes = [C.c_void_p, _f32p, C.c_int]
    L.orc_ptts_forward.restype = C.c_int
    L.orc_ptts_run.argtypes = [C.c_void_p, _f32p, C.c_int, _f32p]
    L.orc_ptts_run.restype = C.c_int
    L.orc_ptts_step.argtypes = [C.c_void_p, C.c_void_p, _f32p, _f32p]
    L.orc_ptts_step.restype = C.c_int


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


# ---- half precision (internal/kern/f16.go:14-71) ----

def f16_to_f32(h: int) -> float:
    return lib().orc_f16_to_f32(h)


def f32_to_f16(f: float) -> int:
    return lib().orc_f32_to_f16(f)


# ---- Q8_0 weights (kern.go:139-170, kern_test.go:10-28) ----

def quant_q8(v: np.ndarray) -> np.ndarray:
    """Round float32 values (a multiple of 32) to ggml Q8_0 bytes."""
    v = _f32(v).ravel()
    assert v.size % QK == 0
    out = np.zeros(v.size // QK * Q8_BYTES, np.uint8)
    lib().orc_quant_q8(v, v.size, out)
    return out


def dequant_q8(q: np.ndarray, nvals: int) -> np.ndarray:
    q = np.ascontiguousarray(q, np.uint8)
    out = np.zeros(nvals, np.float32)
    lib().orc_dequant_q8(out, q, nvals // QK)
    return out


# ---- activations (q8int.go:88-105) ----

def quant_u8(x: np.ndarray):
    x = _f32(x).ravel()
    nb = x.size // QK
    q = np.zeros(nb * QK, np.uint8)
    sc = np.zeros(nb, np.float32)
    lib().orc_quant_u8(q, sc, x, nb)
    return q, sc


def quant_act_i8(x: np.ndarray):
    """Activation rounding with the signed value kept (u8 - 128), per row."""
    x = _f32(x)
    rows = x.reshape(-1, x.shape[-1]) if x.ndim > 1 else x.reshape(1, -1)
    k = rows.shape[1]
    nb = k // QK
    q = np.zeros((rows.shape[0], k), np.int8)
    sc = np.zeros((rows.shape[0], nb), np.float32)
    for i in range(rows.shape[0]):
        qi = np.zeros(k, np.int8)
        si = np.zeros(nb, np.float32)
        lib().orc_quant_act_i8(qi, si, np.ascontiguousarray(rows[i]), nb)
        q[i], sc[i] = qi, si
    return q, sc


# ---- int8 products (q8int.go:148-223, vnni_amd64.s:58-69) ----

def block_dots(qa: np.ndarray, wq: np.ndarray, n: int, k: int) -> np.ndarray:
    qa = np.ascontiguousarray(qa, np.int8).reshape(-1, k)
    m = qa.shape[0]
    s = np.zeros((m, n, k // QK), np.int32)
    lib().orc_block_dots(s, qa, m, np.ascontiguousarray(wq, np.uint8), n, k)
    return s


def matmul_q8_int(x: np.ndarray, wq: np.ndarray, n: int, k: int, bias=None,
                  evex: bool = True) -> np.ndarray:
    """kern.MatMul on the int8 route: x [m][k] float32, wq Q8_0 rows [n]."""
    x = _f32(x).reshape(-1, k)
    m = x.shape[0]
    c = np.zeros((m, n), np.float32)
    b = None if bias is None else _f32(bias)
    lib().orc_matmul_q8_int(c, n, x, k, m, np.ascontiguousarray(wq, np.uint8), n, k, _ptr(b),
                            1 if evex else 0)
    return c


def matmul_q8_int_prequant(qa, sa, wq, n: int, k: int, bias=None) -> np.ndarray:
    qa = np.ascontiguousarray(qa, np.int8).reshape(-1, k)
    sa = _f32(sa).reshape(qa.shape[0], k // QK)
    m = qa.shape[0]
    c = np.zeros((m, n), np.float32)
    b = None if bias is None else _f32(bias)
    lib().orc_matmul_q8_int_prequant(c, n, qa, sa, m, np.ascontiguousarray(wq, np.uint8), n, k,
                                     _ptr(b))
    return c


def matmul_q8_float(x: np.ndarray, wq: np.ndarray, n: int, k: int, bias=None) -> np.ndarray:
    """kern.MatMul on the float route (gemvRows, m <= 16)."""
    x = _f32(x).reshape(-1, k)
    m = x.shape[0]
    assert m <= 16
    c = np.zeros((m, n), np.float32)
    b = None if bias is None else _f32(bias)
    lib().orc_matmul_q8_float(c, n, x, k, m, np.ascontiguousarray(wq, np.uint8), n, k, _ptr(b))
    return c


# ---- float kernels (mathx.go, kernels_amd64.s) ----

def expf(x: float) -> float:
    return lib().orc_expf(x)


def exp8(x: float) -> float:
    return lib().orc_exp8(x)


def expsub(x: np.ndarray, mx: float):
    x = _f32(x).copy()
    s = lib().orc_expsub(x, x.size, mx)
    return x, s


def softmax(x: np.ndarray) -> np.ndarray:
    x = _f32(x).copy()
    lib().orc_softmax(x, x.size)
    return x


def gelu(x: np.ndarray) -> np.ndarray:
    x = _f32(x).copy()
    lib().orc_gelu_vec(x, x.size)
    return x


def silu(x: np.ndarray) -> np.ndarray:
    x = _f32(x).copy()
    lib().orc_silu_vec(x, x.size)
    return x


def axpy(dst: np.ndarray, src: np.ndarray, s: float) -> np.ndarray:
    dst = _f32(dst).copy()
    lib().orc_axpy(dst, _f32(src), dst.size, s)
    return dst


def layernorm(x: np.ndarray, w: np.ndarray, b: np.ndarray) -> np.ndarray:
    x = _f32(x)
    n = x.shape[-1]
    rows = x.size // n
    y = np.zeros_like(x)
    lib().orc_layernorm(y, x, rows, n, _f32(w), _f32(b))
    return y


def layernorm_f64(x: np.ndarray, w=None, b=None, eps: float = 1e-5) -> np.ndarray:
    x = _f32(x)
    n = x.shape[-1]
    rows = x.size // n
    y = np.zeros_like(x)
    wf = None if w is None else _f32(w)
    bf = None if b is None else _f32(b)
    lib().orc_layernorm_f64(y, x, rows, n, _ptr(wf), _ptr(bf), eps)
    return y


def dot_f32_go(x, y) -> float:
    x, y = _f32(x), _f32(y)
    return lib().orc_dot_f32_go(x, y, x.size)


def dot_f32_x4(x, w, ld: int, k: int) -> np.ndarray:
    out = np.zeros(4, np.float32)
    lib().orc_dot_f32_x4(_f32(x), _f32(w), ld, k, out)
    return out


def argmax(x) -> int:
    x = _f32(x)
    return lib().orc_argmax(x, x.size)


# ---- whisper-shaped decoder (whisper/decoder.go:33-140) ----

class _Layer(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in (
        "attn_ln_w", "attn_ln_b", "q", "k", "v", "o", "q_b", "v_b", "o_b",
        "x_ln_w", "x_ln_b", "xq", "xk", "xv", "xo", "xq_b", "xv_b", "xo_b",
        "mlp_ln_w", "mlp_ln_b", "fc1", "fc2", "fc1_b", "fc2_b",
        "cross_k", "cross_v", "self_k", "self_v")]


class _Model(C.Structure):
    _fields_ = [("n_vocab", C.c_int), ("n_text_ctx", C.c_int), ("n_state", C.c_int),
                ("n_head", C.c_int), ("n_layer", C.c_int), ("n_audio_ctx", C.c_int),
                ("tok_emb", C.c_void_p), ("dec_pos", C.c_void_p), ("dec_ln_w", C.c_void_p),
                ("dec_ln_b", C.c_void_p), ("layers", C.c_void_p), ("n", C.c_int)]


class WhisperOracle:
    """Oracle decoder over a tensor dict named as whisper/model.go:376-401 binds
    them ("decoder.blocks.{i}.attn.query.weight", ...); Q8_0 matrices as uint8
    rows, vectors as float32."""

    _LAYER_MAP = {
        "attn_ln_w": "attn_ln.weight", "attn_ln_b": "attn_ln.bias",
        "q": "attn.query.weight", "k": "attn.key.weight", "v": "attn.value.weight",
        "o": "attn.out.weight", "q_b": "attn.query.bias", "v_b": "attn.value.bias",
        "o_b": "attn.out.bias", "x_ln_w": "cross_attn_ln.weight", "x_ln_b": "cross_attn_ln.bias",
        "xq": "cross_attn.query.weight", "xk": "cross_attn.key.weight",
        "xv": "cross_attn.value.weight", "xo": "cross_attn.out.weight",
        "xq_b": "cross_attn.query.bias", "xv_b": "cross_attn.value.bias",
        "xo_b": "cross_attn.out.bias", "mlp_ln_w": "mlp_ln.weight", "mlp_ln_b": "mlp_ln.bias",
        "fc1": "mlp.0.weight", "fc2": "mlp.2.weight", "fc1_b": "mlp.0.bias", "fc2_b": "mlp.2.bias",
    }

    def __init__(self, hp: dict, tensors: dict):
        self.hp = hp
        st, nh, nl = hp["n_state"], hp["n_head"], hp["n_layer"]
        nctx, tctx = hp["n_audio_ctx"], hp["n_text_ctx"]
        self._keep = []

        def keep(a):
            a = np.ascontiguousarray(a)
            self._keep.append(a)
            return a.ctypes.data

        layers = (_Layer * nl)()
        self.cross_k, self.cross_v, self.self_k, self.self_v = [], [], [], []
        for i in range(nl):
            p = f"decoder.blocks.{i}."
            for field, name in self._LAYER_MAP.items():
                setattr(layers[i], field, keep(tensors[p + name]))
            ck = np.zeros(nctx * st, np.float32)
            cv = np.zeros(nctx * st, np.float32)
            sk = np.zeros(tctx * st, np.float32)
            sv = np.zeros(tctx * st, np.float32)
            self.cross_k.append(ck)
            self.cross_v.append(cv)
            self.self_k.append(sk)
            self.self_v.append(sv)
            layers[i].cross_k = keep(ck)
            layers[i].cross_v = keep(cv)
            layers[i].self_k = keep(sk)
            layers[i].self_v = keep(sv)
        self._layers = layers
        m = _Model()
        m.n_vocab, m.n_text_ctx, m.n_state = hp["n_vocab"], tctx, st
        m.n_head, m.n_layer, m.n_audio_ctx = nh, nl, nctx
        m.tok_emb = keep(tensors["decoder.token_embedding.weight"])
        m.dec_pos = keep(tensors["decoder.positional_embedding"])
        m.dec_ln_w = keep(tensors["decoder.ln.weight"])
        m.dec_ln_b = keep(tensors["decoder.ln.bias"])
        m.layers = C.cast(layers, C.c_void_p)
        m.n = 0
        self._m = m

    @property
    def n(self) -> int:
        return self._m.n

    def reset(self):
        self._m.n = 0

    def set_encoder_output(self, enc: np.ndarray):
        lib().orc_whisper_cross_kv(C.byref(self._m), _f32(enc))

    def decode(self, tokens) -> np.ndarray:
        toks = np.ascontiguousarray(tokens, np.int32)
        lg = np.zeros(self.hp["n_vocab"], np.float32)
        rc = lib().orc_whisper_decode(C.byref(self._m), toks, toks.size, _ptr(lg))
        if rc != 0:
            raise ValueError("tokens do not fit the text context")
        return lg

    def greedy(self, prompt, n_steps: int) -> np.ndarray:
        p = np.ascontiguousarray(prompt, np.int32)
        out = np.zeros(n_steps + 1, np.int32)
        lib().orc_whisper_greedy(C.byref(self._m), p, p.size, n_steps, out)
        return out


# ---- float route products (gemm.go:116-259) ----

def matmul_f32(a: np.ndarray, b: np.ndarray, bias=None) -> np.ndarray:
    """ws.matmul with float32 B: a [m][k] . b [n][k]^T (+ bias)."""
    a = _f32(a)
    b = _f32(b)
    m, k = a.shape
    n = b.shape[0]
    c = np.zeros((m, n), np.float32)
    bb = None if bias is None else _f32(bias)
    lib().orc_matmul_f32(c, n, a, k, b, k, m, n, k, _ptr(bb))
    return c


# ---- pocket-TTS flow-LM transformer (pockettts/nn.go, lm.go) ----

def rope_freqs(head_dim: int, period: float = 1e4) -> np.ndarray:
    f = np.zeros(head_dim // 2, np.float32)
    lib().orc_rope_freqs(f, head_dim, period)
    return f


def apply_rope(x: np.ndarray, heads: int, freqs: np.ndarray, pos: int) -> np.ndarray:
    x = _f32(x).copy()
    lib().orc_apply_rope(x, heads, _f32(freqs), freqs.size, pos)
    return x


class _PLayer(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("norm1_w", "norm1_b", "norm2_w", "norm2_b", "qkv", "out", "ff1", "ff2",
                                          "k", "v")]


class _PModel(C.Structure):
    _fields_ = [("d", C.c_int), ("heads", C.c_int), ("ff", C.c_int), ("n_layer", C.c_int), ("max_pos", C.c_int),
                ("ldim", C.c_int), ("freqs", C.c_void_p), ("layers", C.c_void_p), ("input", C.c_void_p),
                ("bos", C.c_void_p), ("out_w", C.c_void_p), ("out_b", C.c_void_p), ("eos_w", C.c_void_p),
                ("eos_b", C.c_float), ("pos", C.c_int)]


class PocketOracle:
    """Oracle flow-LM transformer over tensors named as pockettts/model.go
    reads them ("lm.blk.{i}.attn_qkv.weight", "lm.input.weight", ...)."""

    def __init__(self, hp: dict, tensors: dict):
        self.hp = hp
        d, nl, mp = hp["d"], hp["n_layer"], hp["max_pos"]
        self._keep = []

        def keep(a):
            a = np.ascontiguousarray(a)
            self._keep.append(a)
            return a.ctypes.data

        layers = (_PLayer * nl)()
        self.k, self.v = [], []
        for i in range(nl):
            p = f"lm.blk.{i}."
            for f, n in (("norm1_w", "norm1.weight"), ("norm1_b", "norm1.bias"), ("norm2_w", "norm2.weight"),
                         ("norm2_b", "norm2.bias"), ("qkv", "attn_qkv.weight"), ("out", "attn_out.weight"),
                         ("ff1", "ff1.weight"), ("ff2", "ff2.weight")):
                setattr(layers[i], f, keep(tensors[p + n]))
            kc = np.zeros(mp * d, np.float32)
            vc = np.zeros(mp * d, np.float32)
            self.k.append(kc)
            self.v.append(vc)
            layers[i].k = keep(kc)
            layers[i].v = keep(vc)
        self._layers = layers
        self.freqs = rope_freqs(d // hp["heads"], hp.get("period", 1e4))
        m = _PModel()
        m.d, m.heads, m.ff, m.n_layer, m.max_pos, m.ldim = d, hp["heads"], hp["ff"], nl, mp, hp["ldim"]
        m.freqs = keep(self.freqs)
        m.layers = C.cast(layers, C.c_void_p)
        m.input = keep(tensors["lm.input.weight"])
        m.bos = keep(tensors["lm.bos"])
        m.out_w = keep(tensors["lm.out_norm.weight"])
        m.out_b = keep(tensors["lm.out_norm.bias"])
        m.eos_w = keep(tensors["lm.eos.weight"])
        m.eos_b = float(tensors["lm.eos.bias"][0])
        m.pos = 0
        self._m = m

    @property
    def pos(self) -> int:
        return self._m.pos

    def reset(self):
        self._m.pos = 0

    def set_state(self, k: np.ndarray, v: np.ndarray) -> None:
        """Seed the caches with a state of n positions, k and v [n_layer][n][d]
        (a Voice, pockettts/voice.go:26-64, cloned as speakChunk clones it,
        speak.go:117): rows 0..n-1 of every layer, next position n."""
        d, nl = self.hp["d"], self.hp["n_layer"]
        k = _f32(k).reshape(nl, -1, d)
        v = _f32(v).reshape(nl, -1, d)
        n = k.shape[1]
        if n > self.hp["max_pos"]:
            raise ValueError("the state does not fit the context")
        for i in range(nl):
            self.k[i][: n * d] = k[i].ravel()
            self.v[i][: n * d] = v[i].ravel()
        self._m.pos = n

    def state(self):
        """(k, v) [n_layer][pos][d]: the caches' rows so far."""
        d, n = self.hp["d"], self.pos
        return (np.stack([c[: n * d].reshape(n, d) for c in self.k]),
                np.stack([c[: n * d].reshape(n, d) for c in self.v]))

    def run(self, x: np.ndarray) -> np.ndarray:
        """flowLM.run of T rows (the text prefix): out_norm of the last row."""
        x = _f32(x).copy()
        T = x.size // self.hp["d"]
        out = np.zeros(self.hp["d"], np.float32)
        if lib().orc_ptts_run(C.byref(self._m), x, T, out) != 0:
            raise ValueError("rows do not fit the context")
        return out

    def step(self, latent=None):
        """flowLM.step: (out_norm output, end-of-speech logit)."""
        out = np.zeros(self.hp["d"], np.float32)
        eos = np.zeros(1, np.float32)
        lat = None if latent is None else _f32(latent)
        if lib().orc_ptts_step(C.byref(self._m), _ptr(lat), out, eos) != 0:
            raise ValueError("the step does not fit the context")
        return out, float(eos[0])


# ---- FastConformer encoder (conformer/encoder.go) ----

class _CFF(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("norm_w", "norm_b", "w1", "w2", "b1", "b2")]


class _CBlock(C.Structure):
    _fields_ = ([("ff1", _CFF), ("ff2", _CFF)] +
                [(n, C.c_void_p) for n in ("norm_attn_w", "norm_attn_b", "q", "k", "v", "out", "pos", "q_b", "k_b",
                                           "v_b", "out_b", "pos_u", "pos_v", "norm_conv_w", "norm_conv_b", "pw1",
                                           "pw2", "pw1_b", "pw2_b", "dw", "dw_b", "cn_w", "cn_b", "norm_out_w",
                                           "norm_out_b")])


class _CModel(C.Structure):
    _fields_ = ([(n, C.c_int) for n in ("d", "heads", "layers", "dff", "conv_kernel", "sub_channels", "n_mels",
                                        "xscaling", "conv_ln")] +
                [(n, C.c_void_p) for n in ("w0", "b0", "w2", "b2", "w5", "b5", "w3", "w6", "out", "b3", "b6",
                                           "out_b", "blocks", "w3f", "w6f")] +
                [(n, C.c_int) for n in ("causal_sub", "att_style", "att_left", "att_right", "conv_left",
                                        "conv_right")])


class _CKeys(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("mode", "T", "L", "chunk", "left_chunks", "left", "right", "c", "slot0",
                                       "Tc")]


def _declare_conformer(L):
    L.orc_conf_rel_pos.argtypes = [_f32p, C.c_int, C.c_int]
    L.orc_conf_bn_fold.argtypes = [_f32p, _f32p, _f32p, _f32p, C.c_int, _f32p, _f32p]
    L.orc_conf_subsample.argtypes = [C.c_void_p, _f32p, C.c_int, C.c_int, _f32p, C.POINTER(C.c_int),
                                     C.POINTER(C.c_int)]
    L.orc_conf_block_run.argtypes = [C.c_void_p, C.c_int, _f32p, C.c_int, C.c_int, _f32p]
    L.orc_conformer_encode.argtypes = [C.c_void_p, _f32p, C.c_int, C.c_int, C.c_int, _f32p, C.POINTER(C.c_int),
                                       C.POINTER(C.c_int)]
    L.orc_conf_key_range.argtypes = [C.c_void_p, C.c_int, C.POINTER(C.c_int), C.POINTER(C.c_int)]
    L.orc_conf_key_range.restype = None
    L.orc_conf_offline_keys.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_void_p]
    L.orc_conf_stream_new.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int]
    L.orc_conf_stream_new.restype = C.c_void_p
    L.orc_conf_stream_free.argtypes = [C.c_void_p, C.c_void_p]
    L.orc_conf_stream_free.restype = None
    L.orc_conf_stream_step.argtypes = [C.c_void_p, C.c_void_p, _f32p, C.c_int, C.c_int, C.c_int, _f32p,
                                       C.POINTER(C.c_int)]


def conf_frames_out(frames: int) -> int:
    for _ in range(3):
        frames = (frames - 1) // 2 + 1
    return frames


def conf_rel_pos(n: int, d: int) -> np.ndarray:
    """relPosEmb (conformer/encoder.go:171-191): [2n-1][d]."""
    L = lib()
    _declare_conformer(L)
    out = np.zeros((2 * n - 1) * d, np.float32)
    L.orc_conf_rel_pos(out, n, d)
    return out.reshape(2 * n - 1, d)


def conf_bn_fold(gw, gb, mean, var):
    """conformer/model.go:408-418: batch norm folded to (scale, bias)."""
    L = lib()
    _declare_conformer(L)
    d = len(gw)
    s, b = np.zeros(d, np.float32), np.zeros(d, np.float32)
    L.orc_conf_bn_fold(_f32(gw), _f32(gb), _f32(mean), _f32(var), d, s, b)
    return s, b


def _transpose_taps(w, c, taps):
    """transposeTaps (conformer/model.go:147-159): [c][taps] to [taps][c]."""
    return np.ascontiguousarray(np.asarray(w, np.float32).reshape(c, taps).T)


class ConformerOracle:
    """Oracle encoder over tensors named as conformer/model.go reads them."""

    def __init__(self, hp: dict, tensors: dict):
        self.hp = hp
        L = lib()
        _declare_conformer(L)
        d, c, K, nl = hp["d"], hp["sub_channels"], hp["conv_kernel"], hp["layers"]
        conv_ln = hp.get("conv_norm", "batch_norm") == "layer_norm"
        self._keep = []

        def keep(a):
            if a is None:
                return None
            a = np.ascontiguousarray(a)
            self._keep.append(a)
            return a.ctypes.data

        def pointwise(name, rows, cols):
            w = tensors[name]
            if w.nbytes == rows * cols // QK * Q8_BYTES:
                return w
            # Weight.ToQ8 of a float16 weight (conformer/model.go:397-402)
            return quant_q8(np.frombuffer(np.ascontiguousarray(w).tobytes(), np.float16).astype(np.float32))

        m = _CModel()
        m.d, m.heads, m.layers, m.dff = d, hp["heads"], nl, hp["dff"]
        m.conv_kernel, m.sub_channels, m.n_mels = K, c, hp["n_mels"]
        m.xscaling, m.conv_ln = int(bool(hp.get("xscaling", True))), int(conv_ln)
        chunked = hp.get("att_style", "regular") == "chunked_limited"
        m.att_style = int(chunked)
        m.causal_sub = int(bool(hp.get("causal_sub", chunked)))
        m.att_left, m.att_right = hp.get("att_left", -1), hp.get("att_right", -1)
        m.conv_left, m.conv_right = hp.get("conv_left", -1), hp.get("conv_right", -1)
        pe = "enc.pre_encode."
        m.w0 = keep(_transpose_taps(tensors[pe + "conv.0.weight"], c, 9))
        m.w2 = keep(_transpose_taps(tensors[pe + "conv.2.weight"], c, 9))
        m.w5 = keep(_transpose_taps(tensors[pe + "conv.5.weight"], c, 9))
        for f, n in (("b0", "conv.0.bias"), ("b2", "conv.2.bias"), ("b5", "conv.5.bias"), ("b3", "conv.3.bias"),
                     ("b6", "conv.6.bias"), ("out", "out.weight"), ("out_b", "out.bias")):
            setattr(m, f, keep(tensors[pe + n]))
        # conv.3 / conv.6: Q8_0 bytes, or float32 values (the float route)
        for f, n in (("w3", "conv.3.weight"), ("w6", "conv.6.weight")):
            w = tensors[pe + n]
            setattr(m, f + "f" if w.dtype == np.float32 else f, keep(w))
        blocks = (_CBlock * nl)()
        for i in range(nl):
            p = f"enc.blocks.{i}."
            B = blocks[i]
            for ffn, F in (("ff1", B.ff1), ("ff2", B.ff2)):
                F.norm_w = keep(tensors[p + f"norm_{ffn}.weight"])
                F.norm_b = keep(tensors[p + f"norm_{ffn}.bias"])
                F.w1 = keep(tensors[p + f"{ffn}.linear1.weight"])
                F.w2 = keep(tensors[p + f"{ffn}.linear2.weight"])
                F.b1 = keep(tensors.get(p + f"{ffn}.linear1.bias"))
                F.b2 = keep(tensors.get(p + f"{ffn}.linear2.bias"))
            for f, n in (("norm_attn_w", "norm_attn.weight"), ("norm_attn_b", "norm_attn.bias"),
                         ("q", "attn.linear_q.weight"), ("k", "attn.linear_k.weight"),
                         ("v", "attn.linear_v.weight"), ("out", "attn.linear_out.weight"),
                         ("pos", "attn.linear_pos.weight"), ("pos_u", "attn.pos_bias_u"),
                         ("pos_v", "attn.pos_bias_v"), ("norm_conv_w", "norm_conv.weight"),
                         ("norm_conv_b", "norm_conv.bias"), ("norm_out_w", "norm_out.weight"),
                         ("norm_out_b", "norm_out.bias")):
                setattr(B, f, keep(tensors[p + n]))
            for f, n in (("q_b", "attn.linear_q.bias"), ("k_b", "attn.linear_k.bias"),
                         ("v_b", "attn.linear_v.bias"), ("out_b", "attn.linear_out.bias"),
                         ("pw1_b", "conv.pointwise1.bias"), ("pw2_b", "conv.pointwise2.bias"),
                         ("dw_b", "conv.depthwise.bias")):
                setattr(B, f, keep(tensors.get(p + n)))
            B.pw1 = keep(pointwise(p + "conv.pointwise1.weight", 2 * d, d))
            B.pw2 = keep(pointwise(p + "conv.pointwise2.weight", d, d))
            B.dw = keep(_transpose_taps(tensors[p + "conv.depthwise.weight"], d, K))
            if conv_ln:
                B.cn_w = keep(tensors[p + "conv.bn.weight"])
                B.cn_b = keep(tensors[p + "conv.bn.bias"])
            else:
                s, b = conf_bn_fold(tensors[p + "conv.bn.weight"], tensors[p + "conv.bn.bias"],
                                    tensors[p + "conv.bn.running_mean"], tensors[p + "conv.bn.running_var"])
                B.cn_w, B.cn_b = keep(s), keep(b)
        self._blocks = blocks
        m.blocks = C.cast(blocks, C.c_void_p)
        self._m = m

    def subsample(self, mel: np.ndarray, valid: int):
        """encoder.go:123-167: (pre-encoder output [T][d], T, L)."""
        mel = _f32(mel)
        frames = mel.size // self.hp["n_mels"]
        T = self.frames_out(frames)
        out = np.zeros(T * self.hp["d"], np.float32)
        t, l = C.c_int(), C.c_int()
        lib().orc_conf_subsample(C.byref(self._m), mel, frames, valid, out, C.byref(t), C.byref(l))
        return out.reshape(T, self.hp["d"]), t.value, l.value

    def block(self, i: int, x: np.ndarray, L: int) -> np.ndarray:
        """Block i (encoder.go:411-429, its position projection first) on x [T][d]."""
        x = _f32(x).copy()
        T = x.size // self.hp["d"]
        lib().orc_conf_block_run(C.byref(self._m), i, x, T, L, conf_rel_pos(T, self.hp["d"]).reshape(-1))
        return x.reshape(T, self.hp["d"])

    def encode(self, mel: np.ndarray, valid: int, layers: int | None = None):
        """Model.encode without the prompt: (out [T][d], L); the first L rows are the output."""
        mel = _f32(mel)
        frames = mel.size // self.hp["n_mels"]
        T = self.frames_out(frames)
        out = np.zeros(T * self.hp["d"], np.float32)
        t, l = C.c_int(), C.c_int()
        nl = self.hp["layers"] if layers is None else layers
        lib().orc_conformer_encode(C.byref(self._m), mel, frames, valid, nl, out, C.byref(t), C.byref(l))
        return out.reshape(T, self.hp["d"]), l.value

    def frames_out(self, frames: int) -> int:
        causal = bool(self._m.causal_sub)
        for _ in range(3):
            frames = frames // 2 + 1 if causal else (frames - 1) // 2 + 1
        return frames

    def offline_keys(self, T: int, L: int):
        """offlineKeys (encoder.go:196-212): (the key form, block length)."""
        k = _CKeys()
        bl = lib().orc_conf_offline_keys(C.byref(self._m), T, L, C.byref(k))
        return k, bl

    def stream(self, right: int, left: int, drop: int) -> "ConformerOracleStream":
        return ConformerOracleStream(self, right, left, drop)


def conf_key_range(k, q: int):
    """keyRange of query q under the key form k: (lo, hi)."""
    lo, hi = C.c_int(), C.c_int()
    lib().orc_conf_key_range(C.byref(k), q, C.byref(lo), C.byref(hi))
    return lo.value, hi.value


def conf_stream_keys(L: int, chunk: int, left_chunks: int, c: int, left: int, Tc: int):
    """A streaming chunk's key form (stream.go:273-287)."""
    return _CKeys(mode=3, L=L, chunk=chunk, left_chunks=left_chunks, c=c, slot0=left - c, Tc=Tc)


class ConformerOracleStream:
    """One stream's caches and its chunk steps (stream.go:72-88, 241-307)."""

    def __init__(self, enc: ConformerOracle, right: int, left: int, drop: int):
        self.enc = enc
        self._p = lib().orc_conf_stream_new(C.byref(enc._m), right, left, drop)
        self.first = True

    def step(self, mel: np.ndarray, length: int):
        """One chunk [n_mels][nf] (the cache frames first): its encoder rows [L][d]."""
        mel = _f32(mel)
        nf = mel.size // self.enc.hp["n_mels"]
        out = np.zeros(max(nf, 1) * self.enc.hp["d"], np.float32)
        n = C.c_int()
        r = lib().orc_conf_stream_step(C.byref(self.enc._m), self._p, mel, nf, length, int(self.first), out,
                                       C.byref(n))
        if r != 0:
            raise ValueError("the chunk has more encoder rows than the stream's geometry")
        self.first = False
        return out[:n.value * self.enc.hp["d"]].reshape(n.value, self.enc.hp["d"])

    @property
    def kv_len(self) -> int:
        return C.cast(self._p, C.POINTER(C.c_int * 6)).contents[5]

    def close(self):
        if self._p:
            lib().orc_conf_stream_free(C.byref(self.enc._m), self._p)
            self._p = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---- whisper's token rules and sampler (whisper/transcribe.go:370-536) ----

class _ORules(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("eot", "sot", "translate", "transcribe", "solm", "prev", "nosp",
                                       "no_timestamps", "beg", "n_lang", "space")] + [
        ("suppress", C.POINTER(C.c_int)), ("n_suppress", C.c_int), ("n_audio_ctx", C.c_int),
        ("max_initial_ts", C.c_double)]


class _OSeq(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("n_tokens", "last", "penult", "has_ts", "seek_delta")]


class _OTok(C.Structure):
    _fields_ = [("id", C.c_int), ("tid", C.c_int), ("p", C.c_float), ("plog", C.c_float), ("force_ts", C.c_int)]


def whisper_sample(logits, specials: dict, suppress=(), space: int = -1, tokens=(), has_ts: bool = False,
                   seek_delta: int = 0, temp: float = 0.0, r: float = 0.0, n_audio_ctx: int = 1500,
                   max_initial_ts: float = 1.0) -> dict:
    """session.process + session.sample over one row of logits:
    {id, tid, p, plog, force_ts}."""
    L = lib()
    if not hasattr(L.orc_whisper_sample, "_declared"):
        L.orc_whisper_sample.argtypes = [_f32p, C.c_int, C.c_void_p, C.c_void_p, C.c_float, C.c_float, C.c_void_p]
        L.orc_whisper_sample.restype = None
        L.orc_whisper_sample._declared = True
    lg = _f32(logits).ravel()
    sup = np.ascontiguousarray(suppress, np.int32)
    rules = _ORules(**{k: int(specials[k]) for k in ("eot", "sot", "translate", "transcribe", "solm", "prev",
                                                      "nosp", "no_timestamps", "beg", "n_lang")},
                    space=space, n_suppress=sup.size, n_audio_ctx=n_audio_ctx, max_initial_ts=max_initial_ts)
    rules.suppress = sup.ctypes.data_as(C.POINTER(C.c_int))
    t = list(tokens)
    seq = _OSeq(n_tokens=len(t), last=t[-1] if t else 0, penult=t[-2] if len(t) > 1 else 0, has_ts=int(has_ts),
                seek_delta=seek_delta)
    out = _OTok()
    L.orc_whisper_sample(lg, lg.size, C.byref(rules), C.byref(seq), temp, r, C.byref(out))
    return dict(id=out.id, tid=out.tid, p=out.p, plog=out.plog, force_ts=bool(out.force_ts))



def whisper_window_loop(ref, logits, specials: dict, suppress=(), space: int = -1, n_audio_ctx: int = 1500,
                        seek: int = 0, seek_end: int = 3000, n_max: int = 220, temp: float = 0.0, r=None,
                        delta_min: int = 10, win_frames: int = 3000):
    """The loop of whisper/transcribe.go:207-260 for one seq after its prompt:
    `ref` (a WhisperOracle) has decoded the prompt and `logits` are its last.
    Each iteration samples with the rules (whisper_sample: process + sample,
    transcribe.go:370-494), then applies transcribe.go:211-237 - a timestamp
    above beg sets seekDelta = 2 (id - beg) and the result length, or fails
    the seq when it goes back; eot, or a timestamp reaching the audio's end,
    finishes it (failing it when no result was kept); the last iteration
    fails a seq stuck repeating itself - and decodes the token while the seq
    is active.  Returns (tokens, state)."""
    beg, eot = specials["beg"], specials["eot"]
    toks, ids = [], []
    st = dict(done=0, failed=0, result_len=0, seek_delta=win_frames, has_ts=0)
    lg = logits
    for i in range(n_max):
        t = whisper_sample(lg, specials, suppress=suppress, space=space, tokens=ids, has_ts=bool(st["has_ts"]),
                           seek_delta=st["seek_delta"], temp=temp, r=float(r[i]) if temp > 0 else 0.0,
                           n_audio_ctx=n_audio_ctx)
        toks.append(t)
        ids.append(t["id"])
        if t["id"] > beg:
            nd = 2 * (t["id"] - beg)
            if st["has_ts"] and st["seek_delta"] > nd and st["result_len"] < i:
                st["failed"] = 1
                break
            st["seek_delta"], st["result_len"], st["has_ts"] = nd, i + 1, 1
        at_end = seek + st["seek_delta"] + delta_min >= seek_end
        if t["id"] == eot or (st["has_ts"] and at_end):
            if st["result_len"] == 0:
                if at_end:
                    st["result_len"] = i + 1
                else:
                    st["failed"] = 1
                    break
            st["done"] = 1
            break
        if i == n_max - 1 and (st["result_len"] == 0 or st["seek_delta"] < win_frames // 2):
            st["failed"] = 1
            break
        lg = ref.decode([t["id"]])
    st["n_tokens"] = len(toks)
    return toks, st


# ---- pocket-TTS flow head (pockettts/lm.go:27-160) ----

class PocketFlowOracle:
    """flowHead (SimpleMLPAdaLN) over tensors named as pockettts/model.go:
    230-247 reads them; a matrix is Q8_0 bytes (the float route of a weight
    that keeps its rows) or float32 [rows][cols]."""

    def __init__(self, hp: dict, dim: int, depth: int, steps: int, tensors: dict):
        self.hp, self.dim, self.depth, self.steps, self.t = hp, dim, depth, steps, tensors
        self.tc = self.time_conds(steps)

    def linear(self, name: str, x: np.ndarray, rows: int, cols: int) -> np.ndarray:
        """linear1 (lm.go:55-57): kern.Linear of one row, float route."""
        w = self.t[name + ".weight"]
        bias = self.t.get(name + ".bias")
        x = _f32(x)
        if w.dtype == np.uint8:
            return matmul_q8_float(x, w, rows, cols, bias)[0]
        return matmul_f32(x[None], _f32(w).reshape(rows, cols), bias)[0]

    def embed(self, e: int, t: float) -> np.ndarray:
        """timeEmbed.embed (lm.go:59-87)."""
        p = f"flow.time.{e}."
        f = self.t[p + "freqs"]
        half = f.size
        x = np.zeros(2 * half, np.float32)
        t32 = np.float32(t)
        for i in range(half):
            a = float(np.float32(t32 * f[i]))
            x[i] = np.float32(math.cos(a))
            x[half + i] = np.float32(math.sin(a))
        h = silu(self.linear(p + "fc1", x, self.dim, 2 * half))
        y = self.linear(p + "fc2", h, self.dim, self.dim)
        s = 0.0
        for v in y:
            s += float(v)
        mean = s / len(y)
        q = 0.0
        for v in y:
            q += (float(v) - mean) * (float(v) - mean)
        inv = np.float32(1 / math.sqrt(q / (len(y) - 1) + 1e-5))
        alpha = self.t[p + "norm.alpha"]
        return (y * (alpha * inv).astype(np.float32)).astype(np.float32)

    def time_conds(self, steps: int):
        """flowHead.timeConds (lm.go:89-104)."""
        out = []
        for i in range(steps):
            s = self.embed(0, float(np.float32(i / steps)))
            t = self.embed(1, float(np.float32((i + 1) / steps)))
            out.append(((s + t) / np.float32(2)).astype(np.float32))
        return out

    def net(self, y: np.ndarray, x: np.ndarray) -> np.ndarray:
        """flowHead.net (lm.go:124-160)."""
        D = self.dim
        h = self.linear("flow.input", x, D, self.hp["ldim"])
        sy = silu(y)
        for i in range(self.depth):
            p = f"flow.res.{i}."
            mod = self.linear(p + "ada", sy, 3 * D, D)
            shift, scale, gate = mod[:D], mod[D:2 * D], mod[2 * D:]
            n = layernorm_f64(h, self.t[p + "norm.weight"], self.t[p + "norm.bias"], 1e-6)
            n = (n * (np.float32(1) + scale) + shift).astype(np.float32)
            m = silu(self.linear(p + "fc1", n, D, D))
            n = self.linear(p + "fc2", m, D, D)
            h = (h + gate * n).astype(np.float32)
        mod = self.linear("flow.final.ada", sy, 2 * D, D)
        shift, scale = mod[:D], mod[D:2 * D]
        n = layernorm_f64(h, None, None, 1e-6)
        n = (n * (np.float32(1) + scale) + shift).astype(np.float32)
        return self.linear("flow.final.out", n, self.hp["ldim"], D)

    def sample(self, c: np.ndarray, x0: np.ndarray) -> np.ndarray:
        """flowHead.sample (lm.go:107-122)."""
        y = self.linear("flow.cond", c, self.dim, self.hp["d"])
        cur = _f32(x0).copy()
        n = np.float32(len(self.tc))
        for t in self.tc:
            yi = (y + t).astype(np.float32)
            v = self.net(yi, cur)
            cur = (cur + v / n).astype(np.float32)
        return cur


# ---------------------------------------------------------------- RNN-T / TDT

class _RModel(C.Structure):
    _fields_ = [("d", C.c_int), ("H", C.c_int), ("L", C.c_int), ("V", C.c_int), ("J", C.c_int), ("act", C.c_int),
                ("tdt", C.c_int), ("nd", C.c_int), ("dur", C.c_int * 16), ("max_symbols", C.c_int),
                ("blank", C.c_int), ("embed", C.c_void_p), ("wx", C.c_void_p), ("wh", C.c_void_p),
                ("b", C.c_void_p), ("jenc", C.c_void_p), ("jpred", C.c_void_p), ("jout", C.c_void_p),
                ("jencb", C.c_void_p), ("jpredb", C.c_void_p), ("joutb", C.c_void_p)]


class _RToken(C.Structure):
    _fields_ = [("id", C.c_int), ("frame", C.c_int), ("duration", C.c_int), ("p", C.c_float)]


JOINT_ACTS = {"relu": 0, "sigmoid": 1, "tanh": 2}


def fd_exp(x: float) -> float:
    L = lib()
    L.orc_fd_exp.argtypes = [C.c_double]
    L.orc_fd_exp.restype = C.c_double
    return L.orc_fd_exp(x)


def tanh32(x: float) -> float:
    L = lib()
    L.orc_tanh32.argtypes = [C.c_float]
    L.orc_tanh32.restype = C.c_float
    return L.orc_tanh32(x)


class RnntOracle:
    """Oracle of Model.Decode (conformer/rnnt.go:111-173) over the decoder
    tensors named as conformer/model.go:306-315 reads them.  hp: d,
    pred_hidden, pred_layers, pred_vocab, joint_hidden, joint_act ("relu",
    "sigmoid", "tanh"), head_kind ("rnnt" / "tdt"), durations, max_symbols,
    blank (-1: pred_vocab - 1)."""

    def __init__(self, hp: dict, tensors: dict):
        self.hp = hp
        tdt = hp.get("head_kind", "rnnt") == "tdt"
        m = _RModel()
        m.d, m.H, m.L = hp["d"], hp["pred_hidden"], hp["pred_layers"]
        m.V, m.J = hp["pred_vocab"], hp["joint_hidden"]
        m.act = JOINT_ACTS[hp.get("joint_act", "relu")]
        m.tdt = int(tdt)
        durs = list(hp.get("durations", [])) if tdt else []
        m.nd = len(durs)
        for i, v in enumerate(durs):
            m.dur[i] = v
        m.max_symbols = hp.get("max_symbols", 10) if tdt else 10
        b = hp.get("blank", -1)
        m.blank = b if b >= 0 else hp["pred_vocab"] - 1
        self._keep = []

        def keep(a):
            a = np.ascontiguousarray(a)
            self._keep.append(a)
            return a.ctypes.data

        Ln = m.L
        self._wx = (C.c_void_p * Ln)(*[keep(tensors[f"pred.lstm.{i}.Wx"]) for i in range(Ln)])
        self._wh = (C.c_void_p * Ln)(*[keep(tensors[f"pred.lstm.{i}.Wh"]) for i in range(Ln)])
        self._b = (C.c_void_p * Ln)(*[keep(tensors[f"pred.lstm.{i}.bias"]) for i in range(Ln)])
        m.wx, m.wh, m.b = C.cast(self._wx, C.c_void_p), C.cast(self._wh, C.c_void_p), C.cast(self._b, C.c_void_p)
        m.embed = keep(tensors["pred.embed.weight"])
        for f, n in (("jenc", "joint.enc.weight"), ("jpred", "joint.pred.weight"), ("jout", "joint.out.weight"),
                     ("jencb", "joint.enc.bias"), ("jpredb", "joint.pred.bias"), ("joutb", "joint.out.bias")):
            setattr(m, f, keep(tensors[n]))
        self._m = m
        L = lib()
        L.orc_rnnt_decode.argtypes = [C.c_void_p, _f32p, C.c_int, _f32p, _f32p, C.POINTER(C.c_int), C.c_int,
                                      C.c_void_p, C.c_int]
        L.orc_rnnt_decode.restype = C.c_int

    def new_state(self):
        """NewDecoderState (rnnt.go:26-33): (h, c, last)."""
        H, Ln = self.hp["pred_hidden"], self.hp["pred_layers"]
        return np.zeros((Ln, H), np.float32), np.zeros((Ln, H), np.float32), -1

    def decode(self, enc: np.ndarray, state=None, frame_offset: int = 0):
        """(tokens as (id, frame, duration, p) tuples, final state)."""
        enc = _f32(enc)
        T = enc.size // self.hp["d"]
        h, c, last = self.new_state() if state is None else (state[0].copy(), state[1].copy(), state[2])
        h, c = np.ascontiguousarray(h, np.float32), np.ascontiguousarray(c, np.float32)
        cap = 16 * T + 1024
        out = (_RToken * cap)()
        lv = C.c_int(last)
        n = lib().orc_rnnt_decode(C.byref(self._m), enc, T, h.reshape(-1), c.reshape(-1), C.byref(lv),
                                  frame_offset, C.cast(out, C.c_void_p), cap)
        toks = [(out[i].id, out[i].frame, out[i].duration, float(np.float32(out[i].p))) for i in range(n)]
        return toks, (h, c, lv.value)


# ---- the reference's int8 CPU path with VNNI (grx_vnni.cc): the
# benchmark's CPU baseline, and its parity with orc_matmul_q8_int

_vnni = None


def vnni_lib() -> C.CDLL:
    global _vnni
    if _vnni is None:
        if not os.path.exists(VNNI_PATH):
            build()
        L = C.CDLL(VNNI_PATH)
        L.vnni_kind.restype = C.c_int
        L.vnni_panel_bytes.argtypes = [C.c_int, C.c_int]
        L.vnni_panel_bytes.restype = C.c_size_t
        L.vnni_pack.argtypes = [_u8p, C.c_int, C.c_int, C.c_void_p]
        L.vnni_matmul.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_int, C.c_int,
                                  C.c_void_p, C.c_int, C.c_void_p, C.c_void_p]
        L.vnni_matmul.restype = C.c_int
        L.vnni_ring.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.c_int, C.c_int, C.c_int,
                                C.c_int, C.c_void_p, C.c_void_p]
        L.vnni_ring.restype = C.c_int
        L.vnni_set_threads.argtypes = [C.c_int]
        L.vnni_set_threads.restype = None
        L.vnni_forget.argtypes = []
        L.vnni_forget.restype = None
        _vnni = L
    return _vnni


@contextlib.contextmanager
def vnni_products(threads: int):
    """Within the block, every int8 product of the oracle's graphs (whisper,
    pocket, conformer, Mimi, RNN-T: orc_matmul_q8_int, EVEX order) runs on
    the VNNI restatement of the reference's matmulQ8Int (grx_vnni.cc,
    vnni_q8_product: panels packed once per weight, the reference's task
    split over `threads` threads) - the same bits, the reference's CPU
    speed for the products.  The rest of each graph stays scalar C on one
    thread.  Timing only (the benchmark's CPU baselines)."""
    V, L = vnni_lib(), lib()
    if V.vnni_kind() == 0:
        raise RuntimeError("this processor has neither AVX512-VNNI nor AVX-VNNI")
    V.vnni_set_threads(int(threads))
    V.vnni_forget()
    L.orc_set_q8_product(C.cast(V.vnni_q8_product, C.c_void_p))
    try:
        yield
    finally:
        L.orc_set_q8_product(None)
        V.vnni_forget()


def vnni_kind() -> int:
    """2: AVX512-VNNI (the EVEX kernel), 1: AVX-VNNI (VEX), 0: neither."""
    return vnni_lib().vnni_kind()


class VnniWeight:
    """A Q8_0 matrix packed as the reference's panels (packQ8Panels,
    internal/kern/q8int.go:35-64), for vnni_matmul."""

    def __init__(self, q8: np.ndarray, n: int, k: int):
        self.n, self.k = n, k
        self.panels = np.zeros(vnni_lib().vnni_panel_bytes(n, k), np.uint8)
        vnni_lib().vnni_pack(np.ascontiguousarray(q8, np.uint8), n, k, self.panels.ctypes.data)


class VnniScratch:
    """matmulQ8Int's rounded activations for up to m rows of k values."""

    def __init__(self, m: int, k: int):
        mp = (m + 5) // 6 * 6
        self.q = np.zeros(mp * k, np.uint8)
        self.sc = np.zeros(mp * (k // 32), np.float32)


def vnni_matmul(x: np.ndarray, w: VnniWeight, bias=None, threads: int = 1, out=None, scratch=None) -> np.ndarray:
    """matmulQ8Int (internal/kern/q8int.go:148-223) with the VNNI tile
    kernel: x [m][k] float32 -> [m][n]."""
    x = np.ascontiguousarray(x, np.float32)
    m = x.shape[0]
    y = out if out is not None else np.zeros((m, w.n), np.float32)
    s = scratch if scratch is not None else VnniScratch(m, w.k)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    rc = vnni_lib().vnni_matmul(y.ctypes.data, w.n, x.ctypes.data, w.k, m, w.panels.ctypes.data, w.n, w.k,
                                None if b is None else b.ctypes.data, threads, s.q.ctypes.data, s.sc.ctypes.data)
    if rc != 0:
        raise RuntimeError("vnni_matmul: this processor has neither AVX512-VNNI nor AVX-VNNI")
    return y


def vnni_pack_many(q8: np.ndarray, count: int, n: int, k: int) -> tuple[np.ndarray, int]:
    """count Q8_0 matrices of n x k, back to back in q8, packed as panels:
    (the panels, bytes per matrix)."""
    per = vnni_lib().vnni_panel_bytes(n, k)
    q8 = np.ascontiguousarray(q8, np.uint8)
    src = n * (k // 32) * 34
    out = np.empty(per * count, np.uint8)
    for i in range(count):
        vnni_lib().vnni_pack(q8[i * src:(i + 1) * src], n, k, out[i * per:(i + 1) * per].ctypes.data)
    return out, per


def vnni_ring(y: np.ndarray, x: np.ndarray, panels: np.ndarray, per: int, count: int, n: int, k: int, threads: int,
              reps: int) -> None:
    """reps passes of one-row products over count packed matrices (C loop)."""
    s = VnniScratch(1, k)
    x = np.ascontiguousarray(x, np.float32)
    rc = vnni_lib().vnni_ring(y.ctypes.data, x.ctypes.data, panels.ctypes.data, per, count, n, k, threads, reps,
                              s.q.ctypes.data, s.sc.ctypes.data)
    if rc != 0:
        raise RuntimeError("vnni_ring: this processor has neither AVX512-VNNI nor AVX-VNNI")


# ---- the reference's whisper decode with float16 matrices (grx_vnni.cc
# f16w_decode, whisper/decoder.go:33-140): timing context only

class _F16Layer(C.Structure):
    _fields_ = [(f, C.c_void_p) for f in (
        "attn_ln_w", "attn_ln_b", "q", "k", "v", "o", "q_b", "v_b", "o_b", "x_ln_w", "x_ln_b", "xq", "xo",
        "xq_b", "xo_b", "mlp_ln_w", "mlp_ln_b", "fc1", "fc2", "fc1_b", "fc2_b", "cross_k", "cross_v",
        "self_k", "self_v")]


class _F16Model(C.Structure):
    _fields_ = [("n_vocab", C.c_int), ("n_text_ctx", C.c_int), ("n_state", C.c_int), ("n_head", C.c_int),
                ("n_layer", C.c_int), ("n_audio_ctx", C.c_int), ("tok_emb", C.c_void_p), ("dec_pos", C.c_void_p),
                ("dec_ln_w", C.c_void_p), ("dec_ln_b", C.c_void_p), ("layers", C.c_void_p), ("n", C.c_int)]


def q8_to_f16(q8: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """A Q8_0 matrix widened to float32 (scale times value) and rounded to
    float16, as a float16 model file would hold it."""
    b = np.ascontiguousarray(q8, np.uint8).reshape(rows, cols // 32, 34)
    sc = b[:, :, :2].copy().view(np.float16).astype(np.float32)
    v = b[:, :, 2:].view(np.int8).astype(np.float32)
    return (v * sc).reshape(rows, cols).astype(np.float16)


class WhisperF16:
    """The reference's own CPU decoder (float16 matrices, AVX2/F16C kernels,
    its thread fan-out) over a WhisperOracle's model: its matrices widened
    from Q8_0 to float16, its vectors, positional rows and cross keys and
    values (set the encoder output on the oracle first)."""

    def __init__(self, orc: "WhisperOracle", tensors: dict):
        hp = orc.hp
        st, nl = hp["n_state"], hp["n_layer"]
        self.hp = hp
        self._keep = []

        def keep(a):
            a = np.ascontiguousarray(a)
            self._keep.append(a)
            return a.ctypes.data

        def mat(name, rows, cols):
            return keep(q8_to_f16(tensors[name], rows, cols))

        L = vnni_lib()
        L.f16w_decode.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_int]
        L.f16w_decode.restype = C.c_int
        layers = (_F16Layer * nl)()
        for i in range(nl):
            p = f"decoder.blocks.{i}."
            ly = layers[i]
            for f in ("attn_ln_w", "attn_ln_b", "q_b", "v_b", "o_b", "x_ln_w", "x_ln_b", "xq_b", "xo_b",
                      "mlp_ln_w", "mlp_ln_b", "fc1_b", "fc2_b"):
                setattr(ly, f, keep(np.asarray(tensors[p + WhisperOracle._LAYER_MAP[f]], np.float32)))
            for f in ("q", "k", "v", "o", "xq", "xo"):
                setattr(ly, f, mat(p + WhisperOracle._LAYER_MAP[f], st, st))
            ly.fc1 = mat(p + WhisperOracle._LAYER_MAP["fc1"], 4 * st, st)
            ly.fc2 = mat(p + WhisperOracle._LAYER_MAP["fc2"], st, 4 * st)
            ly.cross_k = keep(orc.cross_k[i])
            ly.cross_v = keep(orc.cross_v[i])
            ly.self_k = keep(np.zeros(hp["n_text_ctx"] * st, np.float32))
            ly.self_v = keep(np.zeros(hp["n_text_ctx"] * st, np.float32))
        self._layers = layers
        m = _F16Model()
        m.n_vocab, m.n_text_ctx, m.n_state = hp["n_vocab"], hp["n_text_ctx"], st
        m.n_head, m.n_layer, m.n_audio_ctx = hp["n_head"], nl, hp["n_audio_ctx"]
        m.tok_emb = mat("decoder.token_embedding.weight", hp["n_vocab"], st)
        m.dec_pos = keep(np.asarray(tensors["decoder.positional_embedding"], np.float32))
        m.dec_ln_w = keep(np.asarray(tensors["decoder.ln.weight"], np.float32))
        m.dec_ln_b = keep(np.asarray(tensors["decoder.ln.bias"], np.float32))
        m.layers = C.cast(layers, C.c_void_p)
        m.n = 0
        self._m = m
        self.logits = np.zeros(hp["n_vocab"], np.float32)

    def reset(self):
        self._m.n = 0

    def decode(self, tokens, threads: int = 1) -> np.ndarray:
        t = np.ascontiguousarray(tokens, np.int32)
        if vnni_lib().f16w_decode(C.byref(self._m), t.ctypes.data, t.size, self.logits.ctypes.data, threads) != 0:
            raise ValueError("tokens do not fit the text context (or 6 or more at once)")
        return self.logits

    def greedy(self, prompt, n_steps: int, threads: int = 1) -> list:
        """The prompt in one call, then n_steps argmax tokens one at a time
        (transcribe.go's greedy loop without its rules)."""
        out = [int(np.argmax(self.decode(prompt, threads)))]
        for _ in range(n_steps):
            out.append(int(np.argmax(self.decode([out[-1]], threads))))
        return out


# ---- pocket-TTS's Mimi decoder (grx_oracle_mimi.c, pockettts/mimi.go) ----

class _MLin(C.Structure):
    _fields_ = [("n", C.c_int), ("k", C.c_int), ("wq", C.c_void_p), ("wf", C.c_void_p), ("b", C.c_void_p)]


class _MConv(C.Structure):
    _fields_ = [("cin", C.c_int), ("cout", C.c_int), ("k", C.c_int), ("stride", C.c_int), ("dil", C.c_int),
                ("w", _MLin)]


class _MConvTr(C.Structure):
    _fields_ = [("cin", C.c_int), ("cout", C.c_int), ("k", C.c_int), ("stride", C.c_int), ("w", _MLin)]


class _SeaStep(C.Structure):
    _fields_ = [("kind", C.c_int), ("elu", C.c_int), ("c", _MConv), ("t", _MConvTr), ("a", _MConv), ("b", _MConv)]


class _MimiLayer(C.Structure):
    _fields_ = [("norm1_w", C.c_void_p), ("norm1_b", C.c_void_p), ("norm2_w", C.c_void_p), ("norm2_b", C.c_void_p),
                ("qkv", _MLin), ("out", _MLin), ("ff1", _MLin), ("ff2", _MLin), ("ls1", C.c_void_p),
                ("ls2", C.c_void_p)]


class _Mimi(C.Structure):
    _fields_ = [("d", C.c_int), ("heads", C.c_int), ("ff", C.c_int), ("n_layer", C.c_int), ("context", C.c_int),
                ("ldim", C.c_int), ("up_s", C.c_int), ("freqs", C.c_void_p), ("layers", C.c_void_p),
                ("quant", _MLin), ("up", C.c_void_p), ("n_steps", C.c_int), ("steps", C.c_void_p)]


def _mimi_lib() -> C.CDLL:
    L = lib()
    if not getattr(L, "_mimi_ready", False):
        L.orc_elu.argtypes = [_f32p, C.c_size_t]
        L.orc_mimi_state_new.argtypes = [C.c_void_p, C.c_int]
        L.orc_mimi_state_new.restype = C.c_void_p
        L.orc_mimi_state_free.argtypes = [C.c_void_p, C.c_void_p]
        L.orc_mimi_decode.argtypes = [C.c_void_p, C.c_void_p, _f32p, C.c_int, _f32p, C.POINTER(C.c_int)]
        L.orc_mimi_decode.restype = C.c_int
        L._mimi_ready = True
    return L


def elu(x: np.ndarray) -> np.ndarray:
    """pockettts/nn.go:51-64 on a copy of x."""
    y = np.array(x, np.float32).ravel()
    _mimi_lib().orc_elu(y, y.size)
    return y.reshape(np.shape(x))


class MimiOracle:
    """The Mimi decoder of pockettts/mimi.go over a tensor dict named as
    pockettts/model.go reads them (Q8_0 matrices as uint8 rows, the rest
    float32), with one streaming state (decState) of max_pos transformer
    positions."""

    def __init__(self, hp: dict, tensors: dict, max_pos: int = 4096):
        from gorelaxor_amd.synth import mimi_steps

        L = _mimi_lib()
        self.hp = hp
        d = hp["d"]
        self._keep = []

        def keep(a):
            a = np.ascontiguousarray(a)
            self._keep.append(a)
            return a.ctypes.data

        def lin(name, n, k, bias=None):
            w = tensors[name]
            ml = _MLin(n, k, None, None, keep(np.asarray(bias, np.float32)) if bias is not None else None)
            if w.dtype == np.uint8:
                ml.wq = keep(w)
            else:
                ml.wf = keep(np.asarray(w, np.float32))
            return ml

        self.hd = d // hp["heads"]
        freqs = np.zeros(self.hd // 2, np.float32)
        L.orc_rope_freqs(freqs, self.hd, float(hp["period"]))
        layers = (_MimiLayer * hp["n_layer"])()
        for i in range(hp["n_layer"]):
            p = f"mimi.dec_tf.{i}."
            ly = layers[i]
            ly.norm1_w, ly.norm1_b = keep(tensors[p + "norm1.weight"]), keep(tensors[p + "norm1.bias"])
            ly.norm2_w, ly.norm2_b = keep(tensors[p + "norm2.weight"]), keep(tensors[p + "norm2.bias"])
            ly.qkv = lin(p + "attn_qkv.weight", 3 * d, d)
            ly.out = lin(p + "attn_out.weight", d, d)
            ly.ff1 = lin(p + "ff1.weight", hp["ff"], d)
            ly.ff2 = lin(p + "ff2.weight", d, hp["ff"])
            ly.ls1 = keep(tensors[p + "ls1"]) if p + "ls1" in tensors else None
            ly.ls2 = keep(tensors[p + "ls2"]) if p + "ls2" in tensors else None
        steps_desc = mimi_steps(hp)
        steps = (_SeaStep * len(steps_desc))()
        for s, (kind, name, el, cin, cout, k, stride, dil) in zip(steps, steps_desc):
            s.elu = int(el)
            if kind == "conv":
                s.kind = 0
                s.c = _MConv(cin, cout, k, stride, dil, lin(name + ".weight", cout, k * cin, tensors[name + ".bias"]))
            elif kind == "convtr":
                s.kind = 1
                s.t = _MConvTr(cin, cout, k, stride, lin(name + ".weight", k * cout, cin, tensors[name + ".bias"]))
            else:
                s.kind = 2
                s.a = _MConv(cin, cout, k, 1, dil, lin(name + ".1.weight", cout, k * cin, tensors[name + ".1.bias"]))
                s.b = _MConv(cout, cin, 1, 1, 1, lin(name + ".3.weight", cin, cout, tensors[name + ".3.bias"]))
        m = _Mimi()
        m.d, m.heads, m.ff, m.n_layer = d, hp["heads"], hp["ff"], hp["n_layer"]
        m.context, m.ldim, m.up_s = hp["context"], hp["ldim"], hp["up_s"]
        m.freqs = keep(freqs)
        m.layers = C.cast(layers, C.c_void_p)
        m.quant = lin("mimi.quant", d, hp["ldim"])
        m.up = keep(tensors["mimi.up"])
        m.n_steps = len(steps_desc)
        m.steps = C.cast(steps, C.c_void_p)
        self._layers, self._steps, self._m = layers, steps, m
        self.samples_per_latent = hp["up_s"] * int(np.prod(hp["ratios"]))
        self.max_pos = max_pos
        self._st = L.orc_mimi_state_new(C.byref(m), max_pos)

    def reset(self):
        lib().orc_mimi_state_free(C.byref(self._m), self._st)
        self._st = lib().orc_mimi_state_new(C.byref(self._m), self.max_pos)

    def decode(self, lat: np.ndarray) -> np.ndarray:
        """n latents [n][ldim] -> n * samples_per_latent samples, continuing
        the stream."""
        lat = _f32(np.atleast_2d(lat))
        n = lat.shape[0]
        out = np.zeros(n * self.samples_per_latent, np.float32)
        no = C.c_int(0)
        if lib().orc_mimi_decode(C.byref(self._m), self._st, lat, n, out, C.byref(no)) != 0:
            raise ValueError("past the transformer's positions")
        assert no.value == out.size
        return out

    def __del__(self):
        try:
            lib().orc_mimi_state_free(C.byref(self._m), self._st)
        except Exception:
            pass
