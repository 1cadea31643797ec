"""Seeded synthetic inputs and random-init Q8_0 models of the benchmark shapes.

Q8_0 weights follow the single-GEMV workload: every 32-value block holds
int8 values uniform in [-127, 127] and an f16 scale |N(0, 0.02)|/127 (about
30% of those scales are f16 subnormals, which the product must keep).
All generators are numpy PCG64 streams from an explicit seed.
"""
from __future__ import annotations

import numpy as np

QK = 32
Q8_BYTES = 34


def q8_weight(rng: np.random.Generator, rows: int, cols: int, sigma: float = 0.02) -> np.ndarray:
    """rows x cols random Q8_0 matrix as ggml bytes (rows*cols/32*34 uint8)."""
    assert cols % QK == 0
    nb = rows * cols // QK
    q = rng.integers(-127, 128, size=(nb, QK), dtype=np.int64).astype(np.int8)
    d = (np.abs(rng.standard_normal(nb)) * sigma / 127.0).astype(np.float32).astype(np.float16)
    out = np.empty((nb, Q8_BYTES), np.uint8)
    out[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    out[:, 2:] = q.view(np.uint8)
    return out.reshape(-1)


def q8_dequant(q8: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """Exact float32 values of a Q8_0 matrix (d * q)."""
    blk = q8.reshape(-1, Q8_BYTES)
    d = blk[:, 0:2].copy().view(np.float16).astype(np.float32)
    q = blk[:, 2:].copy().view(np.int8).astype(np.float32)
    return (q * d).reshape(rows, cols)


def gemv_inputs(seed: int = 1, n: int = 1024, k: int = 1024):
    """The single Q8_0 GEMV: weights n x k, activation 1 x k ~ N(0, 1)."""
    rng = np.random.default_rng(seed)
    w = q8_weight(rng, n, k)
    x = rng.standard_normal(k).astype(np.float32)
    return w, x


WHISPER_BASE_EN = dict(n_vocab=51864, n_text_ctx=448, n_state=512, n_head=8, n_layer=6, n_audio_ctx=1500)
WHISPER_TINY_TEST = dict(n_vocab=1000, n_text_ctx=64, n_state=128, n_head=2, n_layer=2, n_audio_ctx=96)


def whisper_model(hp: dict, seed: int = 7) -> dict:
    """Random-init whisper decoder tensors, named as whisper/model.go binds
    them; matrices Q8_0 bytes, vectors float32."""
    rng = np.random.default_rng(seed)
    st, nv, tctx = hp["n_state"], hp["n_vocab"], hp["n_text_ctx"]
    t = {}

    def vec(n, scale=0.02, base=0.0):
        return (base + scale * rng.standard_normal(n)).astype(np.float32)

    t["decoder.token_embedding.weight"] = q8_weight(rng, nv, st, sigma=0.5)
    t["decoder.positional_embedding"] = vec(tctx * st, 0.1)
    t["decoder.ln.weight"] = vec(st, 0.1, 1.0)
    t["decoder.ln.bias"] = vec(st, 0.1)
    for i in range(hp["n_layer"]):
        p = f"decoder.blocks.{i}."
        for ln in ("attn_ln", "cross_attn_ln", "mlp_ln"):
            t[p + ln + ".weight"] = vec(st, 0.1, 1.0)
            t[p + ln + ".bias"] = vec(st, 0.1)
        for a in ("attn", "cross_attn"):
            for w in ("query", "key", "value", "out"):
                t[p + f"{a}.{w}.weight"] = q8_weight(rng, st, st, sigma=0.15)
            for b in ("query", "value", "out"):
                t[p + f"{a}.{b}.bias"] = vec(st, 0.1)
        t[p + "mlp.0.weight"] = q8_weight(rng, 4 * st, st, sigma=0.1)
        t[p + "mlp.0.bias"] = vec(4 * st, 0.1)
        t[p + "mlp.2.weight"] = q8_weight(rng, st, 4 * st, sigma=0.05)
        t[p + "mlp.2.bias"] = vec(st, 0.1)
    return t


def encoder_output(hp: dict, seed: int = 11) -> np.ndarray:
    """Cross-attention input: n_audio_ctx x n_state float32 ~ N(0, 1)."""
    rng = np.random.default_rng(seed)
    return rng.standard_normal(hp["n_audio_ctx"] * hp["n_state"]).astype(np.float32)


POCKET_TTS_LM = dict(d=1024, heads=16, ff=4096, n_layer=6, ldim=32, max_pos=320, period=1e4)
POCKET_TTS_TINY = dict(d=128, heads=2, ff=512, n_layer=2, ldim=32, max_pos=96, period=1e4)


def pocket_model(hp: dict, seed: int = 5) -> dict:
    """Random-init flow-LM transformer tensors, named as pockettts/model.go
    reads them: transformer matrices Q8_0, the rest float32."""
    rng = np.random.default_rng(seed)
    d, ff, ld = hp["d"], hp["ff"], hp["ldim"]
    t = {}

    def vec(n, scale=0.02, base=0.0):
        return (base + scale * rng.standard_normal(n)).astype(np.float32)

    for i in range(hp["n_layer"]):
        p = f"lm.blk.{i}."
        for n in ("norm1", "norm2"):
            t[p + n + ".weight"] = vec(d, 0.1, 1.0)
            t[p + n + ".bias"] = vec(d, 0.1)
        t[p + "attn_qkv.weight"] = q8_weight(rng, 3 * d, d, sigma=0.1)
        t[p + "attn_out.weight"] = q8_weight(rng, d, d, sigma=0.1)
        t[p + "ff1.weight"] = q8_weight(rng, ff, d, sigma=0.1)
        t[p + "ff2.weight"] = q8_weight(rng, d, ff, sigma=0.05)
    t["lm.input.weight"] = vec(d * ld, 0.2)
    t["lm.bos"] = vec(ld, 1.0)
    t["lm.out_norm.weight"] = vec(d, 0.1, 1.0)
    t["lm.out_norm.bias"] = vec(d, 0.1)
    t["lm.eos.weight"] = vec(d, 0.05)
    t["lm.eos.bias"] = vec(1, 0.1)
    return t


def pocket_inputs(hp: dict, frames: int, prefix: int = 64, seed: int = 6):
    """The text prefix (prefix x d random embedding rows) and teacher-forced
    latents (frames x ldim, N(0,1)), seeded."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((prefix, hp["d"])).astype(np.float32)
    lat = rng.standard_normal((frames, hp["ldim"])).astype(np.float32)
    return x, lat
