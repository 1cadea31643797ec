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
WHISPER_LARGE_V3_TURBO = dict(n_vocab=51866, n_text_ctx=448, n_state=1280, n_head=20, n_layer=4, n_audio_ctx=1500)
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


POCKET_FLOW = dict(dim=512, depth=6, steps=1)
POCKET_FLOW_TINY = dict(dim=64, depth=2, steps=2)


def pocket_flow_model(hp: dict, fhp: dict, seed: int = 12, q8: bool = True) -> dict:
    """Random-init flow head (pockettts/model.go:230-247 names), typed as the
    reference's converter types them: matrices of at least 64 x 64 whose rows
    are whole Q8_0 blocks Q8_0 (when q8), the rest float32; the time
    embedders' frequencies exp(-ln(10^4) i/128) as in the model."""
    rng = np.random.default_rng(seed)
    D, d, ld = fhp["dim"], hp["d"], hp["ldim"]
    t = {}

    def vec(n, scale=0.1, base=0.0):
        return (base + scale * rng.standard_normal(n)).astype(np.float32)

    def mat(rows, cols, gain=1.0):
        if q8 and rows >= 64 and cols >= 64 and cols % QK == 0:
            return q8_weight(rng, rows, cols, sigma=gain * 2.0 / np.sqrt(cols))
        return (rng.standard_normal(rows * cols) * gain / np.sqrt(cols)).astype(np.float32)

    t["flow.cond.weight"], t["flow.cond.bias"] = mat(D, d), vec(D)
    t["flow.input.weight"], t["flow.input.bias"] = mat(D, ld), vec(D)
    for i in range(2):
        p = f"flow.time.{i}."
        t[p + "freqs"] = np.exp(-np.log(1e4) * np.arange(128) / 128).astype(np.float32)
        t[p + "fc1.weight"], t[p + "fc1.bias"] = mat(D, 256), vec(D)
        t[p + "fc2.weight"], t[p + "fc2.bias"] = mat(D, D), vec(D)
        t[p + "norm.alpha"] = vec(D, 0.1, 1.0)
    for i in range(fhp["depth"]):
        p = f"flow.res.{i}."
        t[p + "norm.weight"], t[p + "norm.bias"] = vec(D, 0.1, 1.0), vec(D)
        t[p + "fc1.weight"], t[p + "fc1.bias"] = mat(D, D), vec(D)
        t[p + "fc2.weight"], t[p + "fc2.bias"] = mat(D, D, 0.5), vec(D)
        t[p + "ada.weight"], t[p + "ada.bias"] = mat(3 * D, D, 0.5), vec(3 * D)
    t["flow.final.ada.weight"], t["flow.final.ada.bias"] = mat(2 * D, D, 0.5), vec(2 * D)
    t["flow.final.out.weight"], t["flow.final.out.bias"] = mat(ld, D), vec(ld)
    return t


# Pocket TTS's Mimi decoder: the english_2026-09 settings the reference's
# converter writes (tools/convert_pocket_tts.py:56-72, 336-360): d_model 512,
# 8 heads, 2 layers, FFN 2048, 250 positions of context, 16x upsampling to
# 200 Hz, SEANet ratios 6, 5, 4 (1920 samples per latent at 24 kHz).
MIMI = dict(d=512, heads=8, ff=2048, n_layer=2, context=250, ldim=32, up_s=16, period=1e4, ratios=(6, 5, 4),
            nf=64, k=7, res_k=3, last_k=3, dil_base=2, compress=2, n_res=1)
MIMI_TINY = dict(d=64, heads=2, ff=128, n_layer=2, context=12, ldim=32, up_s=4, period=1e4, ratios=(3, 2),
                 nf=16, k=5, res_k=3, last_k=3, dil_base=2, compress=2, n_res=2)


def mimi_steps(hp: dict) -> list:
    """SEANet's decoder steps as pockettts/model.go:163-181 builds them:
    (kind, name, elu, cin, cout, k, stride, dilation) with kind "conv",
    "convtr" or "res" (a residual block: name.1 of kernel res_k at the
    dilation, then name.3 of kernel 1; cin = the block's channels)."""
    mult = 1 << len(hp["ratios"])
    nf, d = hp["nf"], hp["d"]
    out = [("conv", "mimi.dec.0", False, d, mult * nf, hp["k"], 1, 1)]
    idx = 1
    for r in hp["ratios"]:
        idx += 1
        out.append(("convtr", f"mimi.dec.{idx}", True, mult * nf, mult * nf // 2, 2 * r, r, 1))
        idx += 1
        dim = mult * nf // 2
        for j in range(hp["n_res"]):
            out.append(("res", f"mimi.dec.{idx}", False, dim, dim // hp["compress"], hp["res_k"], 1,
                        hp["dil_base"] ** j))
            idx += 1
        mult //= 2
    idx += 1
    out.append(("conv", f"mimi.dec.{idx}", True, nf, 1, hp["last_k"], 1, 1))
    return out


def mimi_model(hp: dict, seed: int = 15, q8: bool = True) -> dict:
    """Random-init Mimi decoder tensors under the reference's names
    (pockettts/model.go:105-181, 331-335), typed as its converter types them
    (tools/convert_pocket_tts.py:150-156): matrices of at least 64 x 64 whose
    rows are whole Q8_0 blocks Q8_0 (when q8), the rest float32.  Conv
    weights [cout][k*cin], transposed-conv weights [k*cout][cin]."""
    rng = np.random.default_rng(seed)
    d, ff, ld = hp["d"], hp["ff"], hp["ldim"]
    t = {}

    def vec(n, scale=0.1, base=0.0):
        return (base + scale * rng.standard_normal(n)).astype(np.float32)

    def mat(rows, cols, gain=1.0):
        if q8 and rows >= 64 and cols >= 64 and cols % QK == 0:
            return q8_weight(rng, rows, cols, sigma=gain * 2.0 / np.sqrt(cols))
        return (rng.standard_normal(rows * cols) * gain / np.sqrt(cols)).astype(np.float32)

    t["mimi.quant"] = mat(d, ld)
    t["mimi.up"] = vec(d * 2 * hp["up_s"], 0.3)
    for i in range(hp["n_layer"]):
        p = f"mimi.dec_tf.{i}."
        for n in ("norm1", "norm2"):
            t[p + n + ".weight"] = vec(d, 0.1, 1.0)
            t[p + n + ".bias"] = vec(d, 0.1)
        t[p + "attn_qkv.weight"] = mat(3 * d, d)
        t[p + "attn_out.weight"] = mat(d, d)
        t[p + "ff1.weight"] = mat(ff, d)
        t[p + "ff2.weight"] = mat(d, ff, 0.5)
        t[p + "ls1"] = vec(d, 0.05, 0.2)
        t[p + "ls2"] = vec(d, 0.05, 0.2)
    for kind, name, _, cin, cout, k, stride, _ in mimi_steps(hp):
        if kind == "conv":
            t[name + ".weight"], t[name + ".bias"] = mat(cout, k * cin), vec(cout)
        elif kind == "convtr":
            t[name + ".weight"], t[name + ".bias"] = mat(k * cout, cin), vec(cout)
        else:
            t[name + ".1.weight"], t[name + ".1.bias"] = mat(cout, k * cin), vec(cout)
            t[name + ".3.weight"], t[name + ".3.bias"] = mat(cin, cout, 0.5), vec(cin)
    return t


def mimi_latents(hp: dict, n: int, seed: int = 16) -> np.ndarray:
    """n latents as the speak loop hands them to the decoder (scaled back by
    the flow LM's mean and std): [n][ldim] ~ N(0, 1)."""
    return np.random.default_rng(seed).standard_normal((n, hp["ldim"])).astype(np.float32)


def pocket_inputs(hp: dict, frames: int, prefix: int = 64, seed: int = 6):
    """The text prefix (prefix x d random embedding rows) and teacher-forced
    latents (frames x ldim, N(0,1)), seeded."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((prefix, hp["d"])).astype(np.float32)
    lat = rng.standard_normal((frames, hp["ldim"])).astype(np.float32)
    return x, lat


# Parakeet-TDT-0.6B-shaped FastConformer encoder (24 layers of d 1024) and a
# tiny one for the oracle's own checks.
PARAKEET_TDT_06B = dict(d=1024, heads=8, layers=24, dff=4096, conv_kernel=31, sub_channels=256, n_mels=128,
                        xscaling=True, conv_norm="batch_norm")
CONFORMER_TINY = dict(d=64, heads=2, layers=2, dff=256, conv_kernel=9, sub_channels=32, n_mels=32,
                      xscaling=True, conv_norm="batch_norm")
# A cache-aware streaming FastConformer (Nemotron-Speech-Streaming-0.6B
# shape): chunked limited attention with 70 rows of left context and the
# four trained right contexts, a causal convolution of 9 taps with its
# LayerNorm, the causal pre-encoder.
NEMOTRON_STREAMING = dict(d=1024, heads=8, layers=24, dff=4096, conv_kernel=9, sub_channels=256, n_mels=128,
                          xscaling=True, conv_norm="layer_norm", att_style="chunked_limited", att_left=70,
                          att_right=13, context_choices=[(70, 13), (70, 6), (70, 1), (70, 0)], conv_left=8,
                          conv_right=0)


def conformer_model(hp: dict, seed: int = 9, pointwise_f16: bool = True, pre_f32: bool = False) -> dict:
    """Random-init encoder tensors named as conformer/model.go:370-422 reads
    them.  Linear weights Q8_0 (scales sized so activations stay O(1)); the
    pointwise convolutions float16 when pointwise_f16 (as Q8_0 model files
    keep them), else Q8_0; the pre-encoder's conv.3 and conv.6 float32 when
    pre_f32 (as the reference's converter writes them), else Q8_0; taps and
    vectors float32."""
    rng = np.random.default_rng(seed)
    d, c, ff, K = hp["d"], hp["sub_channels"], hp["dff"], hp["conv_kernel"]
    F = hp["n_mels"]
    causal = bool(hp.get("causal_sub", hp.get("att_style", "regular") == "chunked_limited"))
    for _ in range(3):
        F = F // 2 + 1 if causal else (F - 1) // 2 + 1
    t = {}

    def vec(n, scale=0.1, base=0.0):
        return (base + scale * rng.standard_normal(n)).astype(np.float32)

    def lin(rows, cols):
        return q8_weight(rng, rows, cols, sigma=2.0 / np.sqrt(cols))

    pe = "enc.pre_encode."
    for n in ("conv.0", "conv.2", "conv.5"):
        t[pe + n + ".weight"] = vec(c * 9, 0.3)
        t[pe + n + ".bias"] = vec(c)
    for n in ("conv.3", "conv.6"):
        t[pe + n + ".weight"] = vec(c * c, 2.0 / np.sqrt(c)) if pre_f32 else lin(c, c)
        t[pe + n + ".bias"] = vec(c)
    t[pe + "out.weight"] = lin(d, c * F)
    t[pe + "out.bias"] = vec(d)
    for i in range(hp["layers"]):
        p = f"enc.blocks.{i}."
        for f in ("ff1", "ff2"):
            t[p + f"norm_{f}.weight"] = vec(d, 0.1, 1.0)
            t[p + f"norm_{f}.bias"] = vec(d)
            t[p + f"{f}.linear1.weight"] = lin(ff, d)
            t[p + f"{f}.linear1.bias"] = vec(ff)
            t[p + f"{f}.linear2.weight"] = lin(d, ff)
            t[p + f"{f}.linear2.bias"] = vec(d)
        for n in ("norm_attn", "norm_conv", "norm_out"):
            t[p + n + ".weight"] = vec(d, 0.1, 1.0)
            t[p + n + ".bias"] = vec(d)
        for n in ("linear_q", "linear_k", "linear_v", "linear_out"):
            t[p + f"attn.{n}.weight"] = lin(d, d)
            t[p + f"attn.{n}.bias"] = vec(d)
        t[p + "attn.linear_pos.weight"] = lin(d, d)
        t[p + "attn.pos_bias_u"] = vec(d)
        t[p + "attn.pos_bias_v"] = vec(d)
        for n, rows in (("pointwise1", 2 * d), ("pointwise2", d)):
            if pointwise_f16:
                t[p + f"conv.{n}.weight"] = (rng.standard_normal(rows * d) / np.sqrt(d)).astype(np.float16)
            else:
                t[p + f"conv.{n}.weight"] = lin(rows, d)
        t[p + "conv.pointwise1.bias"] = vec(2 * d)
        t[p + "conv.pointwise2.bias"] = vec(d)
        t[p + "conv.depthwise.weight"] = vec(d * K, 0.3)
        t[p + "conv.depthwise.bias"] = vec(d)
        t[p + "conv.bn.weight"] = vec(d, 0.1, 1.0)
        t[p + "conv.bn.bias"] = vec(d)
        t[p + "conv.bn.running_mean"] = vec(d)
        t[p + "conv.bn.running_var"] = rng.uniform(0.5, 1.5, d).astype(np.float32)
    return t


def _slaney_mel(hz):
    f_sp, min_log_hz = 200.0 / 3, 1000.0
    return np.where(hz < min_log_hz, hz / f_sp, min_log_hz / f_sp + np.log(np.maximum(hz, 1e-12) / min_log_hz)
                    / (np.log(6.4) / 27))


def _slaney_hz(mel):
    f_sp, min_log_hz = 200.0 / 3, 1000.0
    min_log_mel = min_log_hz / f_sp
    return np.where(mel < min_log_mel, mel * f_sp, min_log_hz * np.exp(np.log(6.4) / 27 * (mel - min_log_mel)))


def log_mel(pcm: np.ndarray, n_mels: int, sr: int = 16000, n_fft: int = 512, win: int = 400, hop: int = 160):
    """NeMo-style log-mel features as conformer/mel.go computes them
    (pre-emphasis 0.97, n_fft/2 zero padding, centred symmetric Hann window,
    power spectrum, Slaney filterbank to 8 kHz, log(x + 2^-24), per-feature
    normalization), with numpy's FFT: (mel [n_mels][frames], frames, valid)."""
    n = len(pcm)
    frames, valid = n // hop + 1, n // hop
    pad = n_fft // 2
    padded = np.zeros(n + 2 * pad)
    x = pcm.astype(np.float64)
    padded[pad] = x[0]
    padded[pad + 1:pad + n] = x[1:] - 0.97 * x[:-1]
    window = np.zeros(n_fft)
    wp = (n_fft - win) // 2
    window[wp:wp + win] = 0.5 - 0.5 * np.cos(2 * np.pi * np.arange(win) / (win - 1))
    idx = np.arange(frames)[:, None] * hop + np.arange(n_fft)[None, :]
    seg = np.where(idx < len(padded), padded[np.minimum(idx, len(padded) - 1)], 0.0)
    spec = np.fft.rfft(seg * window, axis=1)
    power = (spec.real ** 2 + spec.imag ** 2).astype(np.float32).astype(np.float64)
    nf = n_fft // 2 + 1
    lo, hi = _slaney_mel(np.float64(0.0)), _slaney_mel(np.float64(8000.0))
    hz = _slaney_hz(lo + (hi - lo) * np.arange(n_mels + 2) / (n_mels + 1))
    f = sr * np.arange(nf) / n_fft
    fb = np.zeros((n_mels, nf), np.float32)
    for j in range(n_mels):
        lower = (f - hz[j]) / (hz[j + 1] - hz[j])
        upper = (hz[j + 2] - f) / (hz[j + 2] - hz[j + 1])
        fb[j] = (np.maximum(0, np.minimum(lower, upper)) * (2 / (hz[j + 2] - hz[j]))).astype(np.float32)
    mel = np.log(power @ fb.astype(np.float64).T + 1.0 / (1 << 24)).astype(np.float32).T.copy()
    nn = frames - 1
    rows = mel[:, :nn].astype(np.float64)
    mean = rows.mean(1, keepdims=True)
    std = np.sqrt(((rows - mean) ** 2).sum(1, keepdims=True) / max(nn - 1, 1))
    mel[:, :nn] = ((rows - mean) / (std + 1e-5)).astype(np.float32)
    mel[:, nn] = 0
    return np.ascontiguousarray(mel), frames, valid


def noise_mel(n_mels: int, seconds: float = 10.0, seed: int = 4, sr: int = 16000):
    """White noise N(0, 0.1^2) of the given length through log_mel."""
    rng = np.random.default_rng(seed)
    pcm = (rng.standard_normal(int(seconds * sr)) * 0.1).astype(np.float32)
    return log_mel(pcm, n_mels, sr)


# A Parakeet-TDT-shaped transducer head (FastConformer d=1024, 2-layer LSTM
# of 640, joint 640, 1024 tokens + blank, durations 0..4).
RNNT_TDT = dict(d=1024, pred_hidden=640, pred_layers=2, pred_vocab=1025, joint_hidden=640, joint_act="relu",
                head_kind="tdt", durations=[0, 1, 2, 3, 4], max_symbols=10, blank=-1)
RNNT_TINY = dict(d=64, pred_hidden=64, pred_layers=2, pred_vocab=97, joint_hidden=64, joint_act="relu",
                 head_kind="rnnt", blank=-1)


def rnnt_model(hp: dict, seed: int = 21, blank_bias: float = 2.0, out_sigma: float = 2.0,
               pred_sigma: float = 8.0) -> dict:
    """Random-init decoder tensors named as conformer/model.go:306-315 reads
    them: Q8_0 matrices sized so gates and logits stay O(1), float32
    vectors, the embedding with NeMo's extra padding row, and blank's output
    bias raised by blank_bias so that frames advance as well as emit."""
    rng = np.random.default_rng(seed)
    H, L, V, J, d = hp["pred_hidden"], hp["pred_layers"], hp["pred_vocab"], hp["joint_hidden"], hp["d"]
    nd = len(hp.get("durations", [])) if hp.get("head_kind", "rnnt") == "tdt" else 0
    blank = hp.get("blank", -1)
    blank = blank if blank >= 0 else V - 1
    t = {"pred.embed.weight": (rng.standard_normal((V, H)) * 0.5).astype(np.float32)}
    for i in range(L):
        p = f"pred.lstm.{i}."
        t[p + "Wx"] = q8_weight(rng, 4 * H, H, sigma=2.0 / np.sqrt(H))
        t[p + "Wh"] = q8_weight(rng, 4 * H, H, sigma=2.0 / np.sqrt(H))
        t[p + "bias"] = (rng.standard_normal(4 * H) * 0.1).astype(np.float32)
    t["joint.enc.weight"] = q8_weight(rng, J, d, sigma=2.0 / np.sqrt(d))
    t["joint.enc.bias"] = (rng.standard_normal(J) * 0.1).astype(np.float32)
    t["joint.pred.weight"] = q8_weight(rng, J, H, sigma=pred_sigma / np.sqrt(H))
    t["joint.pred.bias"] = (rng.standard_normal(J) * 0.1).astype(np.float32)
    t["joint.out.weight"] = q8_weight(rng, V + nd, J, sigma=out_sigma / np.sqrt(J))
    ob = (rng.standard_normal(V + nd) * 0.1).astype(np.float32)
    ob[blank] += np.float32(blank_bias)
    t["joint.out.bias"] = ob
    return t


def rnnt_encoder_output(hp: dict, T: int, seed: int = 22) -> np.ndarray:
    """Synthetic encoder output [T][d] (unit normal)."""
    return np.random.default_rng(seed).standard_normal((T, hp["d"])).astype(np.float32)
