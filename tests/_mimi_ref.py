"""An independent float64 restatement of pocket-TTS's Mimi decoder
(pockettts/mimi.go:122-152, nn.go:51-64, 142-327) over a whole latent
sequence at once: no streaming state, causal convolutions with zero left
padding, transposed convolutions as full overlap-add, windowed causal
attention over every position.  Pins the oracle's streamed decode (one
latent per call, carried rows, partials and caches) up to float32
rounding."""
import numpy as np

from gorelaxor_amd.synth import mimi_steps, q8_dequant


def _mat(t, name, rows, cols):
    w = t[name]
    if w.dtype == np.uint8:
        return q8_dequant(w, rows, cols).astype(np.float64)
    return np.asarray(w, np.float64).reshape(rows, cols)


def elu(x):
    return np.where(x > 0, x, np.expm1(np.minimum(x, 0)))


def gelu(x):
    return 0.5 * x * (1 + np.tanh(0.7978845608028654 * x * (1 + 0.044715 * x * x)))


def ln(x, w, b, eps=1e-5):
    m = x.mean(axis=1, keepdims=True)
    v = ((x - m) ** 2).mean(axis=1, keepdims=True)
    return (x - m) / np.sqrt(v + eps) * w + b


def rope(x, heads, freqs, pos0):
    T, d = x.shape
    hd = d // heads
    y = x.reshape(T, heads, hd // 2, 2).copy()
    p = np.arange(pos0, pos0 + T, dtype=np.float64)[:, None]
    a = (freqs.astype(np.float32)[None, :] * p.astype(np.float32)).astype(np.float64)  # f32(f * pos)
    c, s = np.cos(a)[:, None, :], np.sin(a)[:, None, :]
    r, i = y[..., 0].copy(), y[..., 1].copy()
    y[..., 0] = r * c - i * s
    y[..., 1] = r * s + i * c
    return y.reshape(T, d)


def transformer(hp, t, x):
    T, d = x.shape
    H, hd = hp["heads"], d // hp["heads"]
    freqs = (hp["period"] ** (-2.0 * np.arange(hd // 2) / hd)).astype(np.float32)
    for i in range(hp["n_layer"]):
        p = f"mimi.dec_tf.{i}."
        h = ln(x, t[p + "norm1.weight"], t[p + "norm1.bias"])
        qkv = h @ _mat(t, p + "attn_qkv.weight", 3 * d, d).T
        q, k, v = rope(qkv[:, :d], H, freqs, 0), rope(qkv[:, d:2 * d], H, freqs, 0), qkv[:, 2 * d:]
        att = np.zeros((T, d))
        for hh in range(H):
            sl = slice(hh * hd, (hh + 1) * hd)
            s = q[:, sl] @ k[:, sl].T / np.sqrt(hd)
            for r in range(T):
                lo = max(0, r - hp["context"] + 1)
                row = np.full(T, -np.inf)
                row[lo:r + 1] = s[r, lo:r + 1]
                e = np.exp(row - row.max())
                att[r, sl] = (e / e.sum()) @ v[:, sl]
        x = x + t[p + "ls1"] * (att @ _mat(t, p + "attn_out.weight", d, d).T)
        h = ln(x, t[p + "norm2.weight"], t[p + "norm2.bias"])
        f = gelu(h @ _mat(t, p + "ff1.weight", hp["ff"], d).T)
        x = x + t[p + "ls2"] * (f @ _mat(t, p + "ff2.weight", d, hp["ff"]).T)
    return x


def conv(t, name, x, cin, cout, k, stride, dil):
    w = _mat(t, name + ".weight", cout, k * cin).reshape(cout, k, cin)
    P = (k - 1) * dil + 1 - stride
    xp = np.concatenate([np.zeros((P, cin)), x])
    To = x.shape[0] // stride
    y = np.tile(np.asarray(t[name + ".bias"], np.float64), (To, 1))
    for j in range(k):
        y += xp[np.arange(To) * stride + j * dil] @ w[:, j, :].T
    return y


def convtr(t, name, x, cin, cout, k, stride):
    w = _mat(t, name + ".weight", k * cout, cin).reshape(k, cout, cin)
    T = x.shape[0]
    full = np.tile(np.asarray(t[name + ".bias"], np.float64), ((T - 1) * stride + k, 1))
    for j in range(k):
        full[np.arange(T) * stride + j] += x @ w[j].T
    return full[:T * stride]


def decode(hp, t, lat):
    """n latents [n][ldim] -> n * up_s * prod(ratios) samples (float64)."""
    n = lat.shape[0]
    d, S = hp["d"], hp["up_s"]
    z = np.asarray(lat, np.float64) @ _mat(t, "mimi.quant", d, hp["ldim"]).T
    up = np.asarray(t["mimi.up"], np.float64).reshape(d, 2 * S)
    full = np.zeros(((n - 1) * S + 2 * S, d))
    for j in range(2 * S):
        full[np.arange(n) * S + j] += z * up[:, j]
    x = transformer(hp, t, full[:n * S])
    for kind, name, el, cin, cout, k, stride, dil in mimi_steps(hp):
        if el:
            x = elu(x)
        if kind == "conv":
            x = conv(t, name, x, cin, cout, k, stride, dil)
        elif kind == "convtr":
            x = convtr(t, name, x, cin, cout, k, stride)
        else:
            h = elu(conv(t, name + ".1", elu(x), cin, cout, k, 1, dil))
            x = x + conv(t, name + ".3", h, cout, cin, 1, 1, 1)
    return x[:, 0]
