"""A float64 restatement of the FastConformer encoder (conformer/
encoder.go, stream.go of github.com/xattribution/gorelaxor), written from
the model's definition rather than from the reference's operation order,
to pin the oracle within the error Q8_0 activation rounding allows.

Attention is written per query from score(q, k) = (q+u).k_k + (q+v).p(q-k)
over the query's keys [lo, hi); the depthwise convolution as a sum over its
taps with the frames before the first one taken from a cache or left out;
the pre-encoder's convolutions over an explicitly padded plane."""
import numpy as np


def dequant(t, name, rows, cols):
    from gorelaxor_amd.synth import q8_dequant
    a = t[name]
    if a.dtype == np.float16:  # Weight.ToQ8 at load
        from oracle.oracle import quant_q8
        a = quant_q8(a.astype(np.float32))
    return q8_dequant(a, rows, cols).astype(np.float64)


def causal(hp):
    return bool(hp.get("causal_sub", hp.get("att_style", "regular") == "chunked_limited"))


def sub_out(n, c):
    return n // 2 + 1 if c else (n - 1) // 2 + 1


def subsample(hp, t, mel, valid):
    """conv0, ReLU, depthwise, pointwise, ReLU, depthwise, pointwise, ReLU
    (rows past each stage's valid length zero), flatten [t][c*F+f], output
    Linear; a causal pre-encoder pads two before and one after."""
    c, nm = hp["sub_channels"], hp["n_mels"]
    cs = causal(hp)
    pl = 2 if cs else 1
    frames = mel.shape[1]
    pe = "enc.pre_encode."
    x = np.zeros((frames, nm))
    x[:valid] = mel[:, :valid].T

    def conv(inp, w, b, depthwise):
        T, F = inp.shape[:2]
        T1, F1 = sub_out(T, cs), sub_out(F, cs)
        pad = np.zeros((2 * T1 + 2, 2 * F1 + 2) + inp.shape[2:])
        pad[pl:pl + T, pl:pl + F] = inp
        w = w.astype(np.float64).reshape(c, 3, 3)
        out = np.tile(b.astype(np.float64), (T1, F1, 1))
        for kt in range(3):
            for kf in range(3):
                tap = pad[kt:kt + 2 * T1:2, kf:kf + 2 * F1:2]
                out += (tap if depthwise else tap[..., None]) * w[:, kt, kf]
        return out

    L = sub_out(valid, cs)
    x = conv(x, t[pe + "conv.0.weight"], t[pe + "conv.0.bias"], False)
    x[L:] = 0
    x = np.maximum(x, 0)
    for dw, pw in (("conv.2", "conv.3"), ("conv.5", "conv.6")):
        x = conv(x, t[pe + dw + ".weight"], t[pe + dw + ".bias"], True)
        L = sub_out(L, cs)
        x[L:] = 0
        w = t[pe + pw + ".weight"]
        wd = w.astype(np.float64) if w.dtype == np.float32 else dequant(t, pe + pw + ".weight", c, c)
        x = x @ wd.reshape(c, c).T + t[pe + pw + ".bias"]
        x[L:] = 0
        x = np.maximum(x, 0)
    T, F = x.shape[:2]
    flat = x.transpose(0, 2, 1).reshape(T, c * F)
    out = flat @ dequant(t, pe + "out.weight", hp["d"], c * F).T + t[pe + "out.bias"]
    return out, T, max(0, min(L, T))


def rel_pos(r, d):
    """The sinusoidal embedding of relative position r (encoder.go:171-191)."""
    j = np.arange(0, d, 2)
    a = r * 10000.0 ** (-j / d)
    out = np.zeros(d)
    out[0::2], out[1::2] = np.sin(a), np.cos(a)
    return out


def pad_left(hp):
    if hp.get("conv_left", -1) >= 0 and hp.get("conv_right", -1) >= 0:
        return hp["conv_left"]
    return (hp["conv_kernel"] - 1) // 2


def block(hp, t, i, x, L, keys, kv_before=None, conv_prev=None):
    """One block on x [T][d] (valid rows L): keys(q) gives query q's key
    range over the c + T key rows (the c normalized rows of kv_before, then
    this call's own); conv_prev the pad_left gated frames before the first
    (None: none).  Returns (x, key rows, gated frames)."""
    d, H, K = hp["d"], hp["heads"], hp["conv_kernel"]
    hd = d // H
    T = x.shape[0]
    p = f"enc.blocks.{i}."
    V = lambda n: t[p + n].astype(np.float64)  # noqa: E731

    def ln(z, w, b):
        mu = z.mean(-1, keepdims=True)
        return (z - mu) / np.sqrt(z.var(-1, keepdims=True) + 1e-5) * w + b

    def ff(z, f):
        h = ln(z, V(f"norm_{f}.weight"), V(f"norm_{f}.bias"))
        h = h @ dequant(t, p + f + ".linear1.weight", hp["dff"], d).T + V(f + ".linear1.bias")
        h = h / (1 + np.exp(-h))
        return z + 0.5 * (h @ dequant(t, p + f + ".linear2.weight", d, hp["dff"]).T + V(f + ".linear2.bias"))

    x = ff(x, "ff1")
    h = ln(x, V("norm_attn.weight"), V("norm_attn.bias"))
    kv = h if kv_before is None else np.concatenate([kv_before, h])
    c = kv.shape[0] - T
    W = lambda n: dequant(t, p + f"attn.{n}.weight", d, d)  # noqa: E731
    q = h @ W("linear_q").T + V("attn.linear_q.bias")
    k = kv @ W("linear_k").T + V("attn.linear_k.bias")
    v = kv @ W("linear_v").T + V("attn.linear_v.bias")
    wpos = W("linear_pos")
    u, w = V("attn.pos_bias_u"), V("attn.pos_bias_v")
    att = np.zeros((T, d))
    for qi in range(T):
        lo, hi = keys(c + qi)
        if hi <= lo:
            continue
        kj = np.arange(lo, hi)
        pos = np.stack([rel_pos(c + qi - j, d) for j in kj]) @ wpos.T
        for hh in range(H):
            sl = slice(hh * hd, (hh + 1) * hd)
            s = (k[kj, sl] @ (q[qi, sl] + u[sl]) + pos[:, sl] @ (q[qi, sl] + w[sl])) / np.sqrt(hd)
            a = np.exp(s - s.max())
            att[qi, sl] = (a / a.sum()) @ v[kj, sl]
    x = x + att @ W("linear_out").T + V("attn.linear_out.bias")
    h = ln(x, V("norm_conv.weight"), V("norm_conv.bias"))
    a = h @ dequant(t, p + "conv.pointwise1.weight", 2 * d, d).T + V("conv.pointwise1.bias")
    g = a[:, :d] / (1 + np.exp(-a[:, d:]))
    g[L:] = 0
    dw = V("conv.depthwise.weight").reshape(d, K)
    pl = pad_left(hp)
    gp = np.zeros((T + K - 1, d))
    if conv_prev is not None:
        gp[:pl] = conv_prev
    gp[pl:pl + T] = g
    y = np.tile(V("conv.depthwise.bias"), (T, 1))
    for j in range(K):
        y += dw[:, j] * gp[j:j + T]
    if hp.get("conv_norm", "batch_norm") == "layer_norm":
        y = ln(y, V("conv.bn.weight"), V("conv.bn.bias"))
    else:
        y = (y - V("conv.bn.running_mean")) / np.sqrt(V("conv.bn.running_var") + 1e-5) * V("conv.bn.weight") \
            + V("conv.bn.bias")
    y = y / (1 + np.exp(-y))
    x = x + y @ dequant(t, p + "conv.pointwise2.weight", d, d).T + V("conv.pointwise2.bias")
    x = ff(x, "ff2")
    return ln(x, V("norm_out.weight"), V("norm_out.bias")), kv, g


def offline_keys(hp, T, L):
    """offlineKeys (encoder.go:196-212), cut at L: q -> (lo, hi)."""
    al, ar = hp.get("att_left", -1), hp.get("att_right", -1)
    if hp.get("att_style", "regular") == "chunked_limited" and al >= 0 and ar >= 0:
        ch, lc = ar + 1, al // (ar + 1)
        f = lambda q: (max(0, (q // ch - lc) * ch), min(T, (q // ch + 1) * ch))  # noqa: E731
    elif al >= 0 and ar >= 0 and T - 1 > min(al, ar):
        f = lambda q: (max(0, q - al), min(T, q + ar + 1))  # noqa: E731
    else:
        f = lambda q: (0, T)  # noqa: E731
    return lambda q: (0, 0) if q >= L else (f(q)[0], min(f(q)[1], L))


def encode(hp, t, mel, valid):
    x, T, L = subsample(hp, t, mel, valid)
    if hp.get("xscaling", True):
        x = x * np.sqrt(hp["d"])
    keys = offline_keys(hp, T, L)
    for i in range(hp["layers"]):
        x = block(hp, t, i, x, L, keys)[0]
    return x[:L], L


def stream(hp, t, g, chunks):
    """streamEncode (stream.go:249-307) over the chunks: each chunk's rows.
    The chunk's keys are the last `left` earlier rows and its own, limited
    to whole chunks as NeMo's cache slots do."""
    d, nl, pl = hp["d"], hp["layers"], pad_left(hp)
    kv = [np.zeros((0, d)) for _ in range(nl)]
    conv = [np.zeros((pl, d)) for _ in range(nl)]
    out = []
    for mel, length, first in chunks:
        x, T, L = subsample(hp, t, mel, length)
        if not first:
            x, T, L = x[min(g["drop"], T):], max(0, T - g["drop"]), max(0, L - g["drop"])
        L = min(L, T)
        if T <= 0:
            continue
        if hp.get("xscaling", True):
            x = x * np.sqrt(d)
        c = kv[0].shape[0]
        slot0 = g["left"] - c

        def keys(q):
            if q - c >= L:
                return 0, 0
            qc = (slot0 + q) // g["chunk"]
            lo = max(0, (qc - g["left_chunks"]) * g["chunk"] - slot0)
            hi = min(c + L, (qc + 1) * g["chunk"] - slot0)
            return lo, max(hi, lo)

        for i in range(nl):
            x, rows, gl = block(hp, t, i, x, L, keys, kv[i], conv[i])
            kv[i] = rows[-g["left"]:] if g["left"] > 0 else rows[:0]
            conv[i] = np.concatenate([conv[i], gl])[-pl:] if pl else conv[i]
        out.append(x[:L])
    return out
