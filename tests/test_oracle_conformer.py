"""Pins the oracle's FastConformer encoder (conformer/encoder.go, model.go)
without a GPU: closed forms for the relative position table and the batch
norm fold, an independent float64 restatement of the pre-encoder and of
the blocks (relative-position attention written from its definition,
score(q, k) = (q+u).k_k + (q+v).p(q-k)), and invariants of the valid
length."""
import numpy as np
import pytest

from gorelaxor_amd.synth import CONFORMER_TINY, conformer_model, noise_mel, q8_dequant


def test_rel_pos_closed_form(orc):
    """relPosEmb (encoder.go:171-191): row i is relative position n-1-i;
    column 2j sin, 2j+1 cos of pos * 10000^(-2j/d); position 0 gives sin 0,
    cos 1 exactly."""
    n, d = 9, 16
    pe = orc.conf_rel_pos(n, d)
    assert pe.shape == (2 * n - 1, d)
    pos = (n - 1 - np.arange(2 * n - 1))[:, None].astype(np.float64)
    div = 10000.0 ** (-np.arange(0, d, 2) / d)
    assert np.abs(pe[:, 0::2] - np.sin(pos * div)).max() < 1e-6
    assert np.abs(pe[:, 1::2] - np.cos(pos * div)).max() < 1e-6
    assert np.all(pe[n - 1, 0::2] == 0.0) and np.all(pe[n - 1, 1::2] == 1.0)
    assert np.array_equal(pe[n - 1 + 3, 0::2], -pe[n - 1 - 3, 0::2])  # sin is odd


def test_bn_fold_closed_form(orc):
    """conformer/model.go:408-418: s = f32(g / sqrt(var + 1e-5)) from float64,
    b = beta - mean*s in float32."""
    rng = np.random.default_rng(3)
    d = 64
    g, beta, mean = (rng.standard_normal(d).astype(np.float32) for _ in range(3))
    var = rng.uniform(0.1, 2, d).astype(np.float32)
    s, b = orc.conf_bn_fold(g, beta, mean, var)
    want_s = (g.astype(np.float64) / np.sqrt(var.astype(np.float64) + 1e-5)).astype(np.float32)
    assert np.array_equal(s, want_s)
    assert np.array_equal(b, beta - mean * want_s)


def _w(t, name, rows, cols):
    a = t[name]
    if a.dtype == np.float16:  # Weight.ToQ8 at load
        from oracle.oracle import quant_q8
        a = quant_q8(a.astype(np.float32))
    return q8_dequant(a, rows, cols).astype(np.float64)


def _ref_subsample(hp, t, mel, valid):
    """float64 pre-encoder: conv0, ReLU, depthwise, pointwise, ReLU,
    depthwise, pointwise, ReLU (rows past each stage's valid length zero),
    flatten [t][c*F+f], output Linear."""
    c, nm = hp["sub_channels"], hp["n_mels"]
    frames = mel.shape[1]
    pe = "enc.pre_encode."
    so = lambda n: (n - 1) // 2 + 1  # noqa: E731
    x = np.zeros((frames, nm))
    x[:valid] = mel[:, :valid].T

    def conv(inp, w, b, depthwise):
        T, F = inp.shape[:2]
        T1, F1 = so(T), so(F)
        pad = np.zeros((T + 2, F + 2) + inp.shape[2:])
        pad[1:T + 1, 1:F + 1] = inp
        w = w.astype(np.float64).reshape(c, 3, 3)
        out = np.tile(b.astype(np.float64), (T1, F1, 1))
        for kt in range(3):
            for kf in range(3):
                tap = pad[kt:kt + 2 * T1:2, kf:kf + 2 * F1:2]
                out += (tap if depthwise else tap[..., None]) * w[:, kt, kf]
        return out

    L = so(valid)
    x = conv(x, t[pe + "conv.0.weight"], t[pe + "conv.0.bias"], False)
    x[L:] = 0
    x = np.maximum(x, 0)
    for i, (dw, pw) in enumerate((("conv.2", "conv.3"), ("conv.5", "conv.6"))):
        x = conv(x, t[pe + dw + ".weight"], t[pe + dw + ".bias"], True)
        L = so(L)
        x[L:] = 0
        x = x @ _w(t, pe + pw + ".weight", c, c).T + t[pe + pw + ".bias"]
        x[L:] = 0
        x = np.maximum(x, 0)
    T, F = x.shape[:2]
    flat = x.transpose(0, 2, 1).reshape(T, c * F)
    out = flat @ _w(t, pe + "out.weight", hp["d"], c * F).T + t[pe + "out.bias"]
    return out, T, min(L, T)


def _ref_block(hp, t, i, x, L):
    d, H, K = hp["d"], hp["heads"], hp["conv_kernel"]
    hd = d // H
    T = x.shape[0]
    p = f"enc.blocks.{i}."
    V = lambda n: t[p + n].astype(np.float64)  # noqa: E731

    def ln(z, n):
        mu = z.mean(-1, keepdims=True)
        return (z - mu) / np.sqrt(z.var(-1, keepdims=True) + 1e-5) * V(n + ".weight") + V(n + ".bias")

    def ff(z, f):
        h = ln(z, "norm_" + f) @ _w(t, p + f + ".linear1.weight", hp["dff"], d).T + V(f + ".linear1.bias")
        h = h / (1 + np.exp(-h))
        return z + 0.5 * (h @ _w(t, p + f + ".linear2.weight", d, hp["dff"]).T + V(f + ".linear2.bias"))

    x = ff(x, "ff1")
    h = ln(x, "norm_attn")
    lin = lambda n: h @ _w(t, p + f"attn.{n}.weight", d, d).T + V(f"attn.{n}.bias")  # noqa: E731
    q, k, v = lin("linear_q"), lin("linear_k"), lin("linear_v")
    from oracle.oracle import conf_rel_pos
    pos = conf_rel_pos(T, d).astype(np.float64) @ _w(t, p + "attn.linear_pos.weight", d, d).T
    u, w = V("attn.pos_bias_u"), V("attn.pos_bias_v")
    att = np.zeros((T, d))
    for hh in range(H):
        sl = slice(hh * hd, (hh + 1) * hd)
        for qi in range(min(L, T)):
            s = np.array([((q[qi, sl] + u[sl]) @ k[kj, sl] + (q[qi, sl] + w[sl]) @ pos[T - 1 - (qi - kj), sl])
                          for kj in range(L)]) / np.sqrt(hd)
            a = np.exp(s - s.max())
            att[qi, sl] = (a / a.sum()) @ v[:L, sl]
    x = x + att @ _w(t, p + "attn.linear_out.weight", d, d).T + V("attn.linear_out.bias")
    h = ln(x, "norm_conv")
    a = h @ _w(t, p + "conv.pointwise1.weight", 2 * d, d).T + V("conv.pointwise1.bias")
    g = a[:, :d] / (1 + np.exp(-a[:, d:]))
    g[L:] = 0
    dw = V("conv.depthwise.weight").reshape(d, K)
    pad = (K - 1) // 2
    gp = np.zeros((T + K - 1, d))
    gp[pad:pad + T] = g
    y = np.tile(V("conv.depthwise.bias"), (T, 1))
    for j in range(K):
        y += dw[:, j] * gp[j:j + T]
    y = (y - V("conv.bn.running_mean")) / np.sqrt(V("conv.bn.running_var") + 1e-5) * V("conv.bn.weight") \
        + V("conv.bn.bias")
    y = y / (1 + np.exp(-y))
    x = x + y @ _w(t, p + "conv.pointwise2.weight", d, d).T + V("conv.pointwise2.bias")
    x = ff(x, "ff2")
    return ln(x, "norm_out")


def _rel(got, want):
    return float(np.sqrt(((got - want) ** 2).mean() / (want ** 2).mean()))


@pytest.fixture(scope="module")
def tiny():
    hp = dict(CONFORMER_TINY)
    return hp, conformer_model(hp, seed=9)


def test_subsample_vs_float64(orc, tiny):
    """encoder.go:123-167 within the error Q8_0 activation rounding allows."""
    hp, t = tiny
    m = orc.ConformerOracle(hp, t)
    mel, frames, valid = noise_mel(hp["n_mels"], seconds=1.0, seed=4)
    got, T, L = m.subsample(mel, valid - 7)
    want, Tw, Lw = _ref_subsample(hp, t, mel, valid - 7)
    assert (T, L) == (Tw, Lw) == (13, 12)
    assert _rel(got[:L], want[:L]) < 0.025


def test_block_vs_float64(orc, tiny):
    """One block (encoder.go:411-429) on an input with valid length L < T:
    the rows below L within Q8_0 rounding error of the float64 graph."""
    hp, t = tiny
    m = orc.ConformerOracle(hp, t)
    rng = np.random.default_rng(8)
    T, L = 40, 37
    x = rng.standard_normal((T, hp["d"])).astype(np.float32)
    got = m.block(1, x, L)
    want = _ref_block(hp, t, 1, x.astype(np.float64), L)
    assert _rel(got[:L], want[:L]) < 0.02  # a rel-shift off by one gives 0.07


def test_encode_vs_float64(orc, tiny):
    """The whole encode: pre-encoder, xscale, both blocks."""
    hp, t = tiny
    m = orc.ConformerOracle(hp, t)
    mel, frames, valid = noise_mel(hp["n_mels"], seconds=1.5, seed=5)
    got, L = m.encode(mel, valid)
    x, T, Lw = _ref_subsample(hp, t, mel, valid)
    x = x * np.sqrt(hp["d"])
    for i in range(hp["layers"]):
        x = _ref_block(hp, t, i, x, Lw)
    assert L == Lw
    assert _rel(got[:L], x[:L]) < 0.025


def test_encode_ignores_padding_frames(orc, tiny):
    """Frames at or past valid never reach the output (encoder.go:126-130)."""
    hp, t = tiny
    m = orc.ConformerOracle(hp, t)
    mel, frames, valid = noise_mel(hp["n_mels"], seconds=1.0, seed=6)
    v = valid - 20
    a, L = m.encode(mel, v)
    mel2 = mel.copy()
    mel2[:, v:] = np.random.default_rng(1).standard_normal((hp["n_mels"], frames - v))
    b, L2 = m.encode(mel2, v)
    assert L == L2 and np.array_equal(a, b)


def test_encode_layers_compose(orc, tiny):
    """encode over both layers == the pre-encoder, xscale, then each block."""
    hp, t = tiny
    m = orc.ConformerOracle(hp, t)
    mel, frames, valid = noise_mel(hp["n_mels"], seconds=1.0, seed=7)
    full, L = m.encode(mel, valid)
    x, T, L1 = m.subsample(mel, valid)
    x = x * np.float32(np.sqrt(hp["d"]))
    for i in range(hp["layers"]):
        x = m.block(i, x, L1)
    assert np.array_equal(full, x)
