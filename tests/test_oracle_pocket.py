"""Pins the oracle's pocket-TTS flow-LM transformer (pockettts/nn.go,
lm.go) and the float route of MatMulF32 (internal/kern/gemm.go:116-259)
without a GPU: closed forms for the rotary embedding, exact rational
evaluation of the packed micro-kernel's fma chain, the reference tests'
tolerances for the float route, and an independent float64 restatement of
the transformer."""
import numpy as np
import pytest

from gorelaxor_amd.synth import POCKET_TTS_TINY, pocket_inputs, pocket_model, q8_dequant
from tests._exact import bits, fma32


def test_rope_freqs_closed_form(orc):
    """ropeFreqs (nn.go:69-76): f_i = period^(-2i/head_dim)."""
    for hd in (64, 128, 24):
        f = orc.rope_freqs(hd, 1e4)
        want = 1e4 ** (-2.0 * np.arange(hd // 2) / hd)
        assert f[0] == 1.0
        assert np.all(np.abs(f - want) <= 2e-6 * want)


def test_apply_rope_is_a_rotation(orc):
    """applyRope (nn.go:80-93): position 0 leaves x unchanged bit for bit;
    any position multiplies each pair by e^(i f pos) (float64 within 1e-5)."""
    rng = np.random.default_rng(2)
    heads, hd = 4, 64
    f = orc.rope_freqs(hd, 1e4)
    x = rng.standard_normal(heads * hd).astype(np.float32)
    assert np.array_equal(orc.apply_rope(x, heads, f, 0), x)
    for pos in (1, 7, 313):
        y = orc.apply_rope(x, heads, f, pos).reshape(heads, hd // 2, 2)
        z = x.reshape(heads, hd // 2, 2).astype(np.float64)
        ang = f.astype(np.float64) * pos
        want_r = z[..., 0] * np.cos(ang) - z[..., 1] * np.sin(ang)
        want_i = z[..., 0] * np.sin(ang) + z[..., 1] * np.cos(ang)
        assert np.abs(y[..., 0] - want_r).max() < 1e-5 and np.abs(y[..., 1] - want_i).max() < 1e-5


@pytest.mark.parametrize("m,n,k", [(1, 70, 64), (3, 33, 96), (17, 40, 128), (64, 64, 64), (64, 50, 300)])
def test_matmul_f32_vs_float64(orc, m, n, k):
    """TestMatMulTypes (kern_test.go:30-73): both float routes (m <= 16
    gemvRows; m > 16 the 6x16 panels plus gemv for the last m % 6 rows)
    within 1e-3 of float64, with bias."""
    rng = np.random.default_rng(1)
    a = (rng.random((m, k)) * 2 - 1).astype(np.float32)
    b = (rng.random((n, k)) * 2 - 1).astype(np.float32)
    bias = rng.random(n).astype(np.float32)
    got = orc.matmul_f32(a, b, bias)
    want = a.astype(np.float64) @ b.astype(np.float64).T + bias
    assert np.abs(got - want).max() <= 1e-3


def test_matmul_f32_packed_order_exact(orc):
    """Rows in whole groups of six follow k6x16avx (kernels_amd64.s:5-88):
    acc = fma(a_k, b_k, acc) over k in order, then acc + C; checked in exact
    rational arithmetic on the first rows."""
    rng = np.random.default_rng(3)
    m, n, k = 18, 5, 40
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((n, k)).astype(np.float32)
    got = orc.matmul_f32(a, b)
    for i in (0, 5, 11):
        for j in range(n):
            acc = 0.0
            for kk in range(k):
                acc = fma32(a[i, kk], b[j, kk], acc)
            want = np.float32(np.float32(acc) + np.float32(0.0))
            assert bits(got[i, j]) == bits(want), (i, j)


def _ref_forward(hp, t, x, pos0, k_cache, v_cache, freqs):
    """float64 flow-LM transformer with the exact Q8_0 weights and unrounded
    activations: pre-LN blocks, rotary q/k, causal attention over the cache,
    tanh-GELU MLP."""
    d, heads, ff = hp["d"], hp["heads"], hp["ff"]
    hd = d // heads
    W = lambda n, r, c: q8_dequant(t[n], r, c).astype(np.float64)  # noqa: E731
    V = lambda n: t[n].astype(np.float64)  # noqa: E731
    T = x.shape[0]

    def ln(z, w, b):
        mu = z.mean(-1, keepdims=True)
        return (z - mu) / np.sqrt(z.var(-1, keepdims=True) + 1e-5) * w + b

    def rope(z, pos):
        z = z.reshape(heads, hd // 2, 2)
        ang = freqs.astype(np.float64) * pos
        c, s = np.cos(ang), np.sin(ang)
        return np.stack([z[..., 0] * c - z[..., 1] * s, z[..., 0] * s + z[..., 1] * c], -1).reshape(d)

    for i in range(hp["n_layer"]):
        p = f"lm.blk.{i}."
        h = ln(x, V(p + "norm1.weight"), V(p + "norm1.bias"))
        qkv = h @ W(p + "attn_qkv.weight", 3 * d, d).T
        q = np.stack([rope(qkv[r, :d], pos0 + r) for r in range(T)])
        k = np.stack([rope(qkv[r, d:2 * d], pos0 + r) for r in range(T)])
        k_cache[i][pos0:pos0 + T] = k
        v_cache[i][pos0:pos0 + T] = qkv[:, 2 * d:]
        K, Vv = k_cache[i][:pos0 + T], v_cache[i][:pos0 + T]
        att = np.zeros((T, d))
        for hh in range(heads):
            sl = slice(hh * hd, (hh + 1) * hd)
            s = q[:, sl] @ K[:, sl].T / np.sqrt(hd)
            s = s + np.triu(np.full((T, pos0 + T), -np.inf), pos0 + 1)
            a = np.exp(s - s.max(-1, keepdims=True))
            a /= a.sum(-1, keepdims=True)
            att[:, sl] = a @ Vv[:, sl]
        x = x + att @ W(p + "attn_out.weight", d, d).T
        h = ln(x, V(p + "norm2.weight"), V(p + "norm2.bias"))
        f = h @ W(p + "ff1.weight", ff, d).T
        f = 0.5 * f * (1 + np.tanh(np.sqrt(2 / np.pi) * f * (1 + 0.044715 * f * f)))
        x = x + f @ W(p + "ff2.weight", d, ff).T
    return x


def test_oracle_flow_lm_vs_float64(orc):
    """flowLM.text / run / step (lm.go:164-195): the prefix, then frames,
    within the error Q8_0 activation rounding allows of the float64 graph."""
    hp = dict(POCKET_TTS_TINY)
    t = pocket_model(hp, seed=5)
    x, lat = pocket_inputs(hp, 6, prefix=20, seed=6)
    m = orc.PocketOracle(hp, t)
    kc = [np.zeros((hp["max_pos"], hp["d"])) for _ in range(hp["n_layer"])]
    vc = [np.zeros((hp["max_pos"], hp["d"])) for _ in range(hp["n_layer"])]

    def ln_out(z):
        z = z.astype(np.float64)
        return (z - z.mean()) / np.sqrt(z.var() + 1e-5) * t["lm.out_norm.weight"] + t["lm.out_norm.bias"]

    got = m.run(x)
    xr = _ref_forward(hp, t, x.astype(np.float64), 0, kc, vc, m.freqs)
    want = ln_out(xr[-1])
    assert np.sqrt(((got - want) ** 2).mean() / (want ** 2).mean()) < 0.03
    pos = 20
    for f in range(6):
        out, eos = m.step(lat[f])
        xin = t["lm.input.weight"].reshape(hp["d"], hp["ldim"]).astype(np.float64) @ lat[f]
        xr = _ref_forward(hp, t, xin[None], pos, kc, vc, m.freqs)
        want = ln_out(xr[0])
        assert np.sqrt(((out - want) ** 2).mean() / (want ** 2).mean()) < 0.03, f
        we = float(want @ t["lm.eos.weight"] + t["lm.eos.bias"][0])
        assert abs(eos - we) < 0.05 * (1 + abs(we)), (f, eos, we)
        pos += 1
    assert m.pos == 26
    with pytest.raises(ValueError):
        m.run(np.zeros((hp["max_pos"], hp["d"]), np.float32))


def _f64_flow(hp, fhp, t, c, x0):
    """The flow head (pockettts/lm.go:59-160) in float64 from the dequantized
    weights: the structure the oracle must follow, to float32 rounding."""
    from gorelaxor_amd.synth import q8_dequant

    D, d, ld = fhp["dim"], hp["d"], hp["ldim"]

    def W(name, rows, cols):
        w = t[name + ".weight"]
        m = q8_dequant(w, rows, cols) if w.dtype == np.uint8 else w.reshape(rows, cols)
        return m.astype(np.float64), t[name + ".bias"].astype(np.float64)

    def lin(name, x, rows, cols):
        w, b = W(name, rows, cols)
        return w @ x + b

    silu = lambda v: v / (1 + np.exp(-v))  # noqa: E731

    def ln(h, w=None, b=None):
        o = (h - h.mean()) / np.sqrt(h.var() + 1e-6)
        return o * w + b if w is not None else o

    def embed(e, tt):
        p = f"flow.time.{e}."
        f = t[p + "freqs"].astype(np.float64)
        x = np.concatenate([np.cos(tt * f), np.sin(tt * f)])
        y = lin(p + "fc2", silu(lin(p + "fc1", x, D, 256)), D, D)
        return y * t[p + "norm.alpha"] / np.sqrt(y.var(ddof=1) + 1e-5)

    steps = fhp["steps"]
    tc = [(embed(0, i / steps) + embed(1, (i + 1) / steps)) / 2 for i in range(steps)]
    y = lin("flow.cond", c.astype(np.float64), D, d)
    cur = x0.astype(np.float64)
    for tcs in tc:
        sy = silu(y + tcs)
        h = lin("flow.input", cur, D, ld)
        for i in range(fhp["depth"]):
            p = f"flow.res.{i}."
            mod = lin(p + "ada", sy, 3 * D, D)
            n = ln(h, t[p + "norm.weight"], t[p + "norm.bias"]) * (1 + mod[D:2 * D]) + mod[:D]
            h = h + mod[2 * D:] * lin(p + "fc2", silu(lin(p + "fc1", n, D, D)), D, D)
        mod = lin("flow.final.ada", sy, 2 * D, D)
        n = ln(h) * (1 + mod[D:]) + mod[:D]
        cur = cur + lin("flow.final.out", n, ld, D) / steps
    return cur


@pytest.mark.parametrize("q8", [True, False])
def test_flow_head_structure_vs_float64(orc, q8):
    """The oracle's flow head against the float64 restatement of lm.go's
    SimpleMLPAdaLN (time conditions, adaLN shift/scale/gate, the residual
    MLPs, the final modulation, the LSD update): equal to float32 rounding,
    with the Q8_0/float32 typing of converted files and with all-float32."""
    from gorelaxor_amd.synth import POCKET_FLOW_TINY, POCKET_TTS_TINY, pocket_flow_model

    hp, fhp = dict(POCKET_TTS_TINY), dict(POCKET_FLOW_TINY)
    t = pocket_flow_model(hp, fhp, seed=3, q8=q8)
    o = orc.PocketFlowOracle(hp, fhp["dim"], fhp["depth"], fhp["steps"], t)
    rng = np.random.default_rng(4)
    for _ in range(3):
        c = rng.standard_normal(hp["d"]).astype(np.float32)
        x0 = rng.standard_normal(hp["ldim"]).astype(np.float32)
        got = o.sample(c, x0)
        want = _f64_flow(hp, fhp, t, c, x0)
        assert np.allclose(got, want, rtol=2e-4, atol=2e-4), np.abs(got - want).max()


def _same(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def test_oracle_seeded_state_continues_its_run(orc):
    """tstate.clone (nn.go:128-140): a fresh oracle seeded with the state a
    run left (its caches' rows and position) runs on to the same bits as the
    run that made it, for a text prefix and for frames; seeding a state of
    other values gives other outputs (the seeded rows are what attend
    reads)."""
    hp = dict(POCKET_TTS_TINY)
    t = pocket_model(hp, seed=3)
    x, lat = pocket_inputs(hp, 5, prefix=9, seed=4)
    a = orc.PocketOracle(hp, t)
    a.run(x[:6])
    k, v = a.state()
    assert k.shape == (hp["n_layer"], 6, hp["d"])
    want = a.run(x[6:])
    wf = [a.step(lat[j]) for j in range(5)]
    b = orc.PocketOracle(hp, t)
    b.set_state(k, v)
    assert b.pos == 6
    assert _same(b.run(x[6:]), want)
    for j in range(5):
        o, e = b.step(lat[j])
        assert _same(o, wf[j][0]) and _same(e, wf[j][1])
    c = orc.PocketOracle(hp, t)
    c.set_state(k * np.float32(0.5), v)
    assert not _same(c.run(x[6:]), want)
