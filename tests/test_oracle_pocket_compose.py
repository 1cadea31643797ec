"""Pins the oracle's pocket-TTS flow-LM graph bit for bit, without a GPU.

pockettts/nn.go:142-254 (transformer.forward and attend) and
pockettts/lm.go:164-195 (flowLM.run and step) are composed here in Python,
line by line from the reference, out of the oracle's primitives - the int8
product, MatMulF32, ExpSub, AddScaled and GELU, each pinned on its own in
test_oracle_kern.py - and two restatements checked here against the
oracle's C forms (the float64 layerNorm, nn.go:27-49; ropeFreqs and
applyRope, nn.go:67-93).  The oracle's C graph must give the composition's
outputs and end-of-speech logits bit for bit over a text prefix (T = 5, the
transposed-values product) and single steps (T = 1, the AddScaled sums).
Planted mistakes - RoPE one position late, RoPE on the values too, the
float32-mean LayerNorm, an erf GELU, AddScaled sums for T >= 4 - must each
break the equality."""
import math

import numpy as np
import pytest

from gorelaxor_amd.synth import POCKET_TTS_TINY, pocket_inputs, pocket_model

F32 = np.float32


def _bits(a):
    return np.asarray(a, F32).view(np.uint32)


def ln64(x, w, b, eps=1e-5):
    """layerNorm (pockettts/nn.go:27-49): float64 sums left to right, mean
    and inv in float64, each value rounded to float32 before w and b."""
    x = np.asarray(x, F32)
    n = x.size
    mean = np.cumsum(x.astype(np.float64))[-1] / n
    d = x.astype(np.float64) - mean
    inv = 1 / math.sqrt(np.cumsum(d * d)[-1] / n + eps)
    return (d * inv).astype(F32) * np.asarray(w, F32) + np.asarray(b, F32)


def rope_freqs(hd, period):
    """ropeFreqs (nn.go:67-76)."""
    c = F32(-math.log(period) * 2 / hd)
    return np.array([F32(math.exp(float(F32(F32(i) * c)))) for i in range(hd // 2)], F32)


def apply_rope(x, heads, freqs, pos):
    """applyRope (nn.go:80-93): the angle f64(f_i * f32(pos)), cos and sin
    rounded to float32, products and sums unfused in float32."""
    x = np.asarray(x, F32).copy()
    hd = freqs.size * 2
    p = F32(pos)
    for i, f in enumerate(freqs):
        a = float(F32(f * p))
        c, s = F32(math.cos(a)), F32(math.sin(a))
        for h in range(heads):
            j = h * hd + 2 * i
            r, im = x[j], x[j + 1]
            x[j] = F32(r * c) - F32(im * s)
            x[j + 1] = F32(r * s) + F32(im * c)
    return x


def gelu_erf(x):
    x = np.asarray(x, np.float64)
    return (0.5 * x * (1 + np.vectorize(math.erf)(x / math.sqrt(2)))).astype(F32)


class Composed:
    """transformer.forward / flowLM.run / flowLM.step over the oracle's
    primitives; `plant` names one mistake to put in."""

    def __init__(self, orc, hp, t, plant=None):
        self.orc, self.hp, self.t, self.plant = orc, hp, t, plant
        d = hp["d"]
        self.freqs = rope_freqs(d // hp["heads"], hp["period"])
        self.k = [np.zeros((0, d), F32) for _ in range(hp["n_layer"])]
        self.v = [np.zeros((0, d), F32) for _ in range(hp["n_layer"])]
        self.pos = 0

    def ln(self, x, w, b):
        if self.plant == "ln_f32_mean":
            return self.orc.layernorm(x, w, b)
        return ln64(x, w, b)

    def attend(self, qkv, T, li, pos0):
        """attend (nn.go:200-254) with no context limit."""
        orc, d, heads = self.orc, self.hp["d"], self.hp["heads"]
        hd = d // heads
        scale = F32(1 / math.sqrt(hd))
        nk = pos0 + T
        out = np.zeros((T, d), F32)
        for h in range(heads):
            q = np.ascontiguousarray(qkv[:, h * hd:(h + 1) * hd])
            kk = np.ascontiguousarray(self.k[li][:nk, h * hd:(h + 1) * hd])
            vv = np.ascontiguousarray(self.v[li][:nk, h * hd:(h + 1) * hd])
            sc = orc.matmul_f32(q, kk)
            for r in range(T):
                p = pos0 + r
                s = sc[r, :p + 1] * scale
                e, tot = orc.expsub(s, float(s.max()))
                sc[r, :p + 1] = e * (F32(1) / F32(tot))
                sc[r, p + 1:] = 0
            if T < 4 or self.plant == "addscaled_always":
                for r in range(T):
                    o = np.zeros(hd, F32)
                    for j in range(nk):
                        if sc[r, j] != 0:
                            o = orc.axpy(o, vv[j], float(sc[r, j]))
                    out[r, h * hd:(h + 1) * hd] = o
            else:
                out[:, h * hd:(h + 1) * hd] = orc.matmul_f32(sc, np.ascontiguousarray(vv.T))
        return out

    def forward(self, x):
        orc, hp, t = self.orc, self.hp, self.t
        d, ff, heads = hp["d"], hp["ff"], hp["heads"]
        x = np.asarray(x, F32).reshape(-1, d).copy()
        T = x.shape[0]
        rp = 1 if self.plant == "rope_late" else 0
        for li in range(hp["n_layer"]):
            p = f"lm.blk.{li}."
            h = np.stack([self.ln(x[r], t[p + "norm1.weight"], t[p + "norm1.bias"]) for r in range(T)])
            qkv = orc.matmul_q8_int(h, t[p + "attn_qkv.weight"], 3 * d, d)
            for r in range(T):
                qkv[r, :d] = apply_rope(qkv[r, :d], heads, self.freqs, self.pos + r + rp)
                qkv[r, d:2 * d] = apply_rope(qkv[r, d:2 * d], heads, self.freqs, self.pos + r + rp)
                if self.plant == "rope_values":
                    qkv[r, 2 * d:] = apply_rope(qkv[r, 2 * d:], heads, self.freqs, self.pos + r)
            self.k[li] = np.concatenate([self.k[li], qkv[:, d:2 * d]])
            self.v[li] = np.concatenate([self.v[li], qkv[:, 2 * d:]])
            att = self.attend(qkv, T, li, self.pos)
            x = x + orc.matmul_q8_int(att, t[p + "attn_out.weight"], d, d)
            h = np.stack([self.ln(x[r], t[p + "norm2.weight"], t[p + "norm2.bias"]) for r in range(T)])
            f = orc.matmul_q8_int(h, t[p + "ff1.weight"], ff, d)
            f = gelu_erf(f) if self.plant == "erf_gelu" else orc.gelu(f)
            x = x + orc.matmul_q8_int(f, t[p + "ff2.weight"], d, ff)
        self.pos += T
        return x

    def run(self, x):
        x = self.forward(x)
        return self.ln(x[-1], self.t["lm.out_norm.weight"], self.t["lm.out_norm.bias"])

    def step(self, latent=None):
        t, d, ld = self.t, self.hp["d"], self.hp["ldim"]
        lat = t["lm.bos"] if latent is None else np.asarray(latent, F32)
        x = self.orc.matmul_f32(lat[None, :], t["lm.input.weight"].reshape(d, ld))
        out = self.run(x)
        e = self.orc.matmul_f32(out[None, :], t["lm.eos.weight"][None, :])[0, 0]
        return out, F32(e + t["lm.eos.bias"][0])


@pytest.fixture(scope="module")
def model():
    hp = POCKET_TTS_TINY
    t = pocket_model(hp, seed=21)
    x, lat = pocket_inputs(hp, frames=3, prefix=5, seed=22)
    return hp, t, x, lat


def test_restated_primitives_equal_the_oracles(orc):
    rng = np.random.default_rng(8)
    for n in (5, 64, 128, 300):
        x = (rng.standard_normal(n) * 3 + 0.5).astype(F32)
        w, b = rng.standard_normal(n).astype(F32), rng.standard_normal(n).astype(F32)
        assert np.array_equal(_bits(ln64(x, w, b)), _bits(orc.layernorm_f64(x, w, b))), n
    for hd, period in ((64, 1e4), (32, 1e4), (64, 500.0)):
        f = rope_freqs(hd, period)
        assert np.array_equal(_bits(f), _bits(orc.rope_freqs(hd, period)))
        x = rng.standard_normal(2 * hd).astype(F32)
        for pos in (0, 1, 7, 95, 4000):
            assert np.array_equal(_bits(apply_rope(x, 2, f, pos)), _bits(orc.apply_rope(x, 2, f, pos))), pos


def _steps(m, x, lat):
    """The text prefix, the bos step, then the latents' steps."""
    out = [m.run(x)]
    for l in [None] + list(lat):
        o, e = m.step(l)
        out += [o, np.array([e], F32)]
    return out


def test_oracle_graph_is_the_composition(orc, model):
    hp, t, x, lat = model
    want = _steps(orc.PocketOracle(hp, t), x, lat)
    got = _steps(Composed(orc, hp, t), x, lat)
    for k, (g, w) in enumerate(zip(got, want)):
        assert np.array_equal(_bits(g), _bits(w)), k


@pytest.mark.parametrize("plant", ["rope_late", "rope_values", "ln_f32_mean", "erf_gelu", "addscaled_always"])
def test_planted_mistakes_break_the_pin(orc, model, plant):
    hp, t, x, lat = model
    want = _steps(orc.PocketOracle(hp, t), x, lat)
    got = _steps(Composed(orc, hp, t, plant=plant), x, lat)
    assert any(not np.array_equal(_bits(g), _bits(w)) for g, w in zip(got, want)), plant
