"""Pins the oracle's whisper decoder graph bit for bit, without a GPU.

whisper/decoder.go:33-140 (Model.decode) and whisper/encoder.go:120-143 (the
cross keys and values) are composed here in Python, line by line from the
reference, out of the oracle's primitives - each pinned on its own
(test_oracle_kern.py: the int8 product, the dot-product orders, GELU,
expf/EXP8) or restated here from the reference (layerNorm, mathx.go:55-75;
softmax with expSub's eight lane sums, mathx.go:78-90,
kernels_amd64.go:107-117) and checked against the oracle's own.  The
oracle's C graph must give the composition's logits bit for bit at every
step: its wiring (which norm feeds which product, where biases go, which
dot-product order and softmax each attention uses) is then the reference's.
Planted mistakes in the composition - an erf GELU, LayerNorm eps 1e-6, the
float64 LayerNorm form, expf for EXP8 in one softmax, a bias on the cross
keys - must each break the bit-equality, which shows the pin sees them."""
import math

import numpy as np
import pytest

from gorelaxor_amd.synth import WHISPER_TINY_TEST, encoder_output, whisper_model

F32 = np.float32


def _bits(a):
    return np.asarray(a, F32).view(np.uint32)


def ln_kern(x, w, b, eps=1e-5):
    """layerNorm (whisper/mathx.go:55-75): float64 sums left to right (a
    cumulative sum is sequential), mean and inv rounded to float32, then
    ((v - mean) * inv) * w + b in float32."""
    x = np.asarray(x, F32)
    n = x.size
    mean = F32(np.cumsum(x.astype(np.float64))[-1] / n)
    d = (x - mean).astype(np.float64)
    inv = F32(1.0 / math.sqrt(np.cumsum(d * d)[-1] / n + eps))
    return ((x - mean) * inv) * np.asarray(w, F32) + np.asarray(b, F32)


def softmax_py(orc, x, exp8=True):
    """softmax (whisper/mathx.go:78-90) with expSub (kernels_amd64.go:
    107-117): EXP8 below n &^ 7 with eight lane sums added by HSUM, expf
    (expSubGo) past it with its own sum, then x * (1 / s)."""
    x = np.asarray(x, F32)
    n = x.size
    mx = F32(x.max())
    n8 = n & ~7
    e = np.array([(orc.exp8 if (i < n8 and exp8) else orc.expf)(float(F32(x[i] - mx))) for i in range(n)], F32)
    if n8 > 0:
        lanes = [np.cumsum(e[l:n8:8], dtype=F32)[-1] for l in range(8)]
        h = [F32(lanes[l] + lanes[l + 4]) for l in range(4)]
        sa = F32(F32(h[0] + h[1]) + F32(h[2] + h[3]))
    else:
        sa = F32(0)
    tail = np.cumsum(e[n8:], dtype=F32)[-1] if n > n8 else F32(0)
    inv = F32(1) / F32(sa + tail)
    return e * inv


def gelu_erf(x):
    x = np.asarray(x, np.float64)
    return (0.5 * x * (1 + np.vectorize(math.erf)(x / math.sqrt(2)))).astype(F32)


class Composed:
    """decoder.go:33-140 over the oracle's primitives; `plant` names one
    mistake to put in (None: the reference's graph)."""

    def __init__(self, orc, hp, t, enc, plant=None):
        self.orc, self.hp, self.t, self.plant = orc, hp, t, plant
        st, nh = hp["n_state"], hp["n_head"]
        hd = st // nh
        self.sc = F32(1 / math.sqrt(hd))
        nctx = hp["n_audio_ctx"]
        enc = np.asarray(enc, F32).reshape(nctx, st)
        self.ck, self.cv, self.kc, self.vc = [], [], [], []
        for i in range(hp["n_layer"]):
            p = f"decoder.blocks.{i}."
            # encoder.go:120-143: K = enc . Wk^T scaled, V = enc . Wv^T + b
            k = orc.matmul_q8_int(enc, t[p + "cross_attn.key.weight"], st, st)
            if plant == "cross_key_bias":
                k = k + t[p + "cross_attn.value.bias"]
            k = k * self.sc
            v = orc.matmul_q8_int(enc, t[p + "cross_attn.value.weight"], st, st, bias=t[p + "cross_attn.value.bias"])
            self.ck.append(k.reshape(nctx, nh, hd).transpose(1, 0, 2).copy())   # [h][t][d]
            self.cv.append(v.reshape(nctx, nh, hd).transpose(1, 2, 0).copy())   # [h][d][t]
            self.kc.append([])
            self.vc.append([])

    def ln(self, x, w, b, which=""):
        if self.plant == "ln_eps":
            return ln_kern(x, w, b, eps=1e-6)
        if self.plant == "ln_form" and which == "mlp":
            return self.orc.layernorm_f64(x, w, b)
        return ln_kern(x, w, b)

    def mm(self, x, name, n, k, bias=None):
        return self.orc.matmul_q8_int(np.asarray(x, F32)[None, :], self.t[name], n, k,
                                      bias=None if bias is None else self.t[bias])[0]

    def step(self, tok):
        orc, hp, t, st = self.orc, self.hp, self.t, self.hp["n_state"]
        nh = hp["n_head"]
        hd = st // nh
        pos = len(self.kc[0])
        nb = st // 32
        emb = t["decoder.token_embedding.weight"].reshape(hp["n_vocab"], nb * 34)
        # decoder.go:42-46: widen(tokEmb.row(t)) + decPos[pos]
        x = orc.dequant_q8(emb[tok], st) + t["decoder.positional_embedding"].reshape(-1, st)[pos]
        for li in range(hp["n_layer"]):
            p = f"decoder.blocks.{li}."
            cur = self.ln(x, t[p + "attn_ln.weight"], t[p + "attn_ln.bias"])
            q = self.mm(cur, p + "attn.query.weight", st, st, p + "attn.query.bias")
            self.kc[li].append(self.mm(cur, p + "attn.key.weight", st, st))
            self.vc[li].append(self.mm(cur, p + "attn.value.weight", st, st, p + "attn.value.bias"))
            att = np.zeros(st, F32)
            n = pos + 1
            for h in range(nh):
                qi = q[h * hd:(h + 1) * hd]
                s = np.array([F32(orc.dot_f32_go(qi, self.kc[li][j][h * hd:(h + 1) * hd])) * self.sc
                              for j in range(n)], F32)
                s = orc.softmax(s)
                out = np.zeros(hd, F32)
                for j in range(n):
                    out = out + s[j] * self.vc[li][j][h * hd:(h + 1) * hd]
                att[h * hd:(h + 1) * hd] = out
            x = x + self.mm(att, p + "attn.out.weight", st, st, p + "attn.out.bias")
            # cross-attention (decoder.go:92-121)
            cur = self.ln(x, t[p + "cross_attn_ln.weight"], t[p + "cross_attn_ln.bias"])
            q = self.mm(cur, p + "cross_attn.query.weight", st, st, p + "cross_attn.query.bias")
            nctx = hp["n_audio_ctx"]
            for h in range(nh):
                qi, kd, vd = q[h * hd:(h + 1) * hd], self.ck[li][h], self.cv[li][h]
                s = np.zeros(nctx, F32)
                j = 0
                while j + 4 <= nctx:
                    s[j:j + 4] = orc.dot_f32_x4(qi, kd[j:j + 4].ravel(), hd, hd)
                    j += 4
                for j in range(j, nctx):
                    s[j] = orc.dot_f32_go(qi, kd[j])
                s = softmax_py(orc, s, exp8=False) if (self.plant == "expf_softmax" and li == 0) else orc.softmax(s)
                out = np.zeros(hd, F32)
                d = 0
                while d + 4 <= hd:
                    out[d:d + 4] = orc.dot_f32_x4(s, vd[d:d + 4].ravel(), nctx, nctx)
                    d += 4
                for d in range(d, hd):
                    out[d] = orc.dot_f32_go(s, vd[d])
                att[h * hd:(h + 1) * hd] = out
            x = x + self.mm(att, p + "cross_attn.out.weight", st, st, p + "cross_attn.out.bias")
            # feed-forward (decoder.go:124-128): parGelu = geluVec on 1<<14 chunks
            cur = self.ln(x, t[p + "mlp_ln.weight"], t[p + "mlp_ln.bias"], which="mlp")
            ff = self.mm(cur, p + "mlp.0.weight", 4 * st, st, p + "mlp.0.bias")
            ff = gelu_erf(ff) if self.plant == "erf_gelu" else orc.gelu(ff)
            x = x + self.mm(ff, p + "mlp.2.weight", st, 4 * st, p + "mlp.2.bias")
        # decoder.go:131-138: layerNorm, then the tied logits product
        row = self.ln(x, t["decoder.ln.weight"], t["decoder.ln.bias"])
        return self.mm(row, "decoder.token_embedding.weight", hp["n_vocab"], st)


@pytest.fixture(scope="module")
def model(orc):
    hp = dict(WHISPER_TINY_TEST, n_audio_ctx=37)  # 37 keys: a dotF32Go tail past the groups of four
    return hp, whisper_model(hp, seed=11), encoder_output(hp, seed=12)


def test_restated_primitives_equal_the_oracles(orc):
    """The composition's own restatements agree with the oracle's C forms
    bit for bit: layerNorm (kern form) and softmax (EXP8 lanes + expf tail)."""
    rng = np.random.default_rng(5)
    for n in (3, 8, 37, 128, 200):
        x = (rng.standard_normal(n) * 2).astype(F32)
        w, b = rng.standard_normal(n).astype(F32), rng.standard_normal(n).astype(F32)
        assert np.array_equal(_bits(ln_kern(x, w, b)), _bits(orc.layernorm(x, w, b))), n
        assert np.array_equal(_bits(softmax_py(orc, x)), _bits(orc.softmax(x))), n


def test_oracle_graph_is_the_composition(orc, model):
    """The C oracle's logits equal the composition's at every step: the
    4-token prompt one token at a time, then greedy steps."""
    hp, t, enc = model
    ref = orc.WhisperOracle(hp, t)
    ref.set_encoder_output(enc)
    comp = Composed(orc, hp, t, enc)
    toks = [5, 17, 3, 999]
    for k in range(8):
        want = ref.decode([toks[k]])
        got = comp.step(toks[k])
        assert np.array_equal(_bits(got), _bits(want)), k
        if k >= 3:
            toks.append(orc.argmax(want))


@pytest.mark.parametrize("plant", ["erf_gelu", "ln_eps", "ln_form", "expf_softmax", "cross_key_bias"])
def test_planted_mistakes_break_the_pin(orc, model, plant):
    """Each planted mistake changes the logits' bits within the prompt."""
    hp, t, enc = model
    ref = orc.WhisperOracle(hp, t)
    ref.set_encoder_output(enc)
    comp = Composed(orc, hp, t, enc, plant=plant)
    differs = False
    for tok in (5, 17, 3, 999):
        differs |= not np.array_equal(_bits(comp.step(tok)), _bits(ref.decode([tok])))
    assert differs, plant
