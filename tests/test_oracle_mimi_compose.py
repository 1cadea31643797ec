"""Pins the oracle's Mimi decoder bit for bit, without a GPU.

pockettts/mimi.go:122-152 (mimiDecoder.decode: the latent projection, the
depthwise transposed upsampling with its carried overlap, the transformer,
SEANet) with nn.go:142-254 (transformer.forward with the context limit and
layer scales, attend, addScaled), mimi.go:62-108 (runSea), nn.go:272-296
(conv.run: im2col rows and one Linear, past rows carried) and nn.go:308-327
(convtr.run: Linear, overlap-add from the bias, partial carried) are
composed here in Python, line by line from the reference, out of the
oracle's primitives - each pinned on its own (test_oracle_kern.py: the int8
product, kern's float32 product routes, axpy, GELU, ExpSub;
test_oracle_pocket*.py: the float64 LayerNorm, RoPE; test_oracle_mimi.py:
ELU) - and the oracle's streamed decode must give the composition's
samples bit for bit, one latent a call and several a call.  Its wiring
(every carry, the context window, the layer scales, RoPE's positions, the
residual blocks' ELUs and skips) is then the reference's.  Planted mistakes
in the composition must each break the bit-equality, which shows the pin
sees them."""
import math

import numpy as np
import pytest

from gorelaxor_amd.synth import MIMI_TINY, mimi_latents, mimi_model, mimi_steps

F32 = np.float32


def _bits(a):
    return np.asarray(a, F32).view(np.uint32)


class Composed:
    """decode over the oracle's primitives with its own streaming state;
    `plant` names one mistake to put in (None: the reference's decoder)."""

    def __init__(self, orc, hp, t, plant=None):
        self.orc, self.hp, self.t, self.plant = orc, hp, t, plant
        d = hp["d"]
        self.hd = d // hp["heads"]
        self.freqs = orc.rope_freqs(self.hd, float(hp["period"]))
        self.kc = [np.zeros((0, d), F32) for _ in range(hp["n_layer"])]
        self.vc = [np.zeros((0, d), F32) for _ in range(hp["n_layer"])]
        self.pos = 0
        self.up_part = np.zeros((hp["up_s"], d), F32)
        self.steps = mimi_steps(hp)
        # newSeaState (mimi.go:44-60): a conv's past rows, a transposed
        # conv's partial rows, a residual block's two convs' past rows
        self.prev = {}
        for kind, name, el, cin, cout, k, stride, dil in self.steps:
            if kind == "conv":
                self.prev[name] = np.zeros(((k - 1) * dil + 1 - stride, cin), F32)
            elif kind == "convtr":
                self.prev[name] = np.zeros((k - stride, cout), F32)
            else:
                self.prev[name + ".1"] = np.zeros(((k - 1) * dil, cin), F32)
                self.prev[name + ".3"] = np.zeros((0, cout), F32)

    def lin(self, x, name, n, k, bias=None):
        """kern.Linear by the weight's type: the int8 route for Q8_0, the
        float route for float32 (pockettts/model.go:331-366)."""
        w = self.t[name]
        x = np.ascontiguousarray(x, F32).reshape(-1, k)
        if w.dtype == np.uint8:
            return self.orc.matmul_q8_int(x, w, n, k, bias=bias)
        return self.orc.matmul_f32(x, np.asarray(w, F32).reshape(n, k), bias=bias)

    def conv(self, key, name, x, cin, cout, k, stride, dil, bias):
        """conv.run (nn.go:272-296)."""
        T = x.shape[0]
        if k == 1 and stride == 1:
            return self.lin(x, name, cout, k * cin, bias)
        buf = np.concatenate([self.prev[key], x])
        To = T // stride
        col = np.stack([np.concatenate([buf[r * stride + j * dil] for j in range(k)]) for r in range(To)])
        y = self.lin(col, name, cout, k * cin, bias)
        if self.plant != "conv_no_past":
            self.prev[key] = buf[T:].copy()
        return y

    def convtr(self, key, name, x, cin, cout, k, stride, bias):
        """convtr.run (nn.go:308-327)."""
        T = x.shape[0]
        z = self.lin(x, name, k * cout, cin).reshape(T, k, cout)
        L = (T - 1) * stride + k
        full = np.tile(np.asarray(bias, F32), (L, 1))
        for r in range(T):
            for j in range(k):
                full[r * stride + j] = full[r * stride + j] + z[r, j]
        pt = k - stride
        if self.plant != "convtr_no_partial":
            full[:pt] = full[:pt] + self.prev[key]
        self.prev[key] = full[L - pt:] - np.asarray(bias, F32)
        return full[:T * stride]

    def attend(self, qkv, T, li):
        """attend (nn.go:200-254) with the context limit: query p sees keys
        max(lo0, p - context + 1) .. p."""
        orc, hp = self.orc, self.hp
        d, hd, ctx = hp["d"], self.hd, hp["context"]
        if self.plant == "context_long":
            ctx += 1
        scale = F32(1.0 / math.sqrt(hd))
        pos0 = self.pos
        lo0 = max(0, pos0 - ctx + 1) if ctx > 0 else 0
        nk = pos0 + T - lo0
        out = np.zeros((T, d), F32)
        for h in range(hp["heads"]):
            sl = slice(h * hd, (h + 1) * hd)
            kh = np.ascontiguousarray(self.kc[li][lo0:lo0 + nk, sl])
            vh = self.vc[li][lo0:lo0 + nk, sl]
            sc = orc.matmul_f32(np.ascontiguousarray(qkv[:, sl]), kh)
            for r in range(T):
                p = pos0 + r
                lo = max(lo0, p - ctx + 1) if ctx > 0 else lo0
                ns = p + 1 - lo
                s = sc[r, lo - lo0:lo - lo0 + ns] * scale
                e, tot = orc.expsub(s, float(s.max()))
                row = np.zeros(nk, F32)
                row[lo - lo0:lo - lo0 + ns] = e * (F32(1) / F32(tot))
                sc[r] = row
            if T < 4:
                for r in range(T):
                    o = np.zeros(hd, F32)
                    for j in range(nk):
                        if sc[r, j] != 0:
                            o = orc.axpy(o, vh[j], float(sc[r, j]))
                    out[r, sl] = o
            else:
                out[:, sl] = orc.matmul_f32(sc, np.ascontiguousarray(vh.T))
        return out

    def add_scaled(self, x, y, name):
        """addScaled (nn.go:185-196): x + s * y, or x + y without s."""
        s = self.t.get(name)
        if s is None or self.plant == "no_layer_scale":
            return x + y
        return x + np.asarray(s, F32) * y

    def forward(self, x):
        """transformer.forward (nn.go:142-182)."""
        orc, hp, t = self.orc, self.hp, self.t
        T, d, ff = x.shape[0], hp["d"], hp["ff"]
        for li in range(hp["n_layer"]):
            p = f"mimi.dec_tf.{li}."
            h = orc.layernorm_f64(x, t[p + "norm1.weight"], t[p + "norm1.bias"])
            qkv = self.lin(h, p + "attn_qkv.weight", 3 * d, d)
            for r in range(T):
                at = self.pos + r + (1 if self.plant == "rope_late" else 0)
                qkv[r, :d] = orc.apply_rope(qkv[r, :d], hp["heads"], self.freqs, at)
                qkv[r, d:2 * d] = orc.apply_rope(qkv[r, d:2 * d], hp["heads"], self.freqs, at)
            self.kc[li] = np.concatenate([self.kc[li], qkv[:, d:2 * d]])
            self.vc[li] = np.concatenate([self.vc[li], qkv[:, 2 * d:]])
            att = self.attend(qkv, T, li)
            x = self.add_scaled(x, self.lin(att, p + "attn_out.weight", d, d), p + "ls1")
            h = orc.layernorm_f64(x, t[p + "norm2.weight"], t[p + "norm2.bias"])
            f = orc.gelu(self.lin(h, p + "ff1.weight", ff, d).ravel()).reshape(T, ff)
            x = self.add_scaled(x, self.lin(f, p + "ff2.weight", d, ff), p + "ls2")
        self.pos += T
        return x

    def sea(self, x):
        """runSea (mimi.go:62-108): each step after an ELU where it has one."""
        orc, t = self.orc, self.t
        cur = x
        for kind, name, el, cin, cout, k, stride, dil in self.steps:
            if el:
                cur = orc.elu(cur)
            if kind == "conv":
                cur = self.conv(name, name + ".weight", cur, cin, cout, k, stride, dil, t[name + ".bias"])
            elif kind == "convtr":
                cur = self.convtr(name, name + ".weight", cur, cin, cout, k, stride, t[name + ".bias"])
            else:
                v = cur if self.plant == "res_no_elu" else orc.elu(cur)
                hmid = orc.elu(self.conv(name + ".1", name + ".1.weight", v, cin, cout, k, 1, dil,
                                         t[name + ".1.bias"]))
                o = self.conv(name + ".3", name + ".3.weight", hmid, cout, cin, 1, 1, 1, t[name + ".3.bias"])
                cur = (v if self.plant == "res_skip_elu" else cur) + o
        return cur

    def decode(self, lat):
        """mimiDecoder.decode (mimi.go:122-152)."""
        hp, t = self.hp, self.t
        d, S = hp["d"], hp["up_s"]
        K = 2 * S
        n = lat.shape[0]
        z = self.lin(lat, "mimi.quant", d, hp["ldim"])
        w = np.asarray(t["mimi.up"], F32).reshape(d, K)
        L = (n - 1) * S + K
        full = np.zeros((L, d), F32)
        for r in range(n):
            for j in range(K):
                full[r * S + j] = full[r * S + j] + z[r] * w[:, j]
        if self.plant != "up_no_overlap":
            full[:S] = full[:S] + self.up_part
        self.up_part = full[L - S:].copy()
        x = self.forward(full[:n * S])
        return self.sea(x).ravel()


@pytest.fixture(scope="module", params=[False, True], ids=["float32", "q8"])
def model(request):
    hp = dict(MIMI_TINY)
    return hp, mimi_model(hp, seed=15, q8=request.param)


@pytest.mark.parametrize("per_call", [1, 3])
def test_oracle_decode_is_the_composition(orc, model, per_call):
    """The oracle's streamed samples equal the composition's bit for bit:
    nine latents one a call (past the context window of 12 positions at 4
    rows a latent) and three a call (the attention's several-row route)."""
    hp, t = model
    ref = orc.MimiOracle(hp, t)
    comp = Composed(orc, hp, t)
    lat = mimi_latents(hp, 9, seed=16)
    for i in range(0, 9, per_call):
        want = ref.decode(lat[i:i + per_call])
        got = comp.decode(lat[i:i + per_call])
        assert np.array_equal(_bits(got), _bits(want)), i


@pytest.mark.parametrize("plant", ["conv_no_past", "convtr_no_partial", "up_no_overlap", "context_long",
                                   "no_layer_scale", "rope_late", "res_no_elu", "res_skip_elu"])
def test_planted_mistakes_break_the_pin(orc, model, plant):
    """Each planted mistake changes the samples' bits within six latents."""
    hp, t = model
    ref = orc.MimiOracle(hp, t)
    comp = Composed(orc, hp, t, plant=plant)
    lat = mimi_latents(hp, 6, seed=16)
    differs = False
    for i in range(6):
        differs |= not np.array_equal(_bits(comp.decode(lat[i:i + 1])), _bits(ref.decode(lat[i:i + 1])))
    assert differs, plant
