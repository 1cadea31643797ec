"""Pins the oracle's conformer block bit for bit, without a GPU.

conformer/encoder.go:411-429 (runBlock) with feedForward (:244-251),
attention (:259-330, the key ranges of :193-212) and convModule (:343-397),
and the pre-encoder (subsample, :123-167, with conv0 :41-77 and dwConv2
:80-110) and the whole encode (:432-489) over them, are composed here in
Python, line by line from the reference, out of the
oracle's primitives - each pinned on its own (test_oracle_kern.py: the int8
product, kern's float32 product routes, SiLU, axpy, EXP8/expf and expSub,
layerNorm; test_oracle_conformer.py: the relative position table and the
batch norm fold) - and checked against the oracle's own block (one block
offline, its position projection first: encoder.go:474-486).  Bit-equality
shows the oracle's wiring (which norm feeds which product, the half-step
residuals, the position biases u and v, the relative shift, the score
scale, the key ranges and their blocks, the GLU halves and its masked
rows, the depthwise taps and padding, the folded batch norm or the
convolution's LayerNorm; the pre-encoder's padding, masks, ReLUs and
flattening order, the xscale) is the reference's.  Planted mistakes in the
composition must each break the bit-equality, which shows the pin sees
them."""
import math

import numpy as np
import pytest

from gorelaxor_amd.synth import CONFORMER_TINY, conformer_model

F32 = np.float32
QK, Q8_BYTES = 32, 34


def _bits(a):
    return np.asarray(a, F32).view(np.uint32)


def ln_kern(x, w, b, eps=1e-5):
    """layerNorm (internal/kern/mathx.go:55-75) of each row: float64 sums
    left to right, mean and inv rounded to float32, then ((v - mean) * inv)
    * w + b in float32."""
    x = np.asarray(x, F32)
    out = np.empty_like(x)
    for r in range(x.shape[0]):
        v = x[r]
        n = v.size
        mean = F32(np.cumsum(v.astype(np.float64))[-1] / n)
        d = (v - mean).astype(np.float64)
        inv = F32(1.0 / math.sqrt(np.cumsum(d * d)[-1] / n + eps))
        out[r] = ((v - mean) * inv) * np.asarray(w, F32) + np.asarray(b, F32)
    return out


def key_range(hp, T, L, q):
    """keyRange (encoder.go:193-212) cut at the valid length L, with the
    offline key form and query block length (offlineKeys, :196-212):
    chunked limited context for a streaming model with both limits (blocks
    of one chunk), a window for a regular one whose limits are shorter than
    the recording (blocks of 16), else every key (blocks of 32)."""
    al, ar = hp.get("att_left", -1), hp.get("att_right", -1)
    chunked = hp.get("att_style", "regular") == "chunked_limited"
    if chunked and al >= 0 and ar >= 0:
        mode, bl = "chunked", ar + 1
    elif al >= 0 and ar >= 0 and T - 1 > min(al, ar):
        mode, bl = "window", 16
    else:
        mode, bl = "all", 32
    if q is None:
        return bl
    if q >= L:
        return 0, 0
    lo, hi = 0, T
    if mode == "chunked":
        c = q // bl
        lo = max((c - al // bl) * bl, 0)
        hi = min((c + 1) * bl, T)
    elif mode == "window":
        lo, hi = max(q - al, 0), min(q + ar + 1, T)
    return lo, min(hi, L)


class Composed:
    """runBlock over the oracle's primitives; `plant` names one mistake to
    put in (None: the reference's block)."""

    def __init__(self, orc, hp, t, plant=None):
        self.orc, self.hp, self.t, self.plant = orc, hp, t, plant

    def w(self, name, rows, cols):
        """A product's weight as the encoder binds it: Q8_0 bytes, or a
        float16 pointwise weight through Weight.ToQ8 (model.go:397-402)."""
        w = self.t[name]
        if w.nbytes == rows * cols // QK * Q8_BYTES:
            return w
        return self.orc.quant_q8(np.frombuffer(np.ascontiguousarray(w).tobytes(), np.float16).astype(F32))

    def linear(self, x, name, n, k, bias=None):
        b = self.t.get(bias) if bias else None
        return self.orc.matmul_q8_int(x, self.w(name, n, k), n, k, bias=b)

    def ln(self, x, name):
        w, b = self.t[name + ".weight"], self.t[name + ".bias"]
        if self.plant == "ln_eps":
            return ln_kern(x, w, b, eps=1e-6)
        return self.orc.layernorm(x, w, b)

    def feed_forward(self, x, p, f):
        """feedForward (encoder.go:244-251): x += 0.5 * linear2(SiLU(linear1(LN(x))))."""
        orc, hp = self.orc, self.hp
        d, dff = hp["d"], hp["dff"]
        h = self.linear(self.ln(x, p + "norm_" + f), p + f + ".linear1.weight", dff, d, p + f + ".linear1.bias")
        h = orc.silu(h.ravel()).reshape(h.shape)
        y = self.linear(h, p + f + ".linear2.weight", d, dff, p + f + ".linear2.bias")
        s = 1.0 if self.plant == "ff_full_step" else 0.5
        return orc.axpy(x.ravel(), y.ravel(), s).reshape(x.shape)

    def attention(self, x, ln, p, L, kv, keyf, bl, pp):
        """attention (encoder.go:259-330): queries the T rows ln, keys and
        values from the Tk rows kv (the queries' own rows last: query i is
        key Tk - T + i), keyf(key index of a query) its keys [lo, hi),
        queries in blocks of bl, pp the projected position rows for
        relative positions Tk - 1 down."""
        orc, hp, t = self.orc, self.hp, self.t
        T, D, H = x.shape[0], hp["d"], hp["heads"]
        hd = D // H
        Tk = kv.shape[0]
        qoff = Tk - T
        q = self.linear(ln, p + "attn.linear_q.weight", D, D, p + "attn.linear_q.bias")
        k = self.linear(kv, p + "attn.linear_k.weight", D, D, p + "attn.linear_k.bias")
        v = self.linear(kv, p + "attn.linear_v.weight", D, D, p + "attn.linear_v.bias")
        u, w = t[p + "attn.pos_bias_u"].reshape(D), t[p + "attn.pos_bias_v"].reshape(D)
        if self.plant == "pos_bias_swap":
            u, w = w, u
        qu, qv = q + u, q + w
        scale = F32(1.0 / math.sqrt(D if self.plant == "scale_d" else hd))
        out = np.zeros((T, D), F32)
        for h in range(H):
            sl = slice(h * hd, (h + 1) * hd)
            for q0 in range(0, T, bl):
                q1 = min(T, q0 + bl)
                nq = q1 - q0
                rng = [keyf(qoff + qq) for qq in range(q0, q1)]
                k0, k1 = min(r[0] for r in rng), max(r[1] for r in rng)
                nk = k1 - k0
                if nk <= 0:
                    continue
                # the block's scores and position terms by kern's float32
                # products (MatMulF32), the position rows from jlo on
                npos = nq + nk - 1
                jlo = Tk - 1 - (qoff + q1 - 1) + k0
                sc = orc.matmul_f32(np.ascontiguousarray(qu[q0:q1, sl]), np.ascontiguousarray(k[k0:k1, sl]))
                bd = orc.matmul_f32(np.ascontiguousarray(qv[q0:q1, sl]),
                                    np.ascontiguousarray(pp[jlo:jlo + npos, sl]))
                for i in range(nq):
                    lo, hi = rng[i]
                    sh = nq - 1 - i
                    if self.plant == "rel_shift":
                        sh = nq - i if nq - i + nk <= npos else nq - 2 - i
                    row = np.full(nk, -np.inf, F32)
                    for kk in range(nk):
                        if lo <= k0 + kk < hi:
                            row[kk] = F32(sc[i, kk] + bd[i, sh + kk]) * scale
                    ok = row[np.isfinite(row)]
                    if ok.size == 0:
                        sc[i] = 0
                        continue
                    e, s = orc.expsub(row, float(ok.max()))
                    sc[i] = e * (F32(1) / F32(s))
                vt = np.ascontiguousarray(v[k0:k1, sl].T)
                out[q0:q1, sl] = orc.matmul_f32(np.ascontiguousarray(sc), vt)
        att = self.linear(out, p + "attn.linear_out.weight", D, D, p + "attn.linear_out.bias")
        return x + att

    def conv_module(self, x, ln, p, L, prev=None):
        """convModule (encoder.go:343-397); prev: the padL gated frames
        before the first (a stream's; none offline).  Returns (x, the gated
        frames)."""
        orc, hp, t = self.orc, self.hp, self.t
        T, D, K = x.shape[0], hp["d"], hp["conv_kernel"]
        a = self.linear(ln, p + "conv.pointwise1.weight", 2 * D, D, p + "conv.pointwise1.bias")
        # GLU a * sigmoid(b), rows from the valid length on zero
        g = np.zeros((T, D), F32)
        for r in range(T):
            if r >= L and self.plant != "glu_unmasked":
                continue
            lhs, rhs = (a[r, D:], a[r, :D]) if self.plant == "glu_swap" else (a[r, :D], a[r, D:])
            sg = np.array([F32(1) / (F32(1) + F32(orc.expf(float(-z)))) for z in rhs], F32)
            g[r] = lhs * sg
        # depthwise taps from the bias, padL frames of zeros before
        # (convPadLeft, encoder.go:399-404), unfused w * x sums in tap order
        cl, cr = hp.get("conv_left", -1), hp.get("conv_right", -1)
        padL = cl if cl >= 0 and cr >= 0 else (K - 1) // 2
        dw = np.asarray(t[p + "conv.depthwise.weight"], F32).reshape(D, K)
        b = t.get(p + "conv.depthwise.bias")
        y = np.tile(np.asarray(b, F32) if b is not None else np.zeros(D, F32), (T, 1))
        for r in range(T):
            for j in range(K):
                ti = r + j - padL
                tap = dw[:, K - 1 - j] if self.plant == "dw_reversed" else dw[:, j]
                if 0 <= ti < T:
                    y[r] = y[r] + tap * g[ti]
                elif ti < 0 and prev is not None and padL + ti >= 0:
                    y[r] = y[r] + tap * prev[padL + ti]
        if hp.get("conv_norm", "batch_norm") == "layer_norm":
            y = orc.layernorm(y, t[p + "conv.bn.weight"], t[p + "conv.bn.bias"])
        else:
            s, c = orc.conf_bn_fold(t[p + "conv.bn.weight"], t[p + "conv.bn.bias"], t[p + "conv.bn.running_mean"],
                                    t[p + "conv.bn.running_var"])
            y = y * s + c
        y = orc.silu(y.ravel()).reshape(T, D)
        return x + self.linear(y, p + "conv.pointwise2.weight", D, D, p + "conv.pointwise2.bias"), g

    def subsample(self, mel, valid):
        """subsample (encoder.go:123-167): (out [T][d], T, L)."""
        orc, hp, t = self.orc, self.hp, self.t
        nm, c, d = hp["n_mels"], hp["sub_channels"], hp["d"]
        chunked = hp.get("att_style", "regular") == "chunked_limited"
        causal = bool(hp.get("causal_sub", chunked))
        pl = 2 if causal else 1  # rows and bins of padding before (subOut, encoder.go:33-38)
        if self.plant == "sub_pad":
            pl = 3 - pl
        out_n = (lambda n: n // 2 + 1) if causal else (lambda n: (n - 1) // 2 + 1)
        pe = "enc.pre_encode."
        taps = lambda n: np.ascontiguousarray(np.asarray(t[pe + n], F32).reshape(c, 9).T)  # noqa: E731
        mel = np.asarray(mel, F32)
        frames = mel.shape[1]
        x = np.zeros((frames, nm), F32)
        x[:min(frames, valid)] = mel[:, :min(frames, valid)].T

        def mask(y, L):
            if not (self.plant == "sub_unmasked") and L < y.shape[0]:
                y[max(L, 0):] = 0
            return y

        def relu(y):
            return np.where(y < 0, F32(0), y).astype(F32)

        # conv0 (encoder.go:41-77): each output from the bias, AddScaled of
        # the nine taps in order, taps equal to 0 skipped
        T, F = frames, nm
        T1, F1 = out_n(T), out_n(F)
        w0, b0 = taps("conv.0.weight"), np.asarray(t[pe + "conv.0.bias"], F32)
        y = np.empty((T1, F1, c), F32)
        for r in range(T1):
            for f in range(F1):
                o = b0.copy()
                for kt in range(3):
                    for kf in range(3):
                        ti, fi = 2 * r + kt - pl, 2 * f + kf - pl
                        v = x[ti, fi] if (0 <= ti < T and 0 <= fi < F) else F32(0)
                        if v != 0:
                            o = orc.axpy(o, w0[kt * 3 + kf], float(v))
                y[r, f] = o
        L = out_n(valid)
        y = relu(mask(y, L))

        def dw(y, name, L):
            # dwConv2 (encoder.go:80-110): from the bias, w * x unfused over
            # the taps in range, in order
            T, F = y.shape[0], y.shape[1]
            T1, F1 = out_n(T), out_n(F)
            w, b = taps(name + ".weight"), np.asarray(t[pe + name + ".bias"], F32)
            o = np.tile(b, (T1, F1, 1))
            for kt in range(3):
                for kf in range(3):
                    for r in range(T1):
                        ti = 2 * r + kt - pl
                        if not 0 <= ti < T:
                            continue
                        for f in range(F1):
                            fi = 2 * f + kf - pl
                            if 0 <= fi < F:
                                o[r, f] = o[r, f] + w[kt * 3 + kf] * y[ti, fi]
            L = out_n(L)
            return mask(o, L), L

        def pointwise(y, name, L):
            T, F = y.shape[0], y.shape[1]
            w, b = t[pe + name + ".weight"], t[pe + name + ".bias"]
            flat = y.reshape(T * F, c)
            if np.asarray(w).dtype == np.float32:
                z = orc.matmul_f32(flat, np.asarray(w, F32).reshape(c, c), bias=b)
            else:
                z = orc.matmul_q8_int(flat, w, c, c, bias=b)
            return relu(mask(z.reshape(T, F, c), L))

        y, L = dw(y, "conv.2", L)
        y = pointwise(y, "conv.3", L)
        y, L = dw(y, "conv.5", L)
        y = pointwise(y, "conv.6", L)
        T, F = y.shape[0], y.shape[1]
        # flattened [t][c*F+f] (encoder.go:158-166), then the output Linear
        flat = y.reshape(T, F * c) if self.plant == "sub_flatten" else y.transpose(0, 2, 1).reshape(T, c * F)
        out = orc.matmul_q8_int(np.ascontiguousarray(flat), t[pe + "out.weight"], d, c * F, bias=t[pe + "out.bias"])
        return out, T, max(0, min(L, T))

    def encode(self, mel, valid):
        """Model.encode (encoder.go:432-489): the pre-encoder, x *= f32(sqrt(d))
        when the model scales, each block; (out [T][d], L)."""
        x, T, L = self.subsample(mel, valid)
        if self.hp.get("xscaling", True) and self.plant != "no_xscale":
            x = x * F32(math.sqrt(self.hp["d"]))
        for i in range(self.hp["layers"]):
            x = self.block(i, x, L)
        return x, L

    def block(self, i, x, L):
        """One block offline (encoder.go:474-486): the position projection
        of relPosEmb(T), offlineKeys' ranges and blocks, runBlock."""
        T, D = x.shape[0], self.hp["d"]
        pp = self.linear(self.orc.conf_rel_pos(T, D), f"enc.blocks.{i}.attn.linear_pos.weight", D, D)
        return self.run_block(i, x, L, None, lambda q: key_range(self.hp, T, L, q), key_range(self.hp, T, L, None),
                              pp, None)[0]

    def run_block(self, i, x, L, kv_before, keyf, bl, pp, conv_prev):
        """runBlock (encoder.go:411-429); kv_before: a stream's cached
        attention inputs.  Returns (x, the key rows, the gated frames)."""
        p = f"enc.blocks.{i}."
        x = np.asarray(x, F32).copy()
        x = self.feed_forward(x, p, "ff1")
        ln = self.ln(x, p + "norm_attn")
        kv = ln if kv_before is None else np.concatenate([kv_before, ln])
        x = self.attention(x, ln, p, L, kv, keyf, bl, pp)
        x, glu = self.conv_module(x, self.ln(x, p + "norm_conv"), p, L, conv_prev)
        x = self.feed_forward(x, p, "ff2")
        return self.ln(x, p + "norm_out"), kv, glu


# the tiny regular model (every key, blocks of 32, batch norm), and a
# streaming-shaped one (chunked limited context of 4-row chunks with two
# chunks of left context, a causal convolution with its LayerNorm)
CHUNKED = dict(CONFORMER_TINY, conv_norm="layer_norm", att_style="chunked_limited", att_left=8, att_right=3,
               conv_left=8, conv_right=0)


@pytest.fixture(scope="module", params=["regular", "chunked"])
def model(request):
    hp = dict(CONFORMER_TINY) if request.param == "regular" else dict(CHUNKED)
    return hp, conformer_model(hp, seed=9)


def test_restated_layernorm_equals_the_oracles(orc):
    rng = np.random.default_rng(3)
    for n in (32, 64, 96):
        x = (rng.standard_normal((5, n)) * 3).astype(F32)
        w, b = rng.standard_normal(n).astype(F32), rng.standard_normal(n).astype(F32)
        assert np.array_equal(_bits(ln_kern(x, w, b)), _bits(orc.layernorm(x, w, b))), n


def test_key_ranges_equal_the_oracles(orc, model):
    """The composition's key ranges and block length are the oracle's (its
    key range loops are pinned to their closed forms on their own)."""
    hp, t = model
    m = orc.ConformerOracle(hp, t)
    for T, L in ((40, 37), (40, 40), (23, 9)):
        keys, bl = m.offline_keys(T, L)
        assert bl == key_range(hp, T, L, None), (T, L)
        assert [tuple(orc.conf_key_range(keys, q)) for q in range(T)] == [key_range(hp, T, L, q) for q in range(T)]


@pytest.mark.parametrize("T,L", [(40, 37), (23, 23)])
def test_oracle_block_is_the_composition(orc, model, T, L):
    """Each block of the oracle equals the composition bit for bit on an
    input with valid length L (rows from L on masked)."""
    hp, t = model
    m = orc.ConformerOracle(hp, t)
    comp = Composed(orc, hp, t)
    rng = np.random.default_rng(T + L)
    x = rng.standard_normal((T, hp["d"])).astype(F32)
    for i in range(hp["layers"]):
        want = m.block(i, x, L)
        got = comp.block(i, x, L)
        assert np.array_equal(_bits(got), _bits(want)), (i, T, L)
        x = want


@pytest.mark.parametrize("plant", ["ff_full_step", "pos_bias_swap", "rel_shift", "scale_d", "glu_swap",
                                   "glu_unmasked", "dw_reversed", "ln_eps"])
def test_planted_mistakes_break_the_pin(orc, model, plant):
    """Each planted mistake changes the block's bits."""
    hp, t = model
    m = orc.ConformerOracle(hp, t)
    rng = np.random.default_rng(77)
    T, L = 40, 37
    x = rng.standard_normal((T, hp["d"])).astype(F32)
    got = Composed(orc, hp, t, plant=plant).block(0, x, L)
    assert not np.array_equal(_bits(got), _bits(m.block(0, x, L))), plant


def test_oracle_subsample_and_encode_are_the_composition(orc, model):
    """The oracle's pre-encoder and whole encode (pre-encoder, xscale,
    every block) equal the composition bit for bit, valid frames short of
    the recording."""
    from gorelaxor_amd.synth import noise_mel
    hp, t = model
    m = orc.ConformerOracle(hp, t)
    comp = Composed(orc, hp, t)
    mel, frames, valid = noise_mel(hp["n_mels"], seconds=0.8, seed=12)
    for v in (valid, valid - 13):
        want, T, L = m.subsample(mel, v)
        got, T2, L2 = comp.subsample(mel, v)
        assert (T, L) == (T2, L2), v
        assert np.array_equal(_bits(got), _bits(want)), v
        want, L = m.encode(mel, v)
        got, L2 = comp.encode(mel, v)
        assert L == L2 and np.array_equal(_bits(got), _bits(want)), v


@pytest.mark.parametrize("plant", ["sub_pad", "sub_unmasked", "sub_flatten", "no_xscale"])
def test_planted_pre_encoder_mistakes_break_the_pin(orc, model, plant):
    """Each planted pre-encoder mistake changes the encode's bits."""
    from gorelaxor_amd.synth import noise_mel
    hp, t = model
    m = orc.ConformerOracle(hp, t)
    mel, frames, valid = noise_mel(hp["n_mels"], seconds=0.8, seed=12)
    want, L = m.encode(mel, valid - 13)
    got, L2 = Composed(orc, hp, t, plant=plant).encode(mel, valid - 13)
    assert got.shape != want.shape or not np.array_equal(_bits(got), _bits(want)), plant


class StreamComposed:
    """A stream's chunk steps (stream.go:241-307) over Composed: each
    chunk's pre-encoder rows (all but the first chunk's first `drop` cut),
    xscale, and every block with the stream's cached attention inputs (its
    last `left` key rows), the chunk keys of stream.go:273-287 (the closed
    form of its loops), the position rows for relative positions Tk - 1
    down (relPosRange), and the convolution's last padL gated frames."""

    def __init__(self, comp, right, left, drop, plant=None):
        hp = comp.hp
        self.comp, self.left, self.drop, self.plant = comp, left, drop, plant
        self.chunk = right + 1
        self.lchunks = left // self.chunk
        cl, cr = hp.get("conv_left", -1), hp.get("conv_right", -1)
        self.padL = cl if cl >= 0 and cr >= 0 else (hp["conv_kernel"] - 1) // 2
        D = hp["d"]
        self.kv = [np.zeros((0, D), F32) for _ in range(hp["layers"])]
        self.conv = [np.zeros((self.padL, D), F32) for _ in range(hp["layers"])]
        self.first = True

    def step(self, mel, length):
        comp, hp = self.comp, self.comp.hp
        D = hp["d"]
        x, T, L = comp.subsample(mel, length)
        if not self.first and self.plant != "no_drop":
            x = x[min(self.drop, T):]
            T, L = max(T - self.drop, 0), max(L - self.drop, 0)
        self.first = False
        L = min(L, T)
        if T <= 0:
            return np.zeros((0, D), F32)
        if hp.get("xscaling", True):
            x = x * F32(math.sqrt(D))
        c = self.kv[0].shape[0]
        Tk, slot0 = c + T, self.left - c

        def keyf(q):
            if q - c >= L:
                return 0, 0
            qc = (slot0 + q) // self.chunk
            return max(0, (qc - self.lchunks) * self.chunk - slot0), min(c + L, (qc + 1) * self.chunk - slot0)

        for i in range(hp["layers"]):
            pp = comp.linear(comp.orc.conf_rel_pos(Tk, D), f"enc.blocks.{i}.attn.linear_pos.weight", D, D)
            prev = None if self.plant == "conv_no_carry" else self.conv[i]
            x, kv, glu = comp.run_block(i, x, L, self.kv[i], keyf, T, pp, prev)
            self.kv[i] = kv[max(0, Tk - self.left + (1 if self.plant == "kv_keep_fewer" else 0)):]
            if self.padL > 0:
                self.conv[i] = np.concatenate([self.conv[i], glu])[T:]
        return x[:L]


@pytest.mark.parametrize("right", [0, 1, 13])
def test_oracle_stream_is_the_composition(orc, right):
    """The oracle's chunk steps equal the composition's bit for bit at right
    contexts 0 (where streaming differs from the offline encode), 1 and 13,
    past the left context (the key cache full, its oldest rows leaving)."""
    from gorelaxor_amd.conformer import mel_chunks, stream_geom
    from gorelaxor_amd.synth import noise_mel
    hp = dict(CHUNKED, att_left=8, context_choices=[(8, 13), (8, 6), (8, 1), (8, 0)])
    t = conformer_model(hp, seed=9, pointwise_f16=False)
    mel, frames, _ = noise_mel(hp["n_mels"], seconds=2.5, seed=5)
    g = stream_geom(hp, right)
    ref = orc.ConformerOracle(hp, t).stream(right, g["left"], g["drop"])
    comp = StreamComposed(Composed(orc, hp, t), right, g["left"], g["drop"])
    n = 0
    for j, (ch, length, _) in enumerate(mel_chunks(mel, g)):
        want = ref.step(ch, length)
        got = comp.step(ch, length)
        assert np.array_equal(_bits(got), _bits(want)), (right, j)
        n += len(want)
    assert n > 25


@pytest.mark.parametrize("plant", ["no_drop", "conv_no_carry", "kv_keep_fewer"])
def test_planted_stream_mistakes_break_the_pin(orc, plant):
    """Each planted stream mistake changes the chunks' bits: the first
    `drop` rows kept, the convolution's gated frames not carried, one key
    row fewer than the left context kept (one more changes nothing: the
    chunk keys never reach past the left context)."""
    from gorelaxor_amd.conformer import mel_chunks, stream_geom
    from gorelaxor_amd.synth import noise_mel
    hp = dict(CHUNKED, att_left=8, context_choices=[(8, 13), (8, 6), (8, 1), (8, 0)])
    t = conformer_model(hp, seed=9, pointwise_f16=False)
    mel, frames, _ = noise_mel(hp["n_mels"], seconds=2.5, seed=5)
    g = stream_geom(hp, 1)
    ref = orc.ConformerOracle(hp, t).stream(1, g["left"], g["drop"])
    comp = StreamComposed(Composed(orc, hp, t), 1, g["left"], g["drop"], plant=plant)
    differs = False
    for ch, length, _ in mel_chunks(mel, g):
        want, got = ref.step(ch, length), comp.step(ch, length)
        differs |= got.shape != want.shape or not np.array_equal(_bits(got), _bits(want))
    assert differs, plant
