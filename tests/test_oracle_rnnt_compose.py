"""Pins the oracle's RNN-T / TDT greedy decoder bit for bit, without a GPU.

conformer/rnnt.go:111-173 (Model.Decode) with :47-68 (predict: the LSTM
layers from the last token's embedding), :90-106 (joint) and :78-85
(softmaxAt) is composed here in Python, line by line from the reference,
out of the oracle's primitives - each pinned on its own
(test_oracle_kern.py: the int8 product and kern's float route of a Q8_0
weight for one row, expf; test_oracle_rnnt.py: tanh32 against math.tanh,
the float64 exp) - and the oracle's token ids, frames, durations, the bits
of each p and the final state (h, c, last) must be the composition's: its
loop (two state slots, the prediction recomputed only after an emission,
the frame and symbol accounting, TDT's durations, the iteration bound) is
then the reference's.  Planted mistakes must each break the equality."""
import numpy as np
import pytest

from gorelaxor_amd import synth

F32 = np.float32


class Composed:
    """Decode over the oracle's primitives; `plant` names one mistake to put
    in (None: the reference's loop)."""

    def __init__(self, orc, hp, t, plant=None):
        self.orc, self.hp, self.t, self.plant = orc, hp, t, plant
        self.tdt = hp.get("head_kind", "rnnt") == "tdt"
        self.durs = list(hp.get("durations", [])) if self.tdt else []
        self.max_symbols = hp.get("max_symbols", 10) if self.tdt else 10
        b = hp.get("blank", -1)
        self.blank = b if b >= 0 else hp["pred_vocab"] - 1

    def sigm(self, v):
        """conformer/encoder.go:13: 1 / (1 + expf(-v)) in float32."""
        return np.array([F32(1) / (F32(1) + F32(self.orc.expf(float(-x)))) for x in np.ravel(v)], F32)

    def tanh(self, v):
        return np.array([F32(self.orc.tanh32(float(x))) for x in np.ravel(v)], F32)

    def lin1(self, x, name, n, k, bias=None):
        """A one-row product on kern's float route of the Q8_0 weight."""
        b = None if bias is None else self.t[bias]
        return self.orc.matmul_q8_float(np.asarray(x, F32)[None, :], self.t[name], n, k, bias=b)[0]

    def predict(self, h, c, last):
        """predict (rnnt.go:47-68): the last token's embedding (zeros for
        none or blank) through the LSTM layers; (h', c', the top h)."""
        hp = self.hp
        H = hp["pred_hidden"]
        x = np.zeros(H, F32)
        if last >= 0 and last != self.blank and self.plant != "no_embedding":
            x = np.asarray(self.t["pred.embed.weight"], F32).reshape(-1, H)[last].copy()
        hn, cn = np.zeros_like(h), np.zeros_like(c)
        for layer in range(hp["pred_layers"]):
            p = f"pred.lstm.{layer}."
            g = self.lin1(x, p + "Wx", 4 * H, H, p + "bias") + self.lin1(h[layer], p + "Wh", 4 * H, H)
            i, f = self.sigm(g[:H]), self.sigm(g[H:2 * H])
            if self.plant == "gates_if":
                i, f = f, i
            gg, o = self.tanh(g[2 * H:3 * H]), self.sigm(g[3 * H:])
            cn[layer] = f * c[layer] + i * gg
            hn[layer] = o * self.tanh(cn[layer])
            x = hn[layer]
        return hn, cn, x

    def softmax_at(self, v, n, i):
        """softmaxAt (rnnt.go:78-85): float64 sum of exp(v - max) in order."""
        mx = v[int(np.argmax(v[:n]))]
        s = 0.0
        for j in range(n):
            s += self.orc.fd_exp(float(F32(v[j] - mx)))
        return float(F32(self.orc.fd_exp(float(F32(v[i] - mx))) / s))

    def decode(self, enc, state, frame_offset=0):
        """Decode (rnnt.go:111-173): (tokens as (id, frame, duration, p),
        the final state)."""
        orc, hp, t = self.orc, self.hp, self.t
        T, d = enc.shape[0], hp["d"]
        J, V = hp["joint_hidden"], hp["pred_vocab"]
        R = V + len(self.durs)
        if T == 0:
            return [], state
        if T == 1:
            ep = orc.matmul_q8_float(enc, t["joint.enc.weight"], J, d, bias=t["joint.enc.bias"])
        else:
            ep = orc.matmul_q8_int(enc, t["joint.enc.weight"], J, d, bias=t["joint.enc.bias"])
        hs, cs, lastv = [state[0].copy(), None], [state[1].copy(), None], [state[2], -1]
        cur, dirty, step, newsym = 0, True, 0, 0
        toks = []
        pred = None
        max_iters = 16 * T + 1024
        it = 0
        while step < T and it < max_iters:
            it += 1
            if dirty:
                hs[1 - cur], cs[1 - cur], pred = self.predict(hs[cur], cs[cur], lastv[cur])
                dirty = False
            # joint (rnnt.go:90-106)
            v = ep[step] + self.lin1(pred, "joint.pred.weight", J, hp["pred_hidden"], "joint.pred.bias")
            act = hp.get("joint_act", "relu")
            if act == "sigmoid":
                v = self.sigm(v)
            elif act == "tanh":
                v = self.tanh(v)
            else:
                v = np.where(np.isnan(v) | (v > 0), v, F32(0)).astype(F32)
            logits = self.lin1(v, "joint.out.weight", R, J, "joint.out.bias")
            tok = int(np.argmax(logits[:V]))
            blank = tok == self.blank
            duration = 1
            if self.tdt:
                duration = self.durs[int(np.argmax(logits[V:V + len(self.durs)]))]
            if not blank:
                toks.append((tok, frame_offset + step, duration,
                             self.softmax_at(logits, R if self.plant == "p_over_all" else V, tok)))
                lastv[1 - cur] = tok
                cur = 1 - cur
                dirty = True
            if not self.tdt:
                if blank:
                    step, newsym = step + 1, 0
                else:
                    newsym += 1
                    if self.plant != "no_symbol_limit" and self.max_symbols > 0 and newsym >= self.max_symbols:
                        step, newsym = step + 1, 0
                continue
            step += duration
            newsym += 1
            if duration != 0:
                newsym = 0
            elif self.plant != "no_symbol_limit" and self.max_symbols > 0 and newsym >= self.max_symbols:
                step, newsym = step + 1, 0
        return toks, (hs[cur], cs[cur], lastv[cur])


RNNT_TDT_TINY = dict(synth.RNNT_TINY, head_kind="tdt", durations=[0, 1, 2, 3, 4], max_symbols=4)


def _same(a, b):
    ta, (ha, ca, la) = a
    tb, (hb, cb, lb) = b
    return (len(ta) == len(tb) and all(x[:3] == y[:3] and np.float32(x[3]).tobytes() == np.float32(y[3]).tobytes()
                                       for x, y in zip(ta, tb))
            and np.array_equal(ha.view(np.uint32), hb.view(np.uint32))
            and np.array_equal(ca.view(np.uint32), cb.view(np.uint32)) and la == lb)


@pytest.mark.parametrize("hp", [synth.RNNT_TINY, RNNT_TDT_TINY], ids=["rnnt", "tdt"])
@pytest.mark.parametrize("act", ["relu", "sigmoid", "tanh"])
def test_oracle_decode_is_the_composition(orc, hp, act):
    """Tokens, frames, durations, the bits of p and the final state equal
    the composition's, over 30 frames in one call and then chunks of 7 and
    1 frame carrying the state (one frame: the joint's float route)."""
    hp = dict(hp, joint_act=act)
    t = synth.rnnt_model(hp, seed=23)
    ref, comp = orc.RnntOracle(hp, t), Composed(orc, hp, t)
    enc = synth.rnnt_encoder_output(hp, 30, seed=24)
    a = ref.decode(enc)
    b = comp.decode(enc, ref.new_state())
    assert _same(a, b) and len(a[0]) >= 2, (act, len(a[0]), len(b[0]))
    sa, sb = ref.new_state(), ref.new_state()
    for lo, hi in ((0, 7), (7, 8), (8, 15)):
        a = ref.decode(enc[lo:hi], sa, frame_offset=lo)
        b = comp.decode(enc[lo:hi], sb, frame_offset=lo)
        assert _same(a, b), (act, lo)
        sa, sb = a[1], b[1]


@pytest.mark.parametrize("plant", ["gates_if", "no_embedding", "p_over_all", "no_symbol_limit"])
def test_planted_mistakes_break_the_pin(orc, plant):
    """Each planted mistake changes the tokens, their p or the state."""
    hp = dict(RNNT_TDT_TINY) if plant in ("p_over_all", "no_symbol_limit") else dict(synth.RNNT_TINY)
    # a head that emits often, so the symbol limit is met
    t = synth.rnnt_model(hp, seed=23, blank_bias=-2.0 if plant == "no_symbol_limit" else 0.0)
    ref = orc.RnntOracle(hp, t)
    enc = synth.rnnt_encoder_output(hp, 30, seed=24)
    a = ref.decode(enc)
    b = Composed(orc, hp, t, plant=plant).decode(enc, ref.new_state())
    assert not _same(a, b), plant
