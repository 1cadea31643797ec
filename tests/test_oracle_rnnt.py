"""The oracle of greedy RNN-T / TDT decoding (conformer/rnnt.go:46-173),
pinned without the reference: its double exp against the C library's, its
tanh32 against math.tanh, the greedy loop's frame and symbol accounting on
joints whose decision is fixed by the output bias (closed forms for the
token count, frames, durations and the max_iters bound), the emitted
probability against a float64 softmax, and the LSTM state against a float64
restatement of the cell."""
import math

import numpy as np
import pytest

from gorelaxor_amd import synth
from oracle import oracle as O

TINY = synth.RNNT_TINY


def test_fd_exp_within_an_ulp():
    rng = np.random.default_rng(1)
    xs = np.concatenate([rng.uniform(-745, 709, 4000), rng.uniform(-2, 2, 4000), rng.uniform(-1e-6, 1e-6, 500),
                         [0.0, -0.0, 1.0, -1.0, 0.5 * math.log(2), 1.5 * math.log(2), 709.7, -745.1, 1e-9]])
    for x in xs:
        got, want = O.fd_exp(float(x)), math.exp(float(x))
        if want == 0.0 or got == 0.0:
            assert abs(got - want) <= 5e-324 * 2, x
            continue
        assert abs(got - want) <= math.ulp(want), (x, got, want)
    assert O.fd_exp(0.0) == 1.0
    assert O.fd_exp(1000.0) == math.inf and O.fd_exp(-1000.0) == 0.0


def test_tanh32_matches_math_tanh():
    rng = np.random.default_rng(2)
    xs = np.concatenate([rng.standard_normal(20000) * 3, rng.uniform(-0.7, 0.7, 5000), [45.0, -45.0, 50.0, 0.625,
                                                                                         -0.625, 1e-30]])
    xs = xs.astype(np.float32)
    diff = 0
    for x in xs:
        got = np.float32(O.tanh32(float(x)))
        want = np.float32(math.tanh(float(x)))
        if got != want:
            diff += 1
            assert abs(float(got) - float(want)) <= float(np.spacing(np.float32(abs(want)))), x
    assert diff <= 2, diff  # float32 rounding boundaries only
    assert np.float32(O.tanh32(-0.0)).tobytes() == np.float32(-0.0).tobytes()
    assert O.tanh32(100.0) == 1.0 and O.tanh32(-100.0) == -1.0


def _fixed_joint(hp, bias, seed=3):
    """The synthetic head with a zero output matrix: every joint gives the
    output bias, so the greedy decision is fixed."""
    t = synth.rnnt_model(hp, seed=seed)
    t["joint.out.weight"] = np.zeros_like(t["joint.out.weight"])
    t["joint.out.bias"] = np.asarray(bias, np.float32)
    return t


def _softmax_at(b, V, i):
    v = np.asarray(b[:V], np.float64)
    return float(np.exp(v[i] - v.max()) / np.exp(v - v.max()).sum())


def test_all_blank_emits_nothing_and_keeps_the_state():
    V = TINY["pred_vocab"]
    b = np.zeros(V, np.float32)
    b[V - 1] = 5.0
    o = O.RnntOracle(TINY, _fixed_joint(TINY, b))
    toks, (h, c, last) = o.decode(synth.rnnt_encoder_output(TINY, 30))
    assert toks == [] and last == -1 and not h.any() and not c.any()


@pytest.mark.parametrize("T,offset", [(1, 0), (7, 100)])
def test_rnnt_token_every_symbol(T, offset):
    V, k = TINY["pred_vocab"], 13
    b = np.linspace(-1, 1, V).astype(np.float32)
    b[k] = 3.0
    o = O.RnntOracle(TINY, _fixed_joint(TINY, b))
    toks, (_, _, last) = o.decode(synth.rnnt_encoder_output(TINY, T), frame_offset=offset)
    assert len(toks) == 10 * T  # RNN-T: ten symbols a frame
    assert [f for _, f, _, _ in toks] == [offset + s for s in range(T) for _ in range(10)]
    assert all(i == k and d == 1 for i, _, d, _ in toks) and last == k
    p = _softmax_at(b, V, k)
    assert all(abs(q - p) <= 2e-7 * p for _, _, _, q in toks)


@pytest.mark.parametrize("dur_index,blank", [(2, False), (3, False), (2, True), (0, False)])
def test_tdt_durations(dur_index, blank):
    durs = [0, 1, 2, 3]
    hp = dict(TINY, head_kind="tdt", durations=durs, max_symbols=4)
    V, T, k = hp["pred_vocab"], 23, 5
    b = np.zeros(V + len(durs), np.float32)
    b[V - 1 if blank else k] = 4.0
    b[V + dur_index] = 2.0
    o = O.RnntOracle(hp, _fixed_joint(hp, b))
    toks, _ = o.decode(synth.rnnt_encoder_output(hp, T))
    D = durs[dur_index]
    if blank:
        assert toks == []
    elif D == 0:  # four symbols, then the frame advances by one
        assert [f for _, f, _, _ in toks] == [s for s in range(T) for _ in range(4)]
        assert all(d == 0 for _, _, d, _ in toks)
    else:
        assert [f for _, f, _, _ in toks] == list(range(0, T, D))
        assert all(i == k and d == D for i, _, d, _ in toks)


def test_iteration_bound():
    """Duration 0 with 100 symbols a frame: the loop stops at 16T+1024
    iterations (rnnt.go:138), every one of them a token."""
    hp = dict(TINY, head_kind="tdt", durations=[0, 1], max_symbols=100)
    V, T = hp["pred_vocab"], 20
    b = np.zeros(V + 2, np.float32)
    b[7] = 4.0
    b[V] = 2.0
    o = O.RnntOracle(hp, _fixed_joint(hp, b))
    toks, _ = o.decode(synth.rnnt_encoder_output(hp, T))
    assert len(toks) == 16 * T + 1024
    assert [f for _, f, _, _ in toks] == [s for s in range(T) for _ in range(100)][:16 * T + 1024]


def _lstm64(t, hp, x, h, c):
    """float64 LSTM step over the dequantized weights."""
    H = hp["pred_hidden"]
    hn, cn = [], []
    for l in range(hp["pred_layers"]):
        wx = synth.q8_dequant(t[f"pred.lstm.{l}.Wx"], 4 * H, H).astype(np.float64)
        wh = synth.q8_dequant(t[f"pred.lstm.{l}.Wh"], 4 * H, H).astype(np.float64)
        g = wx @ x + t[f"pred.lstm.{l}.bias"] + wh @ h[l]
        sg = lambda v: 1 / (1 + np.exp(-v))
        cc = sg(g[H:2 * H]) * c[l] + sg(g[:H]) * np.tanh(g[2 * H:3 * H])
        hh = sg(g[3 * H:]) * np.tanh(cc)
        hn.append(hh)
        cn.append(cc)
        x = hh
    return np.array(hn), np.array(cn)


def test_lstm_state_against_float64():
    """One token per call (TDT, duration 1, T = 1): the state returned is
    the prediction network's step from the state passed in, fed the last
    token (zeros at the start)."""
    hp = dict(TINY, head_kind="tdt", durations=[1, 2], max_symbols=4)
    V, H, k = hp["pred_vocab"], hp["pred_hidden"], 11
    b = np.zeros(V + 2, np.float32)
    b[k] = 4.0
    b[V] = 1.0
    t = _fixed_joint(hp, b)
    o = O.RnntOracle(hp, t)
    enc = synth.rnnt_encoder_output(hp, 1)
    toks, st = o.decode(enc)
    assert [(i, f, d) for i, f, d, _ in toks] == [(k, 0, 1)] and st[2] == k
    z = np.zeros((hp["pred_layers"], H))
    h1, c1 = _lstm64(t, hp, np.zeros(H), z, z)
    np.testing.assert_allclose(st[0], h1, atol=2e-5)
    np.testing.assert_allclose(st[1], c1, atol=2e-5)
    toks2, st2 = o.decode(enc, state=st, frame_offset=1)
    assert [(i, f) for i, f, _, _ in toks2] == [(k, 1)]
    h2, c2 = _lstm64(t, hp, t["pred.embed.weight"][k].astype(np.float64), h1, c1)
    np.testing.assert_allclose(st2[0], h2, atol=5e-5)
    np.testing.assert_allclose(st2[1], c2, atol=5e-5)
    assert np.abs(h2 - h1).max() > 1e-2  # the embedding of k reached the state


def test_synthetic_heads_emit_and_advance():
    """The random heads the GPU tests use mix tokens and blanks."""
    for hp in (TINY, synth.RNNT_TDT):
        toks, _ = O.RnntOracle(hp, synth.rnnt_model(hp)).decode(synth.rnnt_encoder_output(hp, 40))
        frames = {f for _, f, _, _ in toks}
        assert 5 < len(toks) and len(frames) < 40


def test_boundary_fixture_needs_the_in_order_sum():
    """tests/golden/rnnt_softmax_boundary.npy: 1/s lies within a quarter of
    the decoder's error interval of a float32 rounding boundary."""
    import os
    x = np.load(os.path.join(os.path.dirname(__file__), "golden", "rnnt_softmax_boundary.npy"))
    V = x.size
    s = 0.0
    for v in x:
        s += O.fd_exp(float(np.float32(v - x.max())))
    q = 1.0 / s
    f = np.float32(q)
    other = np.nextafter(f, np.float32(np.inf if q >= float(f) else -np.inf))
    mid = (float(f) + float(other)) / 2
    assert abs(mid - q) <= q * (V + 4) * 2.0 ** -52 / 4
    o = O.RnntOracle(TINY, _fixed_joint(TINY, x))
    toks, _ = o.decode(synth.rnnt_encoder_output(TINY, 1))
    assert toks[0][0] == int(np.argmax(x)) and np.float32(toks[0][3]) == np.float32(q)
