"""Greedy RNN-T / TDT decoding on the GPU (grx_rnnt_decode) against the
oracle (Model.Decode, conformer/rnnt.go:111-173): every token's id, frame,
duration and float32 probability bits identical, and the decoder state left
behind (h and c bits, last token) identical, over RNN-T and TDT heads, the
three joint activations, one frame (the float-route encoder projection) and
many (the int8 route), heads that mostly emit and heads that mostly skip,
decoding in chunks that carry the state, the iteration bound, and the
Parakeet-TDT shape."""
import time

import numpy as np
import pytest

from gorelaxor_amd import GrxError, synth

pytestmark = pytest.mark.gpu

TINY = synth.RNNT_TINY
TDT_TINY = dict(TINY, head_kind="tdt", durations=[0, 1, 2, 3], max_symbols=4)


def _dec(hp, t):
    from gorelaxor_amd.rnnt import TransducerDecoder
    return TransducerDecoder(hp, t)


def _same_tokens(got, want):
    assert len(got) == len(want), (len(got), len(want))
    for g, w in zip(got, want):
        assert (g.ID, g.Frame, g.Duration) == w[:3], (g, w)
        assert np.float32(g.P).tobytes() == np.float32(w[3]).tobytes(), (g, w)


def _same_state(st, ost):
    h, c, last = st.read()
    assert last == ost[2]
    assert h.tobytes() == np.ascontiguousarray(ost[0], np.float32).tobytes()
    assert c.tobytes() == np.ascontiguousarray(ost[1], np.float32).tobytes()


@pytest.mark.parametrize("hp", [TINY, TDT_TINY, dict(TINY, joint_act="tanh"), dict(TDT_TINY, joint_act="sigmoid"),
                                dict(TINY, pred_layers=1, blank=0)], ids=["rnnt", "tdt", "tanh", "sigmoid", "1layer"])
@pytest.mark.parametrize("T", [1, 2, 17, 64])
def test_decode_bit_exact(kern, orc, hp, T):
    for bb in (2.0, 6.0):
        t = synth.rnnt_model(hp, seed=T + 3, blank_bias=bb)
        enc = synth.rnnt_encoder_output(hp, T, seed=T)
        want, ost = orc.RnntOracle(hp, t).decode(enc, frame_offset=5)
        dec = _dec(hp, t)
        st = dec.new_state()
        got = dec.decode(enc, st, frame_offset=5)
        _same_tokens(got, want)
        _same_state(st, ost)
        assert got == dec.decode(enc, None, frame_offset=5)  # no state kept: the same tokens
        dec.close()


@pytest.mark.parametrize("hp", [TINY, TDT_TINY], ids=["rnnt", "tdt"])
def test_chunks_carry_the_state(kern, orc, hp):
    t = synth.rnnt_model(hp, seed=8)
    enc = synth.rnnt_encoder_output(hp, 60, seed=9)
    o = orc.RnntOracle(hp, t)
    dec = _dec(hp, t)
    st = dec.new_state()
    ost = None
    off = 0
    for n in (14, 1, 1, 20, 16, 8):
        want, ost = o.decode(enc[off:off + n], state=ost, frame_offset=off)
        got = dec.decode(enc[off:off + n], st, frame_offset=off)
        _same_tokens(got, want)
        _same_state(st, ost)
        off += n
    # a state written from the host continues as the oracle's does
    h = np.random.default_rng(1).standard_normal((hp["pred_layers"], hp["pred_hidden"])).astype(np.float32) * 0.3
    st.write(h, h * 2, 17)
    want, ost = o.decode(enc[:9], state=(h, h * 2, 17))
    _same_tokens(dec.decode(enc[:9], st), want)
    _same_state(st, ost)
    dec.close()


def test_iteration_bound(kern, orc):
    """Duration 0 and 100 symbols a frame: 16T+1024 tokens, then the loop
    stops, as the oracle's."""
    hp = dict(TINY, head_kind="tdt", durations=[0, 1], max_symbols=100)
    t = synth.rnnt_model(hp, seed=4)
    V = hp["pred_vocab"]
    t["joint.out.weight"] = np.zeros_like(t["joint.out.weight"])
    b = np.zeros(V + 2, np.float32)
    b[7], b[V] = 4.0, 2.0
    t["joint.out.bias"] = b
    enc = synth.rnnt_encoder_output(hp, 20)
    want, _ = orc.RnntOracle(hp, t).decode(enc)
    dec = _dec(hp, t)
    got = dec.decode(enc)
    assert len(got) == 16 * 20 + 1024
    _same_tokens(got, want)
    dec.close()


def test_probability_on_a_rounding_boundary(kern, orc):
    """Logits whose probability sits by a float32 rounding boundary: the
    decoder forms the in-order sum and returns the oracle's bits."""
    import os
    x = np.load(os.path.join(os.path.dirname(__file__), "golden", "rnnt_softmax_boundary.npy"))
    t = synth.rnnt_model(TINY, seed=5)
    t["joint.out.weight"] = np.zeros_like(t["joint.out.weight"])
    t["joint.out.bias"] = x
    enc = synth.rnnt_encoder_output(TINY, 3)
    want, _ = orc.RnntOracle(TINY, t).decode(enc)
    dec = _dec(TINY, t)
    _same_tokens(dec.decode(enc), want)
    dec.close()


def test_device_encoder_output(kern, orc):
    from gorelaxor_amd import hiprt

    hp = TDT_TINY
    t = synth.rnnt_model(hp, seed=12)
    enc = synth.rnnt_encoder_output(hp, 33, seed=13)
    want, _ = orc.RnntOracle(hp, t).decode(enc)
    dec = _dec(hp, t)
    x = hiprt.DeviceBuffer.from_array(enc)
    _same_tokens(dec.decode_dev(x.ptr, 33), want)
    dec.close()


def test_parakeet_tdt_shape(kern, orc):
    """d 1024, 2 x 640 LSTM, joint 640, 1025 outputs + 5 durations."""
    hp = synth.RNNT_TDT
    t = synth.rnnt_model(hp, seed=30)
    enc = synth.rnnt_encoder_output(hp, 125, seed=31)  # 10 s of 80 ms frames
    o = orc.RnntOracle(hp, t)
    t0 = time.perf_counter()
    want, ost = o.decode(enc)
    tc = time.perf_counter() - t0
    dec = _dec(hp, t)
    st = dec.new_state()
    _same_tokens(dec.decode(enc, st), want)
    _same_state(st, ost)
    dec.decode(enc)
    t0 = time.perf_counter()
    for _ in range(5):
        dec.decode(enc)
    tg = (time.perf_counter() - t0) / 5
    print(f"\nparakeet-tdt head, 125 frames, {len(want)} tokens: GPU {tg * 1e3:.2f} ms, oracle {tc * 1e3:.1f} ms",
          flush=True)
    dec.close()


def test_errors(kern):
    from gorelaxor_amd.rnnt import TransducerDecoder

    with pytest.raises(GrxError, match="durations"):
        TransducerDecoder(dict(TINY, head_kind="tdt", durations=[]))
    with pytest.raises(GrxError, match="out of range"):
        TransducerDecoder(dict(TDT_TINY, max_symbols=0))
    with pytest.raises(ValueError, match="not supported"):
        TransducerDecoder(dict(TINY, head_kind="ctc"))
    # a duration that could carry the frame index past int32 is refused at
    # create (nothing is launched)
    for bad in (-1, (1 << 20) + 1, (1 << 31) - 1):
        with pytest.raises(GrxError, match="duration"):
            TransducerDecoder(dict(TDT_TINY, durations=[0, 1, bad]))
    t = synth.rnnt_model(TINY)
    dec = TransducerDecoder(TINY)
    with pytest.raises(GrxError, match="unknown tensor"):
        dec.set_tensor("pred.lstm.9.Wx", t["pred.lstm.0.Wx"])
    with pytest.raises(GrxError, match="bytes"):
        dec.set_tensor("joint.enc.weight", t["pred.lstm.0.Wx"])
    with pytest.raises(GrxError, match="not all set"):
        dec.decode(synth.rnnt_encoder_output(TINY, 3))
    dec.close()
    dec = TransducerDecoder(TINY, t)
    assert dec.decode(np.zeros((0, TINY["d"]), np.float32)) == []
    dec.close()
