"""Pins the oracle's cache-aware streaming encoder (conformer/stream.go:
23-88, 241-307) and the limited-context forms of the offline encoder
(conformer/encoder.go:33-38, 196-212, 343-404) without a GPU:

  - the chunk geometry against NeMo's numbers (a chunk of 8*(R+1) mel
    frames, the first 1+8*R, led by 9 cache frames whose 2 encoder rows
    are dropped), and every chunk giving exactly one chunk of rows;
  - the key ranges' loops (stream.go:273-287) against their closed form;
  - streaming equal, bit for bit, to the offline encode with the same
    limits wherever a chunk's cache frames start at or after frame 0 (right
    context 1 and more: the cache-aware model sees the same frames, rows and
    keys; at right context 0 the second chunk's cache reaches before the
    first frame, and its zero frames become pre-encoder activations the
    offline padding never makes);
  - the oracle within Q8_0 rounding error of a float64 restatement
    (tests/_conf_ref.py) for the causal pre-encoder, chunked and windowed
    attention, the causal convolution with its LayerNorm, and for streams
    chunk by chunk (right context 0 included).
"""
import numpy as np
import pytest

import _conf_ref as R
from gorelaxor_amd.conformer import mel_chunks, stream_geom
from gorelaxor_amd.synth import CONFORMER_TINY, conformer_model, noise_mel

# synthModel(seed, streaming=true) of conformer/synth_test.go:46-111: the
# tiny model with chunked limited attention (70 left, 13 right), its four
# trained right contexts, the causal convolution and its LayerNorm
STREAM_TINY = dict(CONFORMER_TINY, att_style="chunked_limited", att_left=70, att_right=13,
                   context_choices=[(70, 13), (70, 6), (70, 1), (70, 0)], conv_left=8, conv_right=0,
                   conv_norm="layer_norm")


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _rel(got, want):
    return float(np.sqrt(((got - want) ** 2).mean() / (want ** 2).mean()))


@pytest.fixture(scope="module")
def model():
    # Q8_0 pointwise weights everywhere: a float32 pre-encoder pointwise
    # weight takes MatMulF32, whose route depends on a row's index in the
    # matrix, so a chunk's rows would not be the offline rows
    return STREAM_TINY, conformer_model(STREAM_TINY, seed=9, pointwise_f16=False)


def test_geometry_nemo_numbers():
    for right in (13, 6, 1, 0):
        g = stream_geom(STREAM_TINY, right)
        assert (g["chunk"], g["left"], g["left_chunks"]) == (right + 1, 70, 70 // (right + 1))
        assert (g["mel_first"], g["mel_next"], g["mel_cache"], g["drop"]) == (1 + 8 * right, 8 * (right + 1), 9, 2)
    with pytest.raises(ValueError, match="wasn't trained for a right context of 5"):
        stream_geom(STREAM_TINY, 5)
    with pytest.raises(ValueError, match="can't stream"):
        stream_geom(CONFORMER_TINY, 13)
    # without choices the model's own right context is the only one
    hp = dict(STREAM_TINY, context_choices=[])
    assert stream_geom(hp, 13)["left"] == 70
    with pytest.raises(ValueError):
        stream_geom(hp, 6)


def test_chunks_give_one_chunk_of_rows_each(orc, model):
    hp, t = model
    m = orc.ConformerOracle(hp, t)
    mel, frames, _ = noise_mel(hp["n_mels"], seconds=2.3, seed=3)
    for right in (13, 1, 0):
        g = stream_geom(hp, right)
        s = m.stream(right, g["left"], g["drop"])
        chunks = mel_chunks(mel, g)
        for j, (ch, length, first) in enumerate(chunks):
            assert first == (j == 0) and ch.shape[1] == length
            rows = s.step(ch, length)
            if j + 1 < len(chunks):
                assert rows.shape[0] == g["chunk"], (right, j)
            assert s.kv_len == min((j + 1) * g["chunk"], g["left"]) or j + 1 == len(chunks)


def test_key_loops_match_their_closed_form(orc):
    """The loops of stream.go:273-287 against lo = max(0, (qc-lc)*chunk -
    slot0), hi = min(c+L, (qc+1)*chunk - slot0), the form the GPU uses."""
    for left, right in ((70, 13), (70, 6), (70, 1), (70, 0), (20, 3)):
        chunk = right + 1
        lc = left // chunk
        for c in range(0, left + 1, 3 if chunk > 1 else 7):
            for T in {chunk, max(1, chunk - 2)}:
                for L in {T, max(0, T - 1), 0}:
                    k = orc.conf_stream_keys(L, chunk, lc, c, left, T)
                    for q in range(c + T):
                        want = orc.conf_key_range(k, q)
                        if q - c >= L:
                            assert want == (0, 0)
                            continue
                        slot0 = left - c
                        qc = (slot0 + q) // chunk
                        lo = max(0, (qc - lc) * chunk - slot0)
                        hi = min(c + L, (qc + 1) * chunk - slot0)
                        assert want == (lo, hi), (left, right, c, T, L, q)


def test_offline_key_forms(orc, model):
    """offlineKeys (encoder.go:196-212): the chunked form in blocks of one
    chunk, a window in blocks of 16 only when it is shorter than the
    recording, every key in blocks of 32 otherwise; all cut at L."""
    hp, t = model
    m = orc.ConformerOracle(hp, t)
    k, bl = m.offline_keys(40, 37)
    assert bl == 14 and orc.conf_key_range(k, 15) == (0, 28) and orc.conf_key_range(k, 36) == (0, 37)
    assert orc.conf_key_range(k, 37) == (0, 0)
    k, bl = orc.ConformerOracle(dict(hp, att_left=14), t).offline_keys(40, 37)
    assert orc.conf_key_range(k, 36) == (14, 37) and orc.conf_key_range(k, 13) == (0, 14)
    w = orc.ConformerOracle(dict(CONFORMER_TINY, att_left=5, att_right=3), conformer_model(CONFORMER_TINY))
    k, bl = w.offline_keys(40, 40)
    assert bl == 16 and orc.conf_key_range(k, 10) == (5, 14) and orc.conf_key_range(k, 2) == (0, 6)
    k, bl = w.offline_keys(4, 4)  # T-1 = 3 is not past min(5, 3): every key
    assert bl == 32 and orc.conf_key_range(k, 0) == (0, 4)


@pytest.mark.parametrize("right", [13, 6, 1])
def test_stream_equals_offline_bit_for_bit(orc, model, right):
    hp, t = model
    mel, frames, _ = noise_mel(hp["n_mels"], seconds=7.0, seed=5)
    g = stream_geom(hp, right)
    s = orc.ConformerOracle(hp, t).stream(right, g["left"], g["drop"])
    got = np.concatenate([s.step(ch, n) for ch, n, _ in mel_chunks(mel, g)])
    off, L = orc.ConformerOracle(dict(hp, att_right=right), t).encode(mel, frames)
    n = min(len(got), L)
    assert n >= L - 1 and n > 80  # a remainder shorter than 8 frames is not encoded
    assert np.array_equal(_bits(got[:n]), _bits(off[:n]))


def test_right_context_zero_differs_from_offline(orc, model):
    """At right context 0 the second chunk's cache (frames -8..0) reaches
    before the first frame: streaming and offline part from row 1 on."""
    hp, t = model
    mel, frames, _ = noise_mel(hp["n_mels"], seconds=1.0, seed=5)
    g = stream_geom(hp, 0)
    s = orc.ConformerOracle(hp, t).stream(0, g["left"], g["drop"])
    got = np.concatenate([s.step(ch, n) for ch, n, _ in mel_chunks(mel, g)])
    off, L = orc.ConformerOracle(dict(hp, att_right=0), t).encode(mel, frames)
    assert np.array_equal(_bits(got[0]), _bits(off[0]))
    assert not np.array_equal(_bits(got[1]), _bits(off[1]))


def test_offline_chunked_vs_float64(orc, model):
    hp, t = model
    mel, frames, valid = noise_mel(hp["n_mels"], seconds=3.0, seed=6)
    got, L = orc.ConformerOracle(hp, t).encode(mel, valid - 11)
    want, Lw = R.encode(hp, t, mel, valid - 11)
    assert L == Lw
    assert _rel(got[:L], want) < 0.025


def test_offline_window_vs_float64(orc):
    hp = dict(CONFORMER_TINY, att_left=9, att_right=4)
    t = conformer_model(hp, seed=12)
    mel, frames, valid = noise_mel(hp["n_mels"], seconds=3.0, seed=7)
    got, L = orc.ConformerOracle(hp, t).encode(mel, valid)
    want, Lw = R.encode(hp, t, mel, valid)
    assert L == Lw
    assert _rel(got[:L], want) < 0.025
    # the window matters: every key gives another result
    full, _ = orc.ConformerOracle(CONFORMER_TINY, t).encode(mel, valid)
    assert _rel(full[:L], want) > 0.05


@pytest.mark.parametrize("right", [13, 0])
def test_stream_vs_float64(orc, right):
    # a left context of 28 rows, so that 3.5 s (44 rows) reach past it
    hp = dict(STREAM_TINY, att_left=28, context_choices=[(28, 13), (28, 6), (28, 1), (28, 0)])
    t = conformer_model(hp, seed=9, pointwise_f16=False)
    mel, frames, _ = noise_mel(hp["n_mels"], seconds=3.5, seed=8)
    g = stream_geom(hp, right)
    chunks = mel_chunks(mel, g)
    s = orc.ConformerOracle(hp, t).stream(right, g["left"], g["drop"])
    got = [s.step(ch, n) for ch, n, _ in chunks]
    want = R.stream(hp, t, g, chunks)
    assert [len(x) for x in got] == [len(x) for x in want]
    # 0.013 here; a position off by one gives 0.05, one chunk less of left
    # context 0.018 (right context 0) to 0.07, a wrong drop 0.48
    assert _rel(np.concatenate(got), np.concatenate(want)) < 0.016
