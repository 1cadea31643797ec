"""The whisper-shaped Q8_0 decoder on the GPU against the CPU oracle: logits
bit-identical at every step and greedy token sequences identical, at a small
shape, at a shape with ragged attention lengths, and at the whisper base.en
shape (d 512, 8 heads, 6 layers, FFN 2048, vocab 51864, 1500 audio
positions)."""
import os

import numpy as np
import pytest

from gorelaxor_amd.synth import WHISPER_BASE_EN, WHISPER_TINY_TEST, encoder_output, whisper_model

pytestmark = pytest.mark.gpu


def _pair(orc, hp, seed=3):
    from gorelaxor_amd.whisper import WhisperDecoder

    t = whisper_model(hp, seed=seed)
    enc = encoder_output(hp, seed=seed + 1)
    ref = orc.WhisperOracle(hp, t)
    ref.set_encoder_output(enc)
    dec = WhisperDecoder(hp, t)
    dec.set_encoder_output(enc)
    return ref, dec


def _same(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


@pytest.mark.parametrize("gemv1", [1, 0])
@pytest.mark.parametrize("shape", ["tiny", "ragged", "wide"])
def test_decode_logits_bit_exact(kern, orc, shape, gemv1):
    """Every step's logits bit-identical, with the one-row decode kernel
    (GEMV1=1, the default) and with the general product kernel.  The tiny
    and wide shapes (heads of 64) take each head's q|k|v product and its
    self-attention in one launch and the wide one the cross query inside
    the scores kernel (FUSE_SELF_ATTN=0 and FUSE_XSCORES=0 turn both off
    with the general kernel); its 101 audio positions leave a partial last
    run of keys and three keys on dotF32Go's route."""
    hp = dict(WHISPER_TINY_TEST)
    if shape == "ragged":  # audio length not a multiple of 16, odd head count
        hp.update(n_audio_ctx=101, n_head=4, n_state=96, n_vocab=333)
    if shape == "wide":
        hp.update(n_audio_ctx=101, n_head=8, n_state=512, n_vocab=333)
    with kern.tuned(GEMV1=gemv1, FUSE_XSCORES=gemv1, FUSE_SELF_ATTN=gemv1):
        _decode_logits_bit_exact(orc, hp)


@pytest.mark.parametrize("rows", [8, 16, 32, 64])
@pytest.mark.parametrize("shape", ["ragged", "wide"])
def test_decode_each_row_slice(kern, orc, shape, rows):
    """The one-row products on slices of 8, 16 or 32 rows of each 64-row
    tile (GEMV1_ROWS; 64 = whole tiles): the q|k|v cache epilogue, the
    embedding prologue stored once, the residual and rounded GELU
    epilogues; every step's logits bit-identical."""
    hp = dict(WHISPER_TINY_TEST)
    if shape == "ragged":
        hp.update(n_audio_ctx=101, n_head=4, n_state=96, n_vocab=333)
    if shape == "wide":
        hp.update(n_audio_ctx=101, n_head=8, n_state=512, n_vocab=333)
    with kern.tuned(GEMV1_ROWS=rows):
        _decode_logits_bit_exact(orc, hp)


@pytest.mark.parametrize("fuse", [1, 0])
def test_decode_self_attention_past_one_pass(kern, orc, fuse):
    """A context longer than one pass of the fused q|k|v + self-attention
    kernel (256 positions, four threads each): heads of 64 over 300
    positions, logits bit-identical at every step; and the same with the
    product and the attention in launches of their own (FUSE_SELF_ATTN=0)."""
    hp = dict(WHISPER_TINY_TEST, n_text_ctx=320)
    with kern.tuned(FUSE_SELF_ATTN=fuse):
        ref, dec = _pair(orc, hp, seed=21)
        toks = [5, 17, 3, 99]
        lr = ref.decode(toks)
        lg, nxt = dec.decode(toks)
        assert _same(lg, lr)
        for step in range(296):
            tok = nxt
            lr = ref.decode([tok])
            lg, nxt = dec.decode([tok])
            assert _same(lg, lr), f"step {step}: max |diff| {np.abs(lg - lr).max()}"
            assert nxt == orc.argmax(lr)
        assert dec.pos == 300


def _decode_logits_bit_exact(orc, hp):
    ref, dec = _pair(orc, hp)
    toks = [5, 17, 3, 99]
    lr = ref.decode(toks)
    lg, nxt = dec.decode(toks)
    assert _same(lg, lr), f"prompt: max |diff| {np.abs(lg - lr).max()}"
    assert nxt == orc.argmax(lr)
    for step in range(12):  # one token at a time, graph replays after the first
        tok = nxt
        lr = ref.decode([tok])
        lg, nxt = dec.decode([tok])
        assert _same(lg, lr), f"step {step}: max |diff| {np.abs(lg - lr).max()}"
        assert nxt == orc.argmax(lr)
    assert dec.pos == ref.n


def test_greedy_tokens_identical_and_eager_equals_graph(kern, orc):
    hp = dict(WHISPER_TINY_TEST)
    ref, dec = _pair(orc, hp, seed=9)
    want = ref.greedy([1, 2, 3, 4], 40)
    got = dec.greedy([1, 2, 3, 4], 40)
    assert list(got) == list(want)
    with kern.tuned(NO_GRAPH=1):
        from gorelaxor_amd.whisper import WhisperDecoder

        t = whisper_model(hp, seed=9)
        eager = WhisperDecoder(hp, t)
        eager.set_encoder_output(encoder_output(hp, seed=10))
        assert list(eager.greedy([1, 2, 3, 4], 40)) == list(want)
    # replaying the greedy loop again from an empty cache repeats it
    assert list(dec.greedy([1, 2, 3, 4], 40)) == list(want)


def test_context_limit_and_errors(kern, orc):
    from gorelaxor_amd import GrxError
    from gorelaxor_amd.whisper import WhisperDecoder

    hp = dict(WHISPER_TINY_TEST)
    dec = WhisperDecoder(hp, whisper_model(hp, seed=1))
    with pytest.raises(GrxError, match="no encoder output"):
        dec.decode([1])
    dec.set_encoder_output(encoder_output(hp))
    with pytest.raises(GrxError, match="exceed the context"):
        dec.decode(list(range(hp["n_text_ctx"] + 1)))
    with pytest.raises(GrxError, match="vocabulary"):
        dec.decode([hp["n_vocab"]])
    bad = WhisperDecoder(hp)
    with pytest.raises(GrxError, match="wrong shape"):
        bad.set_tensor("decoder.ln.weight", np.zeros(3, np.float32))
    with pytest.raises(GrxError, match="doesn't know"):
        bad.set_tensor("decoder.nope", np.zeros(3, np.float32))


def test_base_en_shape_greedy(kern, orc):
    """whisper base.en shape over the configuration's whole decode: a
    4-token prompt, then 220 greedy steps (the cache grows from 4 to 224
    positions, whisper/transcribe.go:165).  The device's greedy loop gives
    the oracle's tokens, and stepping both one token at a time, every
    step's logits are bit-identical."""
    hp = dict(WHISPER_BASE_EN)
    ref, dec = _pair(orc, hp, seed=7)
    prompt, n_steps = [50257, 50362, 50363, 50258], 220
    want = ref.greedy(prompt, n_steps)
    got = dec.greedy(prompt, n_steps)
    assert list(got) == list(want)
    ref.reset()
    dec.reset()
    lr = ref.decode(prompt)
    lg, nxt = dec.decode(prompt)
    assert _same(lg, lr) and nxt == int(want[0])
    for s in range(n_steps):
        lr = ref.decode([int(want[s])])
        lg, nxt = dec.decode([int(want[s])])
        assert _same(lg, lr), f"step {s}: max |diff| {np.abs(lg - lr).max()}"
        assert nxt == int(want[s + 1]), s
    assert dec.pos == len(prompt) + n_steps


def _streams(hp, t, n, seed):
    from gorelaxor_amd.whisper import WhisperDecoder

    dec = WhisperDecoder(hp, t, streams=n)
    encs = [encoder_output(hp, seed=seed + k) for k in range(n)]
    for k, e in enumerate(encs):
        dec.set_encoder_output_stream(k, e)
    return dec, encs


@pytest.mark.parametrize("fuse_ln", [1, 0])
@pytest.mark.parametrize("n", [2, 4, 8])
def test_streams_tokens_identical_to_each_oracle_decode(kern, orc, n, fuse_ln):
    """Independent streams decoded side by side (every product n rows): each
    stream's greedy tokens are those of its own oracle decode, with each
    stream's LayerNorm row built inside the product (one wave per row) and
    the cross values on 16-output workgroups, or (FUSE_LN=0,
    WAVE_VALUES=0) a row kernel beforehand and the values kernel that
    rounds its outputs."""
    with kern.tuned(FUSE_LN=fuse_ln, WAVE_VALUES=fuse_ln):
        _streams_vs_oracle(orc, n)


@pytest.mark.parametrize("n", [2, 8])
def test_streams_wide_rows_carried_chain(kern, orc, n):
    """Streams at d_model 1280 (the large-v3-turbo width): the out and
    cross-out products on the K-split matrix-core kernel, and fc2 (5120
    inputs, 160 blocks: more than one workgroup holds) in two runs with each
    output's chain carried between them; greedy tokens equal each stream's
    own oracle decode."""
    hp = dict(WHISPER_TINY_TEST, n_state=1280, n_head=20, n_layer=2, n_audio_ctx=64, n_vocab=700)
    _streams_vs_oracle(orc, n, hp, steps=8)


def _streams_vs_oracle(orc, n, hp=None, steps=30):
    hp = dict(hp or WHISPER_TINY_TEST)
    t = whisper_model(hp, seed=21)
    dec, encs = _streams(hp, t, n, seed=40)
    prompts = [[1 + k, 2, 3 + 2 * k, 4] for k in range(n)]
    got = dec.greedy_streams(prompts, steps)
    for k in range(n):
        ref = orc.WhisperOracle(hp, t)
        ref.set_encoder_output(encs[k])
        assert list(got[k]) == list(ref.greedy(prompts[k], steps)), k
    # the loop again from empty caches repeats itself (graph replays)
    assert np.array_equal(dec.greedy_streams(prompts, steps), got)


def test_streams_errors(kern):
    from gorelaxor_amd import GrxError
    from gorelaxor_amd.whisper import WhisperDecoder

    hp = dict(WHISPER_TINY_TEST)
    t = whisper_model(hp, seed=2)
    with pytest.raises(GrxError, match="streams"):
        WhisperDecoder(hp, t, streams=3)
    dec = WhisperDecoder(hp, t, streams=2)
    dec.set_encoder_output_stream(0, encoder_output(hp, seed=1))
    with pytest.raises(GrxError, match="no encoder output"):
        dec.greedy_streams([[1, 2], [3, 4]], 2)  # stream 1 has none
    dec.set_encoder_output_stream(1, encoder_output(hp, seed=2))
    with pytest.raises(GrxError, match="greedy_streams"):
        dec.decode([1])
    with pytest.raises(GrxError, match="stream 2"):
        dec.set_encoder_output_stream(2, encoder_output(hp, seed=3))


def test_large_v3_turbo_eight_streams(kern, orc):
    """large-v3-turbo shape (d 1280, 20 heads, 4 layers, FFN 5120, vocab
    51866, 1500 audio positions), 8 streams over the configuration's 220
    greedy steps each: two streams' tokens against the oracle, the rest
    against their own single-stream GPU decode."""
    from gorelaxor_amd.synth import WHISPER_LARGE_V3_TURBO
    from gorelaxor_amd.whisper import WhisperDecoder

    hp = dict(WHISPER_LARGE_V3_TURBO)
    t = whisper_model(hp, seed=23)
    dec, encs = _streams(hp, t, 8, seed=60)
    prompt = [50258, 50259, 50360, 50364]
    n = 220
    got = dec.greedy_streams([prompt] * 8, n)
    dec.close()
    for k in (0, 5):
        ref = orc.WhisperOracle(hp, t)
        ref.set_encoder_output(encs[k])
        assert list(got[k]) == list(ref.greedy(prompt, n)), k
    one = WhisperDecoder(hp, t)
    for k in (1, 2, 3, 4, 6, 7):
        one.set_encoder_output(encs[k])
        assert list(one.greedy(prompt, n)) == list(got[k]), k
    assert len({tuple(g) for g in got}) > 1  # the streams differ


@pytest.mark.parametrize("n", [2, 4])
def test_forked_streams_equal_redecoding_the_prompt(kern, orc, n):
    """transcribe.go:170-204 over streams: one window's encoder output set
    on stream 0 and shared with the others (no second projection); the
    prompt decoded on stream 0 while the other streams decode other
    prompts; then kvCache.copyFrom (decoder.go:22-28) of stream 0 into
    every other stream.  Every stream then continues exactly as
    re-decoding the prompt does: the same greedy tokens as the oracle's
    prompt decode, and at every step the oracle's logits bit for bit."""
    from gorelaxor_amd.whisper import WhisperDecoder

    hp = dict(WHISPER_TINY_TEST)
    t = whisper_model(hp, seed=23)
    enc = encoder_output(hp, seed=24)
    dec = WhisperDecoder(hp, t, streams=n)
    dec.set_encoder_output_stream(0, enc)
    for k in range(1, n):
        dec.share_encoder_output(k, 0)
    prompt = [7, 3, 11, 5]
    prompts = [prompt] + [[20 + k, 2, 9, 1 + k] for k in range(1, n)]
    first = dec.greedy_streams(prompts, 0)
    ref = orc.WhisperOracle(hp, t)
    ref.set_encoder_output(enc)
    want = ref.greedy(prompt, 12)
    assert first[0, 0] == want[0]
    for k in range(1, n):
        dec.copy_stream(k, 0)
    ref.reset()
    lr = ref.decode(prompt)
    for s in range(12):
        got = dec.steps(1)
        lr = ref.decode([int(want[s])])
        for k in range(n):
            assert got[k, 0] == want[s + 1], (s, k)
            assert _same(dec.logits(k), lr), (s, k)
    assert dec.pos == len(prompt) + 12


def test_stream_copy_errors(kern):
    from gorelaxor_amd import GrxError
    from gorelaxor_amd.whisper import WhisperDecoder

    hp = dict(WHISPER_TINY_TEST)
    dec = WhisperDecoder(hp, whisper_model(hp, seed=1), streams=2)
    with pytest.raises(GrxError, match="streams 2, 0 of 2"):
        dec.copy_stream(2, 0)
    with pytest.raises(GrxError, match="no encoder output"):
        dec.share_encoder_output(1, 0)
    dec.set_encoder_output_stream(0, encoder_output(hp))
    dec.share_encoder_output(1, 0)
    with pytest.raises(GrxError, match="nothing decoded"):
        dec.steps(1)
    with pytest.raises(GrxError, match="nothing decoded"):
        dec.logits(0)
