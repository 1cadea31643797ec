"""grx_whisper_load_ggml: a whisper.cpp (ggml) model file read into the GPU
decoder (whisper.Load and Model.bind, whisper/model.go:93-404).  The file
holds every tensor the reference binds - the encoder's too - with the
decoder's tensors in several stored types; the loaded decoder's logits must
be bit-identical to the oracle's over the tensors the reference's
conversions give (Q8_0 matrices as stored, other matrices widened through
float16 then rounded to Q8_0, vectors by toF32 or through float16), and bad
files must fail with the reference's error texts."""
import numpy as np
import pytest

from gorelaxor_amd.synth import encoder_output, q8_dequant, q8_weight, whisper_model

from tests import _ggml as G

pytestmark = pytest.mark.gpu

# a decoder the loader accepts: n_audio_ctx 1500, n_vocab >= 51864
HP = dict(n_vocab=51864, n_text_ctx=64, n_state=128, n_head=2, n_layer=2, n_audio_ctx=1500)


def _f16(v):
    return np.asarray(v, np.float32).astype(np.float16).astype(np.float32)


def _encoder_records(hp, n_mels=80, n_audio_layer=1):
    st = hp["n_state"]
    z16 = lambda n: np.zeros(n, np.float16)  # noqa: E731
    z32 = lambda n: np.zeros(n, np.float32)  # noqa: E731
    r = [("encoder.positional_embedding", G.F32, [st, 1500], z32(1500 * st)),
         ("encoder.conv1.weight", G.F16, [3, n_mels, st], z16(3 * n_mels * st)),
         ("encoder.conv1.bias", G.F32, [1, st], z32(st)),
         ("encoder.conv2.weight", G.F16, [3, st, st], z16(3 * st * st)),
         ("encoder.conv2.bias", G.F32, [1, st], z32(st)),
         ("encoder.ln_post.weight", G.F32, [st], z32(st)),
         ("encoder.ln_post.bias", G.F32, [st], z32(st))]
    for i in range(n_audio_layer):
        p = f"encoder.blocks.{i}."
        for v in ("attn_ln.weight", "attn_ln.bias", "attn.query.bias", "attn.value.bias", "attn.out.bias",
                  "mlp_ln.weight", "mlp_ln.bias", "mlp.2.bias"):
            r.append((p + v, G.F32, [st], z32(st)))
        r.append((p + "mlp.0.bias", G.F32, [4 * st], z32(4 * st)))
        for w in ("attn.query.weight", "attn.key.weight", "attn.value.weight", "attn.out.weight"):
            r.append((p + w, G.F16, [st, st], z16(st * st)))
        r.append((p + "mlp.0.weight", G.F16, [st, 4 * st], z16(4 * st * st)))
        r.append((p + "mlp.2.weight", G.F16, [4 * st, st], z16(4 * st * st)))
    return r


def _model_file(orc, seed=3):
    """(records, expected decoder tensors): the decoder's tensors in mixed
    stored types and what the reference's conversions make of each."""
    hp = HP
    st, tctx = hp["n_state"], hp["n_text_ctx"]
    rng = np.random.default_rng(seed + 100)
    t = whisper_model(hp, seed=seed)
    want = dict(t)
    rec = {}
    for name, a in t.items():
        if a.dtype == np.uint8:  # Q8_0 matrix rows x cols
            cols = 4 * st if name.endswith("mlp.2.weight") else st
            rows = a.size // 34 * 32 // cols
            rec[name] = (name, G.Q8_0, [cols, rows], a)
        else:
            rec[name] = (name, G.F32, [a.size], a)
    # matrices stored as F16, F32, Q4_0 and Q5_1: widened through float16,
    # then rounded to Q8_0 (Weight.ToQ8)
    n = "decoder.blocks.1.mlp.0.weight"
    v16 = q8_dequant(t[n], 4 * st, st).astype(np.float16)
    rec[n] = (n, G.F16, [st, 4 * st], v16)
    want[n] = orc.quant_q8(v16.astype(np.float32))
    n = "decoder.blocks.0.cross_attn.query.weight"
    v = (rng.standard_normal(st * st) * 0.05).astype(np.float32)
    rec[n] = (n, G.F32, [st, st], v)
    want[n] = orc.quant_q8(_f16(v))
    n = "decoder.blocks.1.attn.key.weight"
    b, v = G.q4_0_blocks(rng, st * st)
    rec[n] = (n, G.Q4_0, [st, st], b)
    want[n] = orc.quant_q8(_f16(v))
    n = "decoder.blocks.0.mlp.2.weight"
    b, v = G.q5_1_blocks(rng, 4 * st * st)
    rec[n] = (n, G.Q5_1, [4 * st, st], b)
    want[n] = orc.quant_q8(_f16(v))
    # vectors: a Q8_0 bias (through float16), the positional embedding as
    # F16, a 2-D F32 vector that load() keeps as float16, and a single-column
    # F32 one it keeps as float32
    n = "decoder.blocks.0.attn.query.bias"
    qb = q8_weight(rng, 1, st, sigma=2.0)
    rec[n] = (n, G.Q8_0, [st], qb)
    want[n] = _f16(q8_dequant(qb, 1, st).reshape(-1))
    n = "decoder.positional_embedding"
    p16 = t[n].astype(np.float16)
    rec[n] = (n, G.F16, [st, tctx], p16)
    want[n] = p16.astype(np.float32)
    n = "decoder.ln.weight"
    rec[n] = (n, G.F32, [st // 2, 2], t[n])
    want[n] = _f16(t[n])
    n = "decoder.ln.bias"
    rec[n] = (n, G.F32, [1, st], t[n])
    assert not np.array_equal(_f16(t[n]), t[n])  # float16 rounding would show
    records = _encoder_records(hp) + list(rec.values())
    return records, want


@pytest.fixture(scope="module")
def model_file(orc, tmp_path_factory):
    records, want = _model_file(orc)
    path = tmp_path_factory.mktemp("ggml") / "model.bin"
    G.write(path, G.whisper_file_hparams(HP), records)
    return path, records, want


def test_load_decode_bit_exact(kern, orc, model_file):
    from gorelaxor_amd.whisper import WhisperDecoder

    path, _, want = model_file
    dec = WhisperDecoder.from_ggml(path)
    assert dec.hp == HP
    enc = encoder_output(HP, seed=4)
    ref = orc.WhisperOracle(HP, want)
    ref.set_encoder_output(enc)
    dec.set_encoder_output(enc)
    toks = [50257, 17, 3, 51000]
    lr = ref.decode(toks)
    lg, nxt = dec.decode(toks)
    assert np.array_equal(lg.view(np.uint32), lr.view(np.uint32)), f"max |diff| {np.abs(lg - lr).max()}"
    assert nxt == orc.argmax(lr)
    for step in range(3):
        lr = ref.decode([nxt])
        lg, nxt2 = dec.decode([nxt])
        assert np.array_equal(lg.view(np.uint32), lr.view(np.uint32)), step
        nxt = nxt2
    dec.close()


def test_load_streams_greedy(kern, orc, model_file):
    """The same file into a two-stream decoder: each stream's tokens are the
    oracle's greedy tokens for its encoder output."""
    from gorelaxor_amd.whisper import WhisperDecoder

    path, _, want = model_file
    dec = WhisperDecoder.from_ggml(path, streams=2)
    prompts = np.array([[50257, 5, 9], [50257, 7, 2]], np.int32)
    for s in range(2):
        dec.set_encoder_output_stream(s, encoder_output(HP, seed=20 + s))
    got = dec.greedy_streams(prompts, 5)
    for s in range(2):
        ref = orc.WhisperOracle(HP, want)
        ref.set_encoder_output(encoder_output(HP, seed=20 + s))
        assert list(got[s]) == list(ref.greedy(prompts[s], 5)), s
    dec.close()


def _bad(records, name, new=None):
    out = [r for r in records if r[0] != name]
    if new is not None:
        out.append(new)
    return out


@pytest.mark.parametrize("case", ["magic", "dims", "missing", "unknown", "shape", "type", "cut", "mels"])
def test_load_errors(kern, orc, model_file, tmp_path, case):
    """Bad files fail with the reference's messages (model.go:117-219, 300-404)."""
    from gorelaxor_amd import GrxError
    from gorelaxor_amd.whisper import WhisperDecoder

    _, records, _ = model_file
    st = HP["n_state"]
    hp = G.whisper_file_hparams(HP)
    kw = {}
    msg = {
        "magic": "not a Whisper model file",
        "dims": "dimensions aren't ones this program knows",
        "missing": "the model file has no tensor decoder.ln.bias",
        "unknown": "doesn't know: decoder.extra",
        "shape": "tensor decoder.blocks.0.mlp.0.weight has the wrong shape",
        "type": r"weight type \(5\)",
        "cut": "cut short",
        "mels": "not a Whisper model file",
    }[case]
    if case == "magic":
        kw["magic"] = 0x67676D6D
    elif case == "dims":
        hp[0] = 51000
    elif case == "missing":
        records = _bad(records, "decoder.ln.bias")
    elif case == "unknown":
        records = records + [("decoder.extra", G.F32, [st], np.zeros(st, np.float32))]
    elif case == "shape":  # rows and columns swapped: the same count, ne[0] wrong
        n = "decoder.blocks.0.mlp.0.weight"
        data = [r for r in records if r[0] == n][0][3]
        records = _bad(records, n, (n, G.Q8_0, [4 * st, st], data))
    elif case == "type":
        records = records + [("decoder.extra", 5, [st], np.zeros(st // 32 * 20, np.uint8))]
    elif case == "cut":
        kw["truncate"] = 100
    elif case == "mels":
        kw["n_mels"] = 40
    path = tmp_path / "bad.bin"
    G.write(path, hp, records, **kw)
    with pytest.raises(GrxError, match=msg):
        WhisperDecoder.from_ggml(path)
