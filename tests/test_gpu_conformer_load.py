"""grx_conformer_load_gguf: the encoder of a FastConformer GGUF file read
into the GPU (conformer.Load, conformer/model.go:163-422).  The file is
laid out as the reference's converter writes it (tools/convert_nemo.py:
linear weights Q8_0, the block's pointwise convolutions float16 in their
[out][in][1] shape, the pre-encoder's conv.3 / conv.6 float32 [out][in][1][1],
taps and vectors float32, settings under stt.parakeet.* and stt.frontend.*);
the loaded encoder's output must be bit-identical to the oracle's over the
same tensors, and bad files must fail with the reference's texts."""
import numpy as np
import pytest

from gorelaxor_amd.synth import CONFORMER_TINY, conformer_model, noise_mel
from tests import _gguf as G

pytestmark = pytest.mark.gpu

HP = dict(CONFORMER_TINY)


def _settings(hp, **over):
    e = "stt.parakeet.encoder."
    s = {"general.architecture": (G.T_STR, "parakeet"),
         e + "d_model": (G.T_U32, hp["d"]), e + "n_heads": (G.T_U32, hp["heads"]),
         e + "n_layers": (G.T_U32, hp["layers"]), e + "d_ff": (G.T_U32, hp["dff"]),
         e + "conv_kernel": (G.T_U32, hp["conv_kernel"]), e + "subsampling_channels": (G.T_U32, hp["sub_channels"]),
         e + "subsampling_factor": (G.T_U32, 8), e + "xscaling": (G.T_BOOL, hp["xscaling"]),
         e + "att_context_style": (G.T_STR, "regular"), e + "conv_norm_type": (G.T_STR, hp["conv_norm"]),
         "stt.parakeet.head_kind": (G.T_STR, "tdt"), "stt.parakeet.predictor.vocab": (G.T_U32, 1025),
         "stt.parakeet.predictor.hidden": (G.T_U32, 640), "stt.parakeet.predictor.n_layers": (G.T_U32, 2),
         "stt.parakeet.joint.hidden": (G.T_U32, 640), "stt.frontend.num_mels": (G.T_U32, hp["n_mels"])}
    no_durations = over.pop("no_durations", False)
    s.update(over)
    kvs = [G.kv(k, t, v) for k, (t, v) in s.items() if t is not None]
    if not no_durations:
        kvs.append(G.kv("stt.parakeet.tdt.durations", G.T_ARR, [0, 1, 2, 3, 4], G.T_I32))
    return kvs


def _tensors(hp, t):
    d, c, K = hp["d"], hp["sub_channels"], hp["conv_kernel"]
    out = []
    for name, a in t.items():
        leaf = name.split(".", 3)[-1] if name.startswith("enc.blocks.") else name[len("enc.pre_encode."):]
        if a.dtype == np.uint8:  # Q8_0 rows x cols
            rows = {"out.weight": d, "ff1.linear1.weight": hp["dff"], "ff2.linear1.weight": hp["dff"]}.get(leaf, d)
            cols = a.size // 34 * 32 // rows
            out.append((name, [cols, rows], G.Q8_0, a.tobytes()))
        elif a.dtype == np.float16:  # a 1x1 convolution [out][in][1]
            rows = 2 * d if leaf == "conv.pointwise1.weight" else d
            out.append((name, [1, d, rows], G.F16, a.tobytes()))
        elif leaf in ("conv.3.weight", "conv.6.weight"):
            out.append((name, [1, 1, c, c], G.F32, a.tobytes()))
        elif leaf in ("conv.0.weight", "conv.2.weight", "conv.5.weight"):
            out.append((name, [3, 3, 1, c], G.F32, a.tobytes()))
        elif leaf == "conv.depthwise.weight":
            out.append((name, [K, 1, d], G.F32, a.tobytes()))
        else:
            out.append((name, [a.size], G.F32, a.tobytes()))
    return out


def _write(path, hp, t, settings=None, tensors=None):
    path.write_bytes(G.build(settings if settings is not None else _settings(hp),
                             tensors if tensors is not None else _tensors(hp, t)))
    return path


@pytest.mark.parametrize("conv_norm", ["batch_norm", "layer_norm"])
def test_load_encode_bit_exact(kern, orc, tmp_path, conv_norm):
    from gorelaxor_amd.conformer import ConformerEncoder

    hp = dict(HP, conv_norm=conv_norm)
    t = conformer_model(hp, seed=41, pointwise_f16=True, pre_f32=True)
    p = _write(tmp_path / "c.gguf", hp, t)
    enc = ConformerEncoder.from_gguf(p)
    assert {k: enc.hp[k] for k in hp} == hp
    assert enc.hp["att_style"] == "regular" and not enc.hp["causal_sub"]
    assert (enc.hp["att_left"], enc.hp["att_right"], enc.hp["conv_left"], enc.hp["conv_right"]) == (-1, -1, -1, -1)
    mel, frames, valid = noise_mel(hp["n_mels"], seconds=1.5, seed=42)
    got, lens = enc.encode(mel[None], [valid])
    want, L = orc.ConformerOracle(hp, t).encode(mel, valid)
    assert lens[0] == L
    assert np.array_equal(got[0].view(np.uint32), want.view(np.uint32)), np.abs(got[0] - want).max()
    enc.close()


def test_load_streaming_model(kern, orc, tmp_path):
    """A cache-aware model's file (readEncoder / readHParams settings:
    chunked_limited attention 28 left, trained right contexts, the causal
    convolution and pre-encoder, the streaming cache settings): the loaded
    encoder streams bit-identically to the oracle."""
    from gorelaxor_amd.conformer import ConformerEncoder, ConformerStream, mel_chunks, stream_geom

    hp = dict(HP, conv_norm="layer_norm", att_style="chunked_limited", att_left=28, att_right=13,
              context_choices=[(28, 13), (28, 1)], conv_left=8, conv_right=0)
    t = conformer_model(hp, seed=43, pointwise_f16=True, pre_f32=True)
    e = "stt.parakeet.encoder."
    sets = _settings(hp, **{e + "att_context_style": (G.T_STR, "chunked_limited"),
                            e + "att_context_left": (G.T_I32, 28), e + "att_context_right": (G.T_I32, 13),
                            e + "conv_context_left": (G.T_I32, 8), e + "conv_context_right": (G.T_I32, 0),
                            e + "streaming.pre_encode_cache_size": (G.T_I32, 9)})
    sets.append(G.kv(e + "att_context_size_choices", G.T_ARR, [28, 13, 28, 1], G.T_I32))
    p = _write(tmp_path / "s.gguf", hp, t, settings=sets)
    enc = ConformerEncoder.from_gguf(p)
    assert enc.hp["att_style"] == "chunked_limited" and enc.hp["causal_sub"]
    assert (enc.hp["att_left"], enc.hp["att_right"], enc.hp["conv_left"], enc.hp["conv_right"]) == (28, 13, 8, 0)
    assert enc.hp["context_choices"] == [(28, 13), (28, 1)] and enc.hp["pre_encode_cache"] == 9
    mel, frames, valid = noise_mel(hp["n_mels"], seconds=3.0, seed=44)
    for right in (1, 13):
        g = stream_geom(hp, right)
        s = ConformerStream(enc, right)
        o = orc.ConformerOracle(hp, t).stream(right, g["left"], g["drop"])
        for j, (ch, n, _) in enumerate(mel_chunks(mel, g)):
            got, want = s.step(ch, n)[0], o.step(ch, n)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (right, j)
        s.close()
    enc.close()


def _case(case, hp, t):
    e = "stt.parakeet.encoder."
    sets, tens = None, _tensors(hp, t)
    if case == "arch":
        sets = _settings(hp, **{"general.architecture": (G.T_STR, "pockettts")})
    elif case == "settings":
        sets = _settings(hp, **{e + "d_model": (None, None)})
    elif case == "subsampling":
        sets = _settings(hp, **{e + "subsampling_factor": (G.T_U32, 4)})
    elif case == "ctc":
        sets = _settings(hp, **{"stt.parakeet.head_kind": (G.T_STR, "ctc")})
    elif case == "durations":
        sets = _settings(hp, no_durations=True)
    elif case == "decoder":
        sets = _settings(hp, **{"stt.parakeet.joint.hidden": (None, None)})
    elif case == "choices":
        sets = _settings(hp)
        sets.append(G.kv(e + "att_context_size_choices", G.T_ARR, [70, 13] * 9, G.T_I32))
    elif case == "missing":
        tens = [r for r in tens if r[0] != "enc.blocks.1.norm_out.bias"]
    elif case == "misfit":  # a linear weight of the wrong size
        n = "enc.blocks.0.ff1.linear1.weight"
        tens = [(n, [hp["d"], hp["dff"] // 2], G.Q8_0, bytes(hp["dff"] // 2 * hp["d"] // 32 * 34)) if r[0] == n
                else r for r in tens]
    elif case == "type":  # a linear weight in float16
        n = "enc.blocks.1.attn.linear_q.weight"
        tens = [(n, [hp["d"], hp["d"]], G.F16, bytes(2 * hp["d"] * hp["d"])) if r[0] == n else r for r in tens]
    return sets, tens


@pytest.mark.parametrize("case, msg", [
    ("arch", 'architecture "pockettts" is not a FastConformer transducer'),
    ("settings", "missing its encoder settings"), ("subsampling", "subsampling 4 is not supported"),
    ("ctc", '"ctc" models are not supported'), ("durations", "a TDT model needs its durations"),
    ("decoder", "missing its decoder settings"), ("choices", "9 attention context choices"),
    ("missing", "the model has no enc.blocks.1.norm_out.bias"),
    ("misfit", r"doesn't fit its own settings \(enc.blocks.0.ff1.linear1.weight is 128x64, want 256x64\)"),
    ("type", "enc.blocks.1.attn.linear_q.weight is type 1"),
])
def test_load_errors(kern, orc, tmp_path, case, msg):
    from gorelaxor_amd import GrxError
    from gorelaxor_amd.conformer import ConformerEncoder

    t = conformer_model(HP, seed=41, pointwise_f16=True, pre_f32=True)
    sets, tens = _case(case, HP, t)
    p = _write(tmp_path / "bad.gguf", HP, t, sets, tens)
    with pytest.raises(GrxError, match=msg):
        ConformerEncoder.from_gguf(p)
