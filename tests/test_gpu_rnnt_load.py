"""grx_rnnt_load_gguf: the transducer head of a FastConformer GGUF file
(conformer/model.go:191-235, 306-315) read into the GPU.  The file is laid
out as the reference's converter writes it (tools/convert_nemo.py:686-694:
LSTM and joint matrices Q8_0, the summed LSTM biases and the embedding
float32, settings under stt.parakeet.*); decoding from the loaded head must
be bit-identical to the oracle's over the same tensors, and bad files must
fail with the reference's texts."""
import numpy as np
import pytest

from gorelaxor_amd import GrxError, synth
from tests import _gguf as G

pytestmark = pytest.mark.gpu

TDT = dict(synth.RNNT_TINY, head_kind="tdt", durations=[0, 1, 2, 3], max_symbols=4, joint_act="tanh")


def _settings(hp, **over):
    q = "stt.parakeet."
    s = {"general.architecture": (G.T_STR, "parakeet"), q + "encoder.d_model": (G.T_U32, hp["d"]),
         q + "head_kind": (G.T_STR, hp["head_kind"]), q + "predictor.vocab": (G.T_U32, hp["pred_vocab"]),
         q + "predictor.hidden": (G.T_U32, hp["pred_hidden"]), q + "predictor.n_layers": (G.T_U32, hp["pred_layers"]),
         q + "joint.hidden": (G.T_U32, hp["joint_hidden"]), q + "joint.activation": (G.T_STR, hp["joint_act"]),
         q + "tdt.max_symbols": (G.T_U32, hp.get("max_symbols", 10))}
    durs = over.pop("durations", hp.get("durations"))
    s.update(over)
    kvs = [G.kv(k, t, v) for k, (t, v) in s.items() if t is not None]
    if durs:
        kvs.append(G.kv(q + "tdt.durations", G.T_ARR, list(durs), G.T_I32))
    return kvs


def _tensors(hp, t):
    H, J, V, d = hp["pred_hidden"], hp["joint_hidden"], hp["pred_vocab"], hp["d"]
    nd = len(hp.get("durations", [])) if hp["head_kind"] == "tdt" else 0
    shapes = {"joint.enc.weight": (J, d), "joint.pred.weight": (J, H), "joint.out.weight": (V + nd, J)}
    out = []
    for name, a in t.items():
        if a.dtype == np.uint8:
            rows, cols = shapes.get(name, (4 * H, H))
            out.append((name, [cols, rows], G.Q8_0, a.tobytes()))
        elif name == "pred.embed.weight":
            out.append((name, [H, a.size // H], G.F32, a.tobytes()))
        else:
            out.append((name, [a.size], G.F32, a.tobytes()))
    return out


@pytest.mark.parametrize("hp", [synth.RNNT_TINY, TDT], ids=["rnnt", "tdt"])
def test_load_decode_bit_exact(kern, orc, tmp_path, hp):
    from gorelaxor_amd.rnnt import TransducerDecoder

    t = synth.rnnt_model(hp, seed=41)
    path = tmp_path / "head.gguf"
    path.write_bytes(G.build(_settings(hp), _tensors(hp, t)))
    dec = TransducerDecoder.from_gguf(str(path))
    assert dec.hp["head_kind"] == hp["head_kind"] and dec.hp["blank"] == hp["pred_vocab"] - 1
    enc = synth.rnnt_encoder_output(hp, 40, seed=42)
    want, _ = orc.RnntOracle(hp, t).decode(enc)
    got = dec.decode(enc)
    assert [(g.ID, g.Frame, g.Duration, np.float32(g.P).tobytes()) for g in got] == \
        [(w[0], w[1], w[2], np.float32(w[3]).tobytes()) for w in want]
    dec.close()


@pytest.mark.parametrize("case,msg", [
    ("arch", "not a FastConformer transducer"),
    ("ctc", "not supported"),
    ("no_durations", "needs its durations"),
    ("max_symbols", "out of range"),
    ("no_vocab", "missing its decoder settings"),
    ("missing", "has no joint.pred.bias"),
    ("shape", "doesn't fit its own settings"),
])
def test_load_errors(kern, tmp_path, case, msg):
    from gorelaxor_amd.rnnt import TransducerDecoder

    hp = TDT
    t = synth.rnnt_model(hp, seed=43)
    over = {}
    tens = _tensors(hp, t)
    if case == "arch":
        over["general.architecture"] = (G.T_STR, "whisper")
    elif case == "ctc":
        over["stt.parakeet.head_kind"] = (G.T_STR, "ctc")
    elif case == "no_durations":
        over["durations"] = []
    elif case == "max_symbols":
        over["stt.parakeet.tdt.max_symbols"] = (G.T_U32, 101)
    elif case == "no_vocab":
        over["stt.parakeet.predictor.vocab"] = (None, None)
    elif case == "missing":
        tens = [x for x in tens if x[0] != "joint.pred.bias"]
    elif case == "shape":  # joint.pred stored transposed-wide: right bytes, wrong shape
        H, J = hp["pred_hidden"], hp["joint_hidden"]
        tens = [(n, [2 * J, H // 2] if n == "joint.pred.weight" else dims, ty, b) for n, dims, ty, b in tens]
    path = tmp_path / f"{case}.gguf"
    path.write_bytes(G.build(_settings(hp, **over), tens))
    with pytest.raises(GrxError, match=msg):
        TransducerDecoder.from_gguf(str(path))
