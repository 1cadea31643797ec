"""grx_pocket_load_gguf: the flow LM of a Pocket TTS GGUF file read into the
GPU (pockettts.Load, pockettts/model.go:49-250).  The file is laid out as
the reference's converter writes it (transformer matrices Q8_0, matrices
under 64 columns float32, settings under pockettts.*), with tensors of the
parts this build does not read (Mimi) beside them; the loaded LM's
prefix output, frame outputs and end-of-speech logits must be bit-identical
to the oracle's over the same tensors, and bad files must fail with the
reference's texts."""
import numpy as np
import pytest

from gorelaxor_amd.synth import POCKET_TTS_TINY, pocket_inputs, pocket_model
from tests import _gguf as G

pytestmark = pytest.mark.gpu

HP = dict(POCKET_TTS_TINY)


def _same(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def _settings(hp, **over):
    s = {"general.architecture": (G.T_STR, "pockettts"), "general.source.sha256": (G.T_STR, "ab" * 32),
         "pockettts.latent_dim": (G.T_U32, hp["ldim"]), "pockettts.lm.d_model": (G.T_U32, hp["d"]),
         "pockettts.lm.heads": (G.T_U32, hp["heads"]), "pockettts.lm.ff": (G.T_U32, hp["ff"]),
         "pockettts.lm.layers": (G.T_U32, hp["n_layer"]), "pockettts.lm.max_period": (G.T_F32, hp["period"])}
    s.update(over)
    return [G.kv(k, t, v) for k, (t, v) in s.items() if t is not None]


def _tensors(hp, t):
    """(name, dims, type, bytes) in GGUF order: dims[0] the row length."""
    d, ff, ld = hp["d"], hp["ff"], hp["ldim"]
    cols = {"attn_qkv": d, "attn_out": d, "ff1": d, "ff2": ff}
    out = []
    for name, a in t.items():
        if a.dtype == np.uint8:
            c = cols[name.split(".")[3]]
            out.append((name, [c, a.size // 34 * 32 // c], G.Q8_0, a.tobytes()))
        elif name == "lm.input.weight":
            out.append((name, [ld, d], G.F32, a.tobytes()))
        elif name == "lm.eos.weight":
            out.append((name, [d, 1], G.F32, a.tobytes()))
        else:
            out.append((name, [a.size], G.F32, a.tobytes()))
    # a part of the model this build leaves to the caller (Mimi)
    out.append(("mimi.quant", [ld, 64], G.F32, np.zeros(64 * ld, np.float32).tobytes()))
    return out


def _write(path, hp, t, settings=None, tensors=None):
    path.write_bytes(G.build(settings if settings is not None else _settings(hp),
                             tensors if tensors is not None else _tensors(hp, t)))
    return path


def test_load_run_and_frames_bit_exact(kern, orc, tmp_path):
    from gorelaxor_amd.pocket import PocketLM

    t = pocket_model(HP, seed=5)
    p = _write(tmp_path / "p.gguf", HP, t)
    lm = PocketLM.from_gguf(p, max_pos=HP["max_pos"])
    assert {k: lm.hp[k] for k in ("d", "heads", "ff", "n_layer", "ldim", "max_pos")} == \
        {k: HP[k] for k in ("d", "heads", "ff", "n_layer", "ldim", "max_pos")}
    ref = orc.PocketOracle(HP, t)
    x, lat = pocket_inputs(HP, 6, prefix=17, seed=3)
    assert _same(lm.run(x), ref.run(x))
    outs, eos = lm.frames(lat)
    for k in range(6):
        wo, we = ref.step(lat[k])
        assert _same(outs[k], wo) and _same(eos[k], we), k
    lm.close()


def _case(case, hp, t):
    d, ff = hp["d"], hp["ff"]
    tens = _tensors(hp, t)
    sets = None
    if case == "arch":
        sets = _settings(hp, **{"general.architecture": (G.T_STR, "parakeet")})
    elif case == "source":
        sets = _settings(hp, **{"general.source.sha256": (None, None)})
    elif case == "setting":
        sets = _settings(hp, **{"pockettts.lm.heads": (G.T_U32, 0)})
    elif case == "layers":
        sets = _settings(hp, **{"pockettts.lm.layers": (G.T_U32, 3)})
    elif case == "heads":
        sets = _settings(hp, **{"pockettts.lm.heads": (G.T_U32, 3)})
    elif case == "shape":  # ff1 stored d rows of ff instead of ff rows of d
        tens = [(n, [ff, d] if n == "lm.blk.0.ff1.weight" else dims, ty, b) for n, dims, ty, b in tens]
    elif case == "type":
        tens = [(n, dims, G.F32, np.zeros(d * d, np.float32).tobytes()) if n == "lm.blk.1.attn_out.weight"
                else (n, dims, ty, b) for n, dims, ty, b in tens]
    elif case == "vec":
        tens = [r for r in tens if r[0] != "lm.out_norm.bias"]
    elif case == "mat":
        tens = [r for r in tens if r[0] != "lm.blk.1.ff2.weight"]
    return sets, tens


@pytest.mark.parametrize("case, msg", [
    ("arch", "isn't a Pocket TTS model"), ("source", "doesn't name its source"),
    ("setting", "the setting pockettts.lm.heads is 0"), ("layers", "the flow LM has 2 layers"),
    ("heads", "128 values don't split into 3 heads"), ("shape", "lm.blk.0.ff1.weight is 128x512, want 512x128"),
    ("type", "lm.blk.1.attn_out.weight is type 0"), ("vec", "no 128-value lm.out_norm.bias"),
    ("mat", "gguf: no tensor lm.blk.1.ff2.weight"),
])
def test_load_errors(kern, orc, tmp_path, case, msg):
    from gorelaxor_amd import GrxError
    from gorelaxor_amd.pocket import PocketLM

    t = pocket_model(HP, seed=5)
    sets, tens = _case(case, HP, t)
    p = _write(tmp_path / "bad.gguf", HP, t, sets, tens)
    with pytest.raises(GrxError, match=msg):
        PocketLM.from_gguf(p, max_pos=HP["max_pos"])



def test_load_flow_head_and_speak_bit_exact(kern, orc, tmp_path):
    """A file that also holds the flow head (settings pockettts.flow.dim,
    flow.depth, decode_steps; Q8_0 matrices, float32 input/output
    projections as the converter writes them): loaded, it speaks the
    oracle's latents bit for bit."""
    from gorelaxor_amd.pocket import PocketLM
    from gorelaxor_amd.synth import POCKET_FLOW_TINY, pocket_flow_model

    fhp = dict(POCKET_FLOW_TINY)
    t = pocket_model(HP, seed=5)
    ft = pocket_flow_model(HP, fhp, seed=6)
    recs = _tensors(HP, t)
    for name, a in ft.items():
        if a.dtype == np.uint8:
            cols = HP["d"] if name == "flow.cond.weight" else (256 if ".time." in name and "fc1" in name else fhp["dim"])
            rows = a.size // 34 * 32 // cols
            recs.append((name, [cols, rows], G.Q8_0, a.tobytes()))
        elif name.endswith(".weight") and name in ("flow.input.weight", "flow.final.out.weight"):
            cols = HP["ldim"] if name == "flow.input.weight" else fhp["dim"]
            recs.append((name, [cols, a.size // cols], G.F32, a.tobytes()))
        else:
            recs.append((name, [a.size], G.F32, a.tobytes()))
    sets = _settings(HP, **{"pockettts.flow.dim": (G.T_U32, fhp["dim"]),
                            "pockettts.flow.depth": (G.T_U32, fhp["depth"]),
                            "pockettts.decode_steps": (G.T_U32, fhp["steps"])})
    p = _write(tmp_path / "f.gguf", HP, t, sets, recs)
    lm = PocketLM.from_gguf(p, max_pos=HP["max_pos"])
    ref = orc.PocketOracle(HP, t)
    flow = orc.PocketFlowOracle(HP, fhp["dim"], fhp["depth"], fhp["steps"], ft)
    x, _ = pocket_inputs(HP, 1, prefix=9, seed=3)
    assert _same(lm.run(x), ref.run(x))
    noise = np.random.default_rng(2).standard_normal((5, HP["ldim"])).astype(np.float32)
    lats, eos = lm.speak(noise)
    latent = None
    for k in range(5):
        h, e = ref.step(latent)
        latent = flow.sample(h, noise[k])
        assert _same(lats[k], latent) and _same(eos[k], e), k
    lm.close()
