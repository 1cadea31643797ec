"""The flow LM's device state (tstate, pockettts/nn.go:113-140).

A Voice (pockettts/voice.go:26-64) seeds the LM as speakChunk clones it
(speak.go:117): the text prefix and the frames after it must be
bit-identical to the oracle seeded with the same keys and values; seeding
again from the same state must repeat them (speaking leaves the voice
unchanged); the LM's state saved after speaking must hold the oracle's
cache rows bit for bit; and LoadVoice's checks and texts must hold over
crafted GGUF voice files."""
import numpy as np
import pytest

from gorelaxor_amd.synth import POCKET_TTS_TINY, pocket_inputs, pocket_model
from tests import _gguf as G
from tests.test_gpu_pocket_load import _write

pytestmark = pytest.mark.gpu

HP = dict(POCKET_TTS_TINY)
SHA = "ab" * 32


def _same(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def _voice(hp, n, seed):
    rng = np.random.default_rng(seed)
    shape = (hp["n_layer"], n, hp["d"])
    return (rng.standard_normal(shape) * 0.7).astype(np.float32), (rng.standard_normal(shape) * 0.7).astype(np.float32)


def _text_and_frames(lm, ref, x, lat):
    assert _same(lm.run(x), ref.run(x)), "text prefix"
    outs, eos = lm.frames(lat)
    for k in range(lat.shape[0]):
        wo, we = ref.step(lat[k])
        assert _same(outs[k], wo) and _same(eos[k], we), f"frame {k}"
    return outs, eos


@pytest.mark.parametrize("n", [1, 37, 64])
def test_voice_text_frames_bit_exact(kern, orc, n):
    """Seeded from an n-position voice: text, then frames, every output and
    end-of-speech logit bit-identical; seeding again repeats them; the
    state read back is the voice; the LM's state after speaking is the
    oracle's cache, rows and position."""
    from gorelaxor_amd.pocket import PocketLM

    t = pocket_model(HP, seed=11)
    ref = orc.PocketOracle(HP, t)
    lm = PocketLM(HP, t)
    k, v = _voice(HP, n, seed=n)
    st = lm.make_state(k, v)
    assert st.positions == n
    kr, vr = st.read()
    assert _same(kr, k) and _same(vr, v)
    x, lat = pocket_inputs(HP, 8, prefix=5, seed=n + 1)
    ref.set_state(k, v)
    lm.set_state(st)
    assert lm.pos == ref.pos == n
    outs, eos = _text_and_frames(lm, ref, x, lat)
    assert lm.pos == ref.pos == n + 13
    saved = lm.state()
    ks, vs = saved.read()
    rk, rv = ref.state()
    assert saved.positions == n + 13
    assert _same(ks, rk) and _same(vs, rv)
    # the voice is unchanged: a second chunk from it repeats the first
    lm.set_state(st)
    assert lm.pos == n
    x2 = lm.run(x)
    ref.set_state(k, v)
    assert _same(x2, ref.run(x))
    outs2, eos2 = lm.frames(lat)
    assert _same(outs2, outs) and _same(eos2, eos)
    # a saved state seeds as the voice does: continuing from it
    lm.set_state(saved)
    ref.set_state(rk, rv)
    _, lat3 = pocket_inputs(HP, 4, prefix=1, seed=99)
    outs3, _ = lm.frames(lat3)
    for j in range(4):
        assert _same(outs3[j], ref.step(lat3[j])[0]), j
    for s in (st, saved):
        s.close()
    lm.close()


def test_state_limits(kern):
    """A state larger than the LM's context, of another width, or of
    another layer count is refused; an empty state seeds position 0."""
    from gorelaxor_amd import GrxError
    from gorelaxor_amd.pocket import PocketLM

    t = pocket_model(HP, seed=11)
    lm = PocketLM(HP, t)
    big = lm.make_state(*_voice(HP, HP["max_pos"] + 1, seed=1))
    with pytest.raises(GrxError, match="exceed"):
        lm.set_state(big)
    other = PocketLM(dict(HP, n_layer=1), {k: a for k, a in t.items() if ".blk.1." not in k})
    with pytest.raises(GrxError, match="layers"):
        lm.set_state(other.make_state(*_voice(dict(HP, n_layer=1), 4, seed=2)))
    empty = lm.make_state(np.zeros((HP["n_layer"], 0, HP["d"]), np.float32),
                          np.zeros((HP["n_layer"], 0, HP["d"]), np.float32))
    lm.run(np.ones((2, HP["d"]), np.float32))
    lm.set_state(empty)
    assert lm.pos == 0
    for o in (big, empty, other, lm):
        o.close()


def _voice_file(path, hp, k, v, typ=G.F32, **over):
    """A voice file as tools/convert_pocket_tts.py's convert_voice writes
    one: settings, then voice.{i}.k and voice.{i}.v of [positions][d]."""
    nl, n, d = k.shape
    sets = {"general.architecture": (G.T_STR, "pockettts-voice"), "pockettts.voice.model.sha256": (G.T_STR, SHA),
            "pockettts.voice.layers": (G.T_U32, nl), "pockettts.voice.positions": (G.T_U32, n)}
    sets.update({kk: vv for kk, vv in over.items() if not kk.startswith("_")})
    tens = []
    for i in range(nl):
        for c, a in (("k", k[i]), ("v", v[i])):
            data = a.astype(np.float16).tobytes() if typ == G.F16 else a.astype(np.float32).tobytes()
            tens.append((f"voice.{i}.{c}", [d, n], typ, data))
    tens = over.get("_tensors", lambda ts: ts)(tens)
    path.write_bytes(G.build([G.kv(kk, t, vv) for kk, (t, vv) in sets.items() if t is not None], tens))
    return path


@pytest.mark.parametrize("typ", [G.F32, G.F16])
def test_load_voice_and_speak(kern, orc, tmp_path, typ):
    """LoadVoice of a float32 or float16 voice file (widened as File.Float32
    widens it) into an LM loaded from its model file: the positions, the
    values read back, then text and frames bit-identical to the oracle
    seeded with the widened values."""
    from gorelaxor_amd.pocket import PocketLM

    t = pocket_model(HP, seed=5)
    lm = PocketLM.from_gguf(_write(tmp_path / "m.gguf", HP, t), max_pos=HP["max_pos"])
    k, v = _voice(HP, 21, seed=4)
    if typ == G.F16:
        k, v = k.astype(np.float16).astype(np.float32), v.astype(np.float16).astype(np.float32)
    voice = lm.load_voice(_voice_file(tmp_path / "v.gguf", HP, k, v, typ))
    assert voice.positions == 21
    kr, vr = voice.read()
    assert _same(kr, k) and _same(vr, v)
    ref = orc.PocketOracle(HP, t)
    ref.set_state(k, v)
    lm.set_state(voice)
    x, lat = pocket_inputs(HP, 6, prefix=4, seed=8)
    _text_and_frames(lm, ref, x, lat)
    voice.close()
    lm.close()


def _nan(ts):
    name, dims, typ, data = ts[1]
    a = np.frombuffer(data, np.float32).copy()
    a[5] = np.nan
    return [ts[0], (name, dims, typ, a.tobytes())] + ts[2:]


BAD = {
    "arch": ({"general.architecture": (G.T_STR, "pockettts")}, "isn't a Pocket TTS voice"),
    "sha": ({"pockettts.voice.model.sha256": (G.T_STR, "cd" * 32)}, "was made for a different model file"),
    "no_sha": ({"pockettts.voice.model.sha256": (None, None)}, "was made for a different model file"),
    "layers": ({"pockettts.voice.layers": (G.T_U32, 3)}, "holds 3 layers of 12 positions"),
    "zero": ({"pockettts.voice.positions": (G.T_U32, 0)}, "holds 2 layers of 0 positions"),
    "many": ({"pockettts.voice.positions": (G.T_U32, 4097)}, "holds 2 layers of 4097 positions"),
    "missing": ({"_tensors": lambda ts: [r for r in ts if r[0] != "voice.1.v"]}, "has no 12×128 voice.1.v"),
    "dims": ({"_tensors": lambda ts: [(n, [d, 11] if n == "voice.0.v" else [d, p], ty, b) for n, (d, p), ty, b in ts]},
             "has no 12×128 voice.0.v"),
    "nan": ({"_tensors": _nan}, "has values that aren't numbers"),
}


@pytest.mark.parametrize("case", sorted(BAD))
def test_load_voice_errors(kern, tmp_path, case):
    """Each of LoadVoice's checks, in its order, with the reference's text
    (voice.go:33-60)."""
    from gorelaxor_amd import GrxError
    from gorelaxor_amd.pocket import PocketLM

    t = pocket_model(HP, seed=5)
    lm = PocketLM.from_gguf(_write(tmp_path / "m.gguf", HP, t), max_pos=HP["max_pos"])
    k, v = _voice(HP, 12, seed=6)
    over, text = BAD[case]
    p = _voice_file(tmp_path / "v.gguf", HP, k, v, **over)
    with pytest.raises(GrxError, match=text):
        lm.load_voice(p)
    lm.close()


def test_load_voice_of_a_tensor_built_model_is_refused(kern, tmp_path):
    """An LM built from tensors names no model file, so no voice file
    matches it (the reference's model always has its source hash)."""
    from gorelaxor_amd import GrxError
    from gorelaxor_amd.pocket import PocketLM

    lm = PocketLM(HP, pocket_model(HP, seed=5))
    with pytest.raises(GrxError, match="different model file"):
        lm.load_voice(_voice_file(tmp_path / "v.gguf", HP, *_voice(HP, 3, seed=1)))
    lm.close()
