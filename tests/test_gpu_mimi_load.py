"""grx_mimi_load_gguf: the Mimi decoder of a Pocket TTS GGUF file read into
the GPU (the Mimi part of pockettts.Load, pockettts/model.go:201-213 and
280-308, with decoder() and resBlocks(), model.go:140-181).  The file is laid
out as the reference's converter writes it (matrices of at least 64 x 64 in
whole Q8_0 blocks Q8_0, the rest float32, settings under pockettts.*), with
tensors of the parts the loader does not read (the flow LM) beside them; the
loaded decoder's audio must be bit-identical to the oracle's over the same
tensors, and bad files must fail with the reference's texts."""
import numpy as np
import pytest

from gorelaxor_amd._lib import GrxError
from gorelaxor_amd.synth import MIMI, MIMI_TINY, mimi_latents, mimi_model, mimi_steps
from tests import _gguf as G

pytestmark = pytest.mark.gpu


def _same(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def _hop(hp):
    h = hp["up_s"]
    for r in hp["ratios"]:
        h *= r
    return h


def _settings(hp, **over):
    """The Mimi settings as model.go:201-213, 280-293 reads them; the frame
    size (sample_rate / frame_rate) is upsample x the ratios."""
    s = {"general.architecture": (G.T_STR, "pockettts"), "general.source.sha256": (G.T_STR, "cd" * 32),
         "pockettts.latent_dim": (G.T_U32, hp["ldim"]), "pockettts.sample_rate": (G.T_U32, 24000),
         "pockettts.frame_rate": (G.T_F32, 24000.0 / _hop(hp)),
         "pockettts.mimi.d_model": (G.T_U32, hp["d"]), "pockettts.mimi.heads": (G.T_U32, hp["heads"]),
         "pockettts.mimi.ff": (G.T_U32, hp["ff"]), "pockettts.mimi.context": (G.T_U32, hp["context"]),
         "pockettts.mimi.max_period": (G.T_F32, hp["period"]), "pockettts.mimi.upsample": (G.T_U32, hp["up_s"]),
         "pockettts.seanet.ratios": (G.T_ARR, (G.T_I32, list(hp["ratios"]))),
         "pockettts.seanet.n_filters": (G.T_U32, hp["nf"]), "pockettts.seanet.dimension": (G.T_U32, hp["d"]),
         "pockettts.seanet.kernel_size": (G.T_U32, hp["k"]),
         "pockettts.seanet.residual_kernel_size": (G.T_U32, hp["res_k"]),
         "pockettts.seanet.last_kernel_size": (G.T_U32, hp["last_k"]),
         "pockettts.seanet.dilation_base": (G.T_U32, hp["dil_base"]),
         "pockettts.seanet.compress": (G.T_U32, hp["compress"]),
         "pockettts.seanet.n_residual_layers": (G.T_U32, hp["n_res"])}
    s.update(over)
    out = []
    for k, (t, v) in s.items():
        if t is None:
            continue
        out.append(G.kv(k, t, v[1], v[0]) if t == G.T_ARR else G.kv(k, t, v))
    return out


def _shapes(hp):
    """rows x cols of every matrix the decoder reads (model.go:128-181)."""
    d, ff, ld = hp["d"], hp["ff"], hp["ldim"]
    sh = {"mimi.quant": (d, ld)}
    for i in range(hp["n_layer"]):
        p = f"mimi.dec_tf.{i}."
        sh.update({p + "attn_qkv.weight": (3 * d, d), p + "attn_out.weight": (d, d), p + "ff1.weight": (ff, d),
                   p + "ff2.weight": (d, ff)})
    for kind, name, _, cin, cout, k, _, _ in mimi_steps(hp):
        if kind == "conv":
            sh[name + ".weight"] = (cout, k * cin)
        elif kind == "convtr":
            sh[name + ".weight"] = (k * cout, cin)
        else:
            sh[name + ".1.weight"] = (cout, k * cin)
            sh[name + ".3.weight"] = (cin, cout)
    return sh


def _tensors(hp, t):
    """(name, dims, type, bytes) in GGUF order: dims[0] the row length."""
    sh = _shapes(hp)
    out = []
    for name, a in t.items():
        if name in sh:
            rows, cols = sh[name]
            out.append((name, [cols, rows], G.Q8_0 if a.dtype == np.uint8 else G.F32, a.tobytes()))
        else:
            out.append((name, [a.size], G.F32, a.tobytes()))
    # a part of the model this loader leaves to the others (the flow LM)
    out.append(("lm.bos", [hp["ldim"]], G.F32, np.zeros(hp["ldim"], np.float32).tobytes()))
    return out


def _write(path, hp, t, settings=None, tensors=None):
    path.write_bytes(G.build(settings if settings is not None else _settings(hp),
                             tensors if tensors is not None else _tensors(hp, t)))
    return path


@pytest.mark.parametrize("shape", ["tiny", "english_2026-09"])
def test_load_and_decode_bit_exact(kern, orc, tmp_path, shape):
    """The loaded decoder's settings are the file's and its audio, latent by
    latent across calls, is the oracle's to the bit."""
    from gorelaxor_amd.mimi import MimiDecoder

    hp = dict(MIMI_TINY if shape == "tiny" else MIMI)
    t = mimi_model(hp, seed=21, q8=True)
    p = _write(tmp_path / "m.gguf", hp, t)
    dec = MimiDecoder.from_gguf(p, max_latents=2)
    for k in ("d", "heads", "ff", "n_layer", "context", "ldim", "up_s", "nf", "k", "res_k", "last_k", "dil_base",
              "compress", "n_res"):
        assert dec.hp[k] == hp[k], k
    assert tuple(dec.hp["ratios"]) == tuple(hp["ratios"]) and dec.hp["period"] == hp["period"]
    assert dec.samples_per_latent == _hop(hp)
    ref = orc.MimiOracle(hp, t)
    n = 8 if shape == "tiny" else 3
    lat = mimi_latents(hp, n, seed=22)
    for i in range(n):
        assert _same(dec.decode(lat[i:i + 1]), ref.decode(lat[i:i + 1])), f"latent {i}"
    dec.close()


def _case(case, hp, t):
    tens = _tensors(hp, t)
    sets = None
    if case == "arch":
        sets = _settings(hp, **{"general.architecture": (G.T_STR, "whisper")})
    elif case == "source":
        sets = _settings(hp, **{"general.source.sha256": (None, None)})
    elif case == "ratio_range":
        sets = _settings(hp, **{"pockettts.seanet.ratios": (G.T_ARR, (G.T_I32, [0, 6]))})
    elif case == "ratios_frame":
        sets = _settings(hp, **{"pockettts.seanet.ratios": (G.T_ARR, (G.T_I32, [3, 2, 2]))})
    elif case == "setting":
        sets = _settings(hp, **{"pockettts.mimi.context": (None, None)})
    elif case == "frame_rate":
        sets = _settings(hp, **{"pockettts.frame_rate": (G.T_F32, 7.0)})
    elif case == "heads":
        sets = _settings(hp, **{"pockettts.mimi.heads": (G.T_U32, 3)})
    elif case == "no_layers":
        tens = [x for x in tens if not x[0].startswith("mimi.dec_tf.")]
    elif case == "shape":
        tens = [(n, ([16, d[1]] if n == "mimi.quant" else d), ty, (b if n != "mimi.quant" else
                 np.zeros(16 * hp["d"], np.float32).tobytes())) for n, d, ty, b in tens]
    elif case == "missing_vec":
        tens = [x for x in tens if x[0] != "mimi.dec_tf.1.ls2"]
    elif case == "missing_conv":
        tens = [x for x in tens if x[0] != "mimi.dec.4.3.weight"]
    return sets, tens


@pytest.mark.parametrize("case,text", [
    ("arch", "isn't a Pocket TTS model"),
    ("source", "pockettts: the file doesn't name its source"),
    ("ratio_range", "pockettts: a SEANet ratio of 0"),
    ("ratios_frame", "pockettts: SEANet's ratios [3 2 2] don't make 24-sample frames"),
    ("setting", "pockettts: the setting pockettts.mimi.context is -1"),
    ("frame_rate", "pockettts: a frame rate of 7"),
    ("heads", "pockettts: 64 values don't split into 3 heads"),
    ("no_layers", "pockettts: no mimi.dec_tf layers"),
    ("shape", "pockettts: mimi.quant is 64x16, want 64x32"),
    ("missing_vec", "pockettts: no 64-value mimi.dec_tf.1.ls2"),
    ("missing_conv", "mimi.dec.4.3.weight"),
])
def test_bad_files_fail_with_the_reference_texts(kern, tmp_path, case, text):
    """Each malformed file fails to load, naming what the reference's loader
    names, and leaves nothing behind."""
    from gorelaxor_amd.mimi import MimiDecoder

    hp = dict(MIMI_TINY)
    t = mimi_model(hp, seed=23, q8=True)
    sets, tens = _case(case, hp, t)
    p = _write(tmp_path / f"{case}.gguf", hp, t, sets, tens)
    with pytest.raises(GrxError) as e:
        MimiDecoder.from_gguf(p)
    assert text in str(e.value), str(e.value)
