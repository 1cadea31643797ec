"""The pocket-TTS flow-LM transformer on the GPU against the CPU oracle:
the text prefix's out_norm output and every frame's output and
end-of-speech logit bit-identical, at a small shape (prefix lengths that
take each of MatMulF32's routes) and at the configured shape (d 1024, 16
heads, 6 layers, FFN 4096, 64-row prefix)."""
import os

import numpy as np
import pytest

from gorelaxor_amd.synth import POCKET_TTS_LM, POCKET_TTS_TINY, pocket_inputs, pocket_model

pytestmark = pytest.mark.gpu


def _same(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def _pair(orc, hp, seed=5):
    from gorelaxor_amd.pocket import PocketLM

    t = pocket_model(hp, seed=seed)
    return orc.PocketOracle(hp, t), PocketLM(hp, t)


@pytest.mark.parametrize("prefix", [1, 3, 4, 16, 17, 20])
def test_prefix_and_frames_bit_exact(kern, orc, prefix):
    """T < 4 (AddScaled), 4 <= T <= 16 (gemvRows), T > 16 (6x16 panels and
    gemv rows) for the prefix; then teacher-forced frames."""
    _prefix_and_frames(orc, prefix)


def test_frames_general_gemv_kernel(kern, orc):
    """The same with one-row products on the general kernel (GRX_GEMV1=0)."""
    os.environ["GRX_GEMV1"] = "0"
    try:
        _prefix_and_frames(orc, 3)
    finally:
        del os.environ["GRX_GEMV1"]


def _prefix_and_frames(orc, prefix):
    hp = dict(POCKET_TTS_TINY)
    ref, lm = _pair(orc, hp)
    x, lat = pocket_inputs(hp, 8, prefix=prefix, seed=prefix)
    want = ref.run(x)
    got = lm.run(x)
    assert _same(got, want), f"prefix: max |diff| {np.abs(got - want).max()}"
    outs, eos = lm.frames(lat)
    for k in range(lat.shape[0]):
        wo, we = ref.step(lat[k])
        assert _same(outs[k], wo), f"frame {k}: max |diff| {np.abs(outs[k] - wo).max()}"
        assert _same(eos[k], we), f"frame {k}: eos {eos[k]} vs {we}"
    assert lm.pos == ref.pos == prefix + 8


def test_frames_in_two_calls_and_bos(kern, orc):
    """Frames split over calls continue the same state; a frame without a
    latent takes the bos input (lm.go:186-188)."""
    hp = dict(POCKET_TTS_TINY)
    ref, lm = _pair(orc, hp, seed=8)
    x, lat = pocket_inputs(hp, 6, prefix=10, seed=2)
    ref.run(x)
    lm.run(x)
    o1, e1 = lm.frames(None, 1)
    wo, we = ref.step(None)
    assert _same(o1[0], wo) and _same(e1[0], we)
    o2, e2 = lm.frames(lat[:3])
    o3, e3 = lm.frames(lat[3:])
    for k in range(6):
        wo, we = ref.step(lat[k])
        got_o, got_e = (o2[k], e2[k]) if k < 3 else (o3[k - 3], e3[k - 3])
        assert _same(got_o, wo) and _same(got_e, we), k


def test_context_limit(kern, orc):
    from gorelaxor_amd import GrxError
    from gorelaxor_amd.pocket import PocketLM

    hp = dict(POCKET_TTS_TINY)
    lm = PocketLM(hp, pocket_model(hp))
    with pytest.raises(GrxError, match="exceed"):
        lm.run(np.zeros((hp["max_pos"] + 1, hp["d"]), np.float32))
    with pytest.raises(GrxError, match="wrong shape"):
        PocketLM(hp).set_tensor("lm.bos", np.zeros(3, np.float32))


def test_configured_shape(kern, orc):
    """d 1024, 16 heads, 6 layers, FFN 4096: a 64-row prefix, then 24
    frames, bit-identical."""
    hp = dict(POCKET_TTS_LM)
    ref, lm = _pair(orc, hp, seed=5)
    x, lat = pocket_inputs(hp, 24, prefix=64, seed=6)
    assert _same(lm.run(x), ref.run(x))
    outs, eos = lm.frames(lat)
    for k in range(24):
        wo, we = ref.step(lat[k])
        assert _same(outs[k], wo) and _same(eos[k], we), k
