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


@pytest.mark.parametrize("prefix", [1, 3, 4, 16, 17, 20, 33])
def test_prefix_and_frames_bit_exact(kern, orc, prefix):
    """T < 4 (AddScaled), 4 <= T <= 16 (gemvRows), T > 16 (6x16 panels and
    gemv rows) for the prefix; every whole group of 8 rows of a product in
    one launch (16: two groups, 33: four and a last row); then
    teacher-forced frames."""
    _prefix_and_frames(orc, prefix)


def test_long_prefix(kern, orc):
    """A prefix of 150 rows (keys past one wave's 64 lanes, softmax rows of
    up to 150 scores): the output and the frames after it are the
    oracle's."""
    hp = dict(POCKET_TTS_TINY, max_pos=200)
    ref, lm = _pair(orc, hp, seed=12)
    x, lat = pocket_inputs(hp, 3, prefix=150, seed=13)
    assert _same(lm.run(x), ref.run(x))
    outs, eos = lm.frames(lat)
    for k in range(lat.shape[0]):
        wo, we = ref.step(lat[k])
        assert _same(outs[k], wo) and _same(eos[k], we), k


def test_frames_general_gemv_kernel(kern, orc):
    """The same with one-row products on the general kernel (GEMV1=0)."""
    with kern.tuned(GEMV1=0):
        _prefix_and_frames(orc, 3)


@pytest.mark.parametrize("rows", [8, 16, 32, 64])
def test_frames_each_row_slice(kern, orc, rows):
    """The frames with one-row products on slices of 8, 16 or 32 rows of
    each tile (GEMV1_ROWS; 64 = whole tiles): the rotary q|k|v epilogue
    (pairs in adjacent lanes), the float64 LayerNorm prologue, the rounded
    GELU: bit-identical."""
    with kern.tuned(GEMV1_ROWS=rows):
        _prefix_and_frames(orc, 3)


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
    """d 1024, 16 heads, 6 layers, FFN 4096: a 64-row prefix, then the
    configuration's 250 frames (the cache grows from 64 to 314 positions),
    every frame's output and eos logit bit-identical."""
    hp = dict(POCKET_TTS_LM)
    ref, lm = _pair(orc, hp, seed=5)
    x, lat = pocket_inputs(hp, 250, prefix=64, seed=6)
    assert _same(lm.run(x), ref.run(x))
    outs, eos = lm.frames(lat)
    assert lm.pos == 314
    for k in range(250):
        wo, we = ref.step(lat[k])
        assert _same(outs[k], wo) and _same(eos[k], we), k


def _speak_pair(orc, hp, fhp, seed, q8=True):
    from gorelaxor_amd.pocket import PocketLM
    from gorelaxor_amd.synth import pocket_flow_model

    t = pocket_model(hp, seed=seed)
    ft = pocket_flow_model(hp, fhp, seed=seed + 1, q8=q8)
    lm = PocketLM(hp, t)
    lm.flow_init(fhp["dim"], fhp["depth"], fhp["steps"])
    for k, v in ft.items():
        lm.set_tensor(k, v)
    return lm, orc.PocketOracle(hp, t), orc.PocketFlowOracle(hp, fhp["dim"], fhp["depth"], fhp["steps"], ft)


def _speak_check(lm, ref, flow, hp, prefix, frames, seed, chunks=1):
    x, _ = pocket_inputs(hp, 1, prefix=prefix, seed=seed)
    assert _same(lm.run(x), ref.run(x))
    noise = np.random.default_rng(seed).standard_normal((frames, hp["ldim"])).astype(np.float32) * np.float32(0.7)
    got_l, got_e = [], []
    latent = None
    for part in np.array_split(np.arange(frames), chunks):
        lat, eos = lm.speak(noise[part], first_latent=latent)
        got_l.append(lat)
        got_e.append(eos)
        latent = lat[-1]
    got_l, got_e = np.concatenate(got_l), np.concatenate(got_e)
    latent = None
    for k in range(frames):
        h, e = ref.step(latent)
        nxt = flow.sample(h, noise[k])
        assert _same(got_e[k], e), f"frame {k}: eos {got_e[k]} vs {e}"
        assert _same(got_l[k], nxt), f"frame {k}: max |diff| {np.abs(got_l[k] - nxt).max()}"
        latent = nxt


@pytest.mark.parametrize("q8", [True, False])
def test_speak_frames_with_flow_head_bit_exact(kern, orc, q8):
    """speakChunk's loop on the device: each frame's transformer step fed the
    previous frame's sampled latent, the flow head (two LSD steps, two
    residual blocks) from its output and the frame's noise - latents and
    end-of-speech logits bit-identical, over two calls that continue one
    another; the flow matrices Q8_0 as converted files hold them, or all
    float32."""
    from gorelaxor_amd.synth import POCKET_FLOW_TINY

    hp, fhp = dict(POCKET_TTS_TINY), dict(POCKET_FLOW_TINY)
    lm, ref, flow = _speak_pair(orc, hp, fhp, seed=13, q8=q8)
    _speak_check(lm, ref, flow, hp, prefix=5, frames=7, seed=14, chunks=2)


def test_speak_configured_shape(kern, orc):
    """d 1024 transformer with a 512-wide, 6-block flow head (one LSD step):
    a 64-row prefix, then 12 frames, bit-identical."""
    from gorelaxor_amd.synth import POCKET_FLOW

    hp, fhp = dict(POCKET_TTS_LM), dict(POCKET_FLOW)
    lm, ref, flow = _speak_pair(orc, hp, fhp, seed=15)
    _speak_check(lm, ref, flow, hp, prefix=64, frames=12, seed=16)
