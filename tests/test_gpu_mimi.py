"""Pocket-TTS's Mimi decoder on the GPU against the CPU oracle, bit for bit:
latents decoded one per call as the speak loop decodes them (pockettts/
speak.go:177-189), the stream's carries (the upsampling overlap, the
transformer's cache and context window, each convolution's past rows and
each transposed convolution's partial) across calls; several latents per
call; float32 and Q8_0 weights (the converter's typing); the
english_2026-09 shape."""
import numpy as np
import pytest

from gorelaxor_amd.synth import MIMI, MIMI_TINY, mimi_latents, mimi_model

pytestmark = pytest.mark.gpu


def _same(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def _pair(orc, hp, t, max_latents=4):
    from gorelaxor_amd.mimi import MimiDecoder

    return orc.MimiOracle(hp, t), MimiDecoder(hp, t, max_latents=max_latents)


@pytest.mark.parametrize("q8", [False, True])
def test_tiny_streamed_bit_exact(kern, orc, q8):
    """Twenty latents one per call (past the 12-position context window
    from the fourth call on): every sample's bits."""
    hp = dict(MIMI_TINY)
    t = mimi_model(hp, seed=15, q8=q8)
    ref, dec = _pair(orc, hp, t)
    lat = mimi_latents(hp, 20, seed=16)
    for i in range(20):
        want = ref.decode(lat[i:i + 1])
        got = dec.decode(lat[i:i + 1])
        assert _same(got, want), f"latent {i}: max |diff| {np.abs(got - want).max()}"
    dec.close()


@pytest.mark.parametrize("mx", [-1, 0])
@pytest.mark.parametrize("per_call", [2, 3, 4])
def test_tiny_several_latents_per_call(kern, orc, per_call, mx):
    """n latents per call (T = 4n rows: the MatMulF32 routes past 16 rows)
    and a reset in between: the oracle's bits.  GEMV_MX=0 sends the groups
    of 8 rows to the dot-product several-row kernel instead of the
    matrix-core one (its rounding prologue, the in-place residual and the
    groups' offsets in one launch)."""
    with kern.tuned(GEMV_MX=mx):
        _several_per_call(orc, per_call)


def _several_per_call(orc, per_call):
    hp = dict(MIMI_TINY)
    t = mimi_model(hp, seed=19, q8=True)
    ref, dec = _pair(orc, hp, t)
    lat = mimi_latents(hp, 12, seed=20)
    for rnd in range(2):
        for i in range(0, 12, per_call):
            want = ref.decode(lat[i:i + per_call])
            got = dec.decode(lat[i:i + per_call])
            assert _same(got, want), f"round {rnd} latents {i}..: max |diff| {np.abs(got - want).max()}"
        ref.reset()
        dec.reset()
    dec.close()


@pytest.mark.parametrize("mx", [-1, 0])
def test_real_shape_bit_exact(kern, orc, mx):
    """The english_2026-09 shape (d 512, 8 heads, SEANet 6/5/4, Q8_0 and
    float32 as the converter types them): 6 latents one per call; also with
    the several-row products on the dot-product kernel (GEMV_MX=0)."""
    with kern.tuned(GEMV_MX=mx):
        _real_shape(orc)


def _real_shape(orc):
    hp = dict(MIMI)
    t = mimi_model(hp, seed=17)
    ref, dec = _pair(orc, hp, t, max_latents=1)
    lat = mimi_latents(hp, 6, seed=18)
    for i in range(6):
        want = ref.decode(lat[i:i + 1])
        got = dec.decode(lat[i:i + 1])
        assert got.shape == (1920,)
        assert _same(got, want), f"latent {i}: max |diff| {np.abs(got - want).max()}"
    dec.close()


def test_errors(kern):
    """Missing tensors, a wrong size, too many latents per call."""
    from gorelaxor_amd.mimi import MimiDecoder
    from gorelaxor_amd._lib import GrxError

    hp = dict(MIMI_TINY)
    t = mimi_model(hp, seed=15)
    dec = MimiDecoder(hp, max_latents=2)
    with pytest.raises(GrxError):
        dec.decode(mimi_latents(hp, 1))
    with pytest.raises(GrxError):
        dec.set_tensor("mimi.up", t["mimi.up"][:-1])
    with pytest.raises(GrxError):
        dec.set_tensor("mimi.nothing", t["mimi.up"])
    for k, v in t.items():
        dec.set_tensor(k, v)
    with pytest.raises(GrxError):
        dec.decode(mimi_latents(hp, 3))
    assert dec.decode(mimi_latents(hp, 2)).shape == (2 * dec.samples_per_latent,)
    dec.close()
