"""Pins the oracle's Mimi decoder (pockettts/mimi.go, nn.go) without a GPU:
ELU's closed form and its EXP8/expf split, and the streamed decode (one
latent per call, as the speak loop decodes, speak.go:177-189) against an
independent float64 restatement of the whole sequence at once; a dropped
carry (past rows, transposed-conv partial, upsampling overlap, the
transformer's cache or its context window) fails it."""
import numpy as np
import pytest

from gorelaxor_amd.synth import MIMI, MIMI_TINY, mimi_latents, mimi_model
from tests import _mimi_ref


def test_elu_closed_form(orc):
    """x above 0 unchanged; below, e^x - 1 to within a few float32 ulp
    (EXP8 over each 512-value chunk's whole groups of eight, expf past
    them); -0 and 0 give +0."""
    rng = np.random.default_rng(3)
    for n in (8, 13, 512, 515, 1030):
        x = (rng.standard_normal(n) * 4).astype(np.float32)
        x[:2] = [-0.0, 0.0]
        y = orc.elu(x)
        pos = x > 0
        assert np.array_equal(y[pos], x[pos])
        want = np.expm1(x[~pos].astype(np.float64))
        assert np.abs(y[~pos] - want).max() <= 4 * np.finfo(np.float32).eps
        assert np.all(np.signbit(y[:2]) == False)  # noqa: E712


def _streamed(orc, hp, t, lat):
    o = orc.MimiOracle(hp, t)
    return np.concatenate([o.decode(lat[i:i + 1]) for i in range(lat.shape[0])])


@pytest.mark.parametrize("q8", [False, True])
def test_streamed_decode_matches_float64_whole_sequence(orc, q8):
    """The tiny shape (two residual layers per stage, dilation 2, a context
    of 12 positions at 4 rows a latent) over 9 latents: float32 weights on
    the float route within 1e-5 of the float64 restatement's scale; Q8_0
    weights (activations rounded to Q8_0 on the int8 route) within 3e-2."""
    hp = dict(MIMI_TINY)
    t = mimi_model(hp, seed=15, q8=q8)
    lat = mimi_latents(hp, 9, seed=16)
    got = _streamed(orc, hp, t, lat)
    want = _mimi_ref.decode(hp, t, lat)
    err = np.abs(got - want).max() / np.abs(want).max()
    assert err < (3e-2 if q8 else 1e-5), err
    # the tiny shape has few matrices big enough for Q8_0: check the typing
    assert any(v.dtype == np.uint8 for v in t.values()) == q8


def test_dropped_carry_fails_the_pin(orc):
    """The same comparison with each call decoded from a fresh state (no
    carried rows) is far off: the pin sees the carries."""
    hp = dict(MIMI_TINY)
    t = mimi_model(hp, seed=15, q8=False)
    lat = mimi_latents(hp, 9, seed=16)
    want = _mimi_ref.decode(hp, t, lat)
    fresh = np.concatenate([orc.MimiOracle(hp, t).decode(lat[i:i + 1]) for i in range(9)])
    assert np.abs(fresh - want).max() / np.abs(want).max() > 1e-2


def test_real_shape_first_latents(orc):
    """The english_2026-09 shape (Q8_0 as converted): three latents streamed
    against the float64 restatement, within the int8 route's rounding."""
    hp = dict(MIMI)
    t = mimi_model(hp, seed=17)
    lat = mimi_latents(hp, 3, seed=18)
    got = _streamed(orc, hp, t, lat)
    want = _mimi_ref.decode(hp, t, lat)
    assert got.shape == (3 * 1920,)
    assert np.abs(got - want).max() / np.abs(want).max() < 3e-2
