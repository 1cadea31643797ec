"""The host-side tables built with C's libm (exp, log, sin, cos) where the
reference calls Go's math package: the rotary angles of the pocket flow LM
and the Mimi transformer (ropeFreqs/applyRope, pockettts/nn.go:66-93) and the
conformer's relative-position table (relPosRange, conformer/encoder.go:
171-191).  Each library returns results within an ulp or two of the exact
value in float64.  These tests show that at the configurations' sizes every
float32 the tables hold (and every float32 on the way) is the same for ANY
float64 result within ULPS ulps of numpy's, so C's libm and Go's math give
identical tables and the device's tables equal the reference's."""
import math

import numpy as np

from gorelaxor_amd.synth import MIMI, POCKET_TTS_LM

ULPS = 8  # window around numpy's float64 result, both ways


def _window(v: np.ndarray):
    lo, hi = v.copy(), v.copy()
    for _ in range(ULPS):
        lo = np.nextafter(lo, -np.inf)
        hi = np.nextafter(hi, np.inf)
    return lo, hi


def _same_f32(v: np.ndarray) -> np.ndarray:
    """Per entry: every float64 within the window rounds to one float32."""
    lo, hi = _window(np.asarray(v, np.float64))
    return lo.astype(np.float32) == hi.astype(np.float32)


def _rope_freqs_robust(hd: int, period: float) -> np.ndarray:
    # c = f32(-ln(period) * 2 / hd): the products by 2 and 1/hd (powers of
    # two here) are exact, so the window on ln carries over to c
    assert hd & (hd - 1) == 0
    ln = np.float64(math.log(period))
    assert _same_f32(np.array([-ln * 2 / hd])).all(), "f32(c) depends on the last bits of ln(period)"
    c = np.float32(-ln * 2 / hd)
    t = np.arange(hd // 2, dtype=np.float32) * c  # float32 products, as the reference forms them
    e = np.exp(t.astype(np.float64))
    assert _same_f32(e).all(), "a rotary frequency depends on the last bits of exp"
    return e.astype(np.float32)


def _rope_angles_robust(f: np.ndarray, positions: int) -> None:
    p = np.arange(positions, dtype=np.float32)[:, None]
    a = (f[None, :] * p).astype(np.float64)  # f32(f_i * pos), widened
    for fn, name in ((np.cos, "cos"), (np.sin, "sin")):
        ok = _same_f32(fn(a))
        assert ok.all(), f"{name} of {np.count_nonzero(~ok)} angles depends on its last bits: {a[~ok][:4]}"


def test_pocket_lm_rope_table():
    """Heads of 64 (d 1024, 16 heads), period 1e4, every position the flow
    LM holds (max_pos 320)."""
    hp = dict(POCKET_TTS_LM)
    f = _rope_freqs_robust(hp["d"] // hp["heads"], hp["period"])
    _rope_angles_robust(f, hp["max_pos"])


def test_mimi_rope_table():
    """Heads of 64 (d 512, 8 heads), period 1e4, positions up to 8192 (the
    angles of a long decode; the transformer's context is 250 rows)."""
    hp = dict(MIMI)
    f = _rope_freqs_robust(hp["d"] // hp["heads"], hp["period"])
    _rope_angles_robust(f, 8192)


def test_conformer_rel_pos_table():
    """d 1024, relative positions -1024..1024 (offline encodes of 126 rows use
    -125..125; streaming chunk steps a left context of 70 plus the chunk)."""
    d = 1024
    ln = np.float64(math.log(10000.0))
    lo_ln, hi_ln = _window(np.array([ln]))
    j = np.arange(0, d, 2, dtype=np.float64)
    div = None
    # div_j = f32(exp(j * -(ln / d))): the window on ln and on exp together
    for lnv in (lo_ln[0], ln, hi_ln[0]):
        x = j * -(lnv / d)
        lo, hi = _window(np.exp(x))
        a, b = lo.astype(np.float32), hi.astype(np.float32)
        assert np.array_equal(a, b), "a frequency depends on the last bits of exp"
        assert div is None or np.array_equal(div, a), "a frequency depends on the last bits of ln(10000)"
        div = a
    pos = np.arange(1024, -1025, -1, dtype=np.float32)[:, None]
    ang = (pos * div[None, :]).astype(np.float64)  # f64(f32(pos) * div)
    for fn, name in ((np.sin, "sin"), (np.cos, "cos")):
        ok = _same_f32(fn(ang))
        assert ok.all(), f"{name} of {np.count_nonzero(~ok)} angles depends on its last bits: {ang[~ok][:4]}"


def test_window_catches_a_float32_boundary():
    """The check itself: a float64 value on a float32 rounding boundary (the
    midpoint 1 + 2^-24), or within ULPS ulps of it, is flagged; one a quarter
    of a float32 ulp away is not."""
    mid = 1.0 + 2.0 ** -24
    near = np.nextafter(np.nextafter(mid, 2.0), 2.0)
    v = np.array([mid, near, 1.0 + 2.0 ** -25, -mid])
    assert list(_same_f32(v)) == [False, False, True, False]
