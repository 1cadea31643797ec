"""CPU model of the GPU LayerNorms' parallel sums and of their bound check
(gorelaxor_amd/csrc/grx_ln.h), for tests and for the boundary fixtures.

The reference sums float64 terms left to right (internal/kern/mathx.go:
55-75, pockettts/nn.go:27-49); the oracle does the same.  The GPU sums in a
tree and falls back to the in-order sums when a float32 result could
differ.  This module restates the two trees the kernels use, in the same
order of additions (numpy float64 and float32 arithmetic round like the
device's), so that a test can show that a row needs the fallback:
  - "block": ln_block_reduce with 256 threads: thread t sums terms t, t+256,
    ... in order; each wave's 64 partials as wave_sum_f64 below; the four
    waves' sums in order;
  - "wave": wave_ln32/wave_ln64 with the row as float4 pieces per lane
    (piece P = 64 j + lane, j < 5): lane sums its pieces' values in order;
    DPP xor 1, xor 2, mirror of 8, mirror of 16; then (r0 + r16) + (r32 +
    r48).
"""
from __future__ import annotations

import numpy as np

U = 2.0 ** -53
IDX = np.arange(64)


def serial(t: np.ndarray) -> np.ndarray:
    """In-order float64 sums of each row (the reference's loop)."""
    return np.add.accumulate(t, axis=1)[:, -1] if t.shape[1] else np.zeros(t.shape[0])


HALF_MIRROR = (IDX & ~7) | (7 - (IDX & 7))
MIRROR = (IDX & ~15) | (15 - (IDX & 15))


def _dpp_wave(v: np.ndarray) -> np.ndarray:
    """wave_sum_f64 over the last axis (64 lanes)."""
    for perm in (IDX ^ 1, IDX ^ 2, HALF_MIRROR, MIRROR):
        v = v + v[..., perm]
    return (v[..., 0] + v[..., 16]) + (v[..., 32] + v[..., 48])


def tree_block(t: np.ndarray, threads: int = 256) -> np.ndarray:
    rows, n = t.shape
    k = -(-n // threads)
    pad = np.zeros((rows, k * threads))
    pad[:, :n] = t
    p = np.zeros((rows, threads))
    for j in range(k):
        p = p + pad[:, j * threads:(j + 1) * threads]
    w = _dpp_wave(p.reshape(rows, threads // 64, 64))
    s = np.zeros(rows)
    for i in range(threads // 64):
        s = s + w[:, i]
    return s


def tree_wave(t: np.ndarray, pieces: int = 5) -> np.ndarray:
    rows, n = t.shape
    npc = n // 4
    lanes = np.zeros((rows, 64))
    for j in range(pieces):
        P = 64 * j + IDX
        ok = P < npc
        Pc = np.minimum(P, npc - 1)
        for c in range(4):
            lanes = lanes + np.where(ok, t[:, 4 * Pc + c], 0.0)
    return _dpp_wave(lanes)


def tree(t: np.ndarray, impl: str) -> np.ndarray:
    return tree_block(t) if impl == "block" else tree_wave(t)


# ---- the device's bound check (grx_ln.h), in the same float64 steps

def depth(n: int, impl: str) -> int:
    """Additions on the longest path of the tree (ln_block_depth,
    ln_wave_depth)."""
    if impl == "block":
        return -(-n // 256) + 6 + 4
    return 4 * -(-(n // 4) // 64) + 6


def slack(n: int, dep: int, a):
    return ((float(n + dep) + 8.0) * (U * 1.001)) * a


def ulp_exp(x: np.ndarray) -> np.ndarray:
    """ln_ulp_exp: the exponent of each float32's unit in the last place
    (127 for zero)."""
    b = np.asarray(x, np.float32).view(np.uint32) & 0x7FFFFFFF
    e = np.maximum((b >> 23).astype(np.int64), 1) - 150
    return np.where(b == 0, 127, e)


def sum_exact(a, mn):
    """ln_sum_exact: every partial sum of float32 values a float64, given
    a = n max|v| and mn = the smallest nonzero |v| (inf if none)."""
    with np.errstate(over="ignore"):
        lim = np.ldexp(1.0, np.minimum(53 + ulp_exp(mn), 1023))
    return ~(mn < np.inf) | (a < lim)


def _mean32(s, n):
    return (s / float(n)).astype(np.float32)


def _inv32(vs, n):
    with np.errstate(invalid="ignore"):
        return (1.0 / np.sqrt(vs / float(n) + 1e-5)).astype(np.float32)


def _same(x, y):
    return np.asarray(x, np.float32).view(np.uint32) == np.asarray(y, np.float32).view(np.uint32)


def mean32_sure(s, a, n, dep):
    e = slack(n, dep, a)
    return _same(_mean32(s - e, n), _mean32(s + e, n))


def inv_width(r):
    """ln_inv_width: the relative half-width around 1/sqrt(x/n + eps)."""
    r = np.asarray(r, np.float64)
    with np.errstate(invalid="ignore"):
        w = (0.5 * r) * (1.0 + 5.0 * r) + 10.5 * U
    return np.where(r <= 0.5, w, np.inf)


def inv32_sure(inv_d, n, dep):
    w = inv_width(slack(n, dep, 1.0))
    with np.errstate(invalid="ignore"):
        return _same((inv_d * (1.0 - w)).astype(np.float32), (inv_d * (1.0 + w)).astype(np.float32))


def _inv64(q, n, eps):
    with np.errstate(invalid="ignore"):
        return 1.0 / np.sqrt(q / float(n) + eps)


def ln64_bound(mean, inv, a, q, n, dep, exact, eps):
    am, dn = np.abs(mean), float(n)
    es = np.where(exact, 0.0, slack(n, dep, a))
    em = np.where(exact, 0.0, (es / dn) * 1.001 + (3.0 * U) * am)
    shift = (2.0 * em) * (es + (dn * U * 1.001) * am) + dn * (em * em)
    with np.errstate(invalid="ignore", divide="ignore"):
        r = np.where(exact, slack(n, dep, 1.0), slack(n, dep, 1.0) + shift / (q + dn * eps))
    w = inv_width(r * 1.01)
    ihi = inv * (1.0 + w)
    c1 = (em * ihi) * 1.0102
    c2 = (w * inv + (8.1 * U) * ihi) * 1.01
    return c1, c2


def out64_sure(d, x, c1, c2):
    dl = c1[:, None] + np.abs(d) * c2[:, None]
    return _same((x - dl).astype(np.float32), (x + dl).astype(np.float32))


def values(x: np.ndarray, impl: str):
    """The values' tree sum, n max|v| (>= their magnitudes' sum) and whether
    the sum is exact in every order (ln_block_values / ln_wave_values)."""
    xd = x.astype(np.float64)
    ax = np.abs(x.astype(np.float32))
    a = float(x.shape[1]) * ax.max(axis=1).astype(np.float64)
    mn = np.where(ax > 0, ax, np.float32(np.inf)).min(axis=1)
    return tree(xd, impl), a, sum_exact(a, mn)


# ---- the two LayerNorms as the GPU forms them

def ln32(x, w, b, impl: str, check: bool = True):
    """kern's layerNorm (mathx.go:55-75) through the GPU's sums; returns
    (outputs, rows that took an in-order pass)."""
    x = np.ascontiguousarray(x, np.float32)
    rows, n = x.shape
    dep = depth(n, impl)
    xd = x.astype(np.float64)
    s, a, exact = values(x, impl)
    fell = np.zeros(rows, bool)
    if check:
        bad = ~exact & ~mean32_sure(s, a, n, dep)
        s = np.where(bad, serial(xd), s)
        fell |= bad
    mean = _mean32(s, n)
    d = (x - mean[:, None]).astype(np.float64)
    vs = tree(d * d, impl)
    if check:
        bad = ~inv32_sure(1.0 / np.sqrt(vs / float(n) + 1e-5), n, dep)
        vs = np.where(bad, serial(d * d), vs)
        fell |= bad
    inv = _inv32(vs, n)
    t = (x - mean[:, None]) * inv[:, None]
    return (t * np.asarray(w, np.float32)) + np.asarray(b, np.float32), fell


def ln64(x, w, b, eps: float, impl: str, check: bool = True):
    """pockettts' layerNorm (nn.go:27-49) through the GPU's sums; returns
    (outputs, rows that took the in-order pass)."""
    x = np.ascontiguousarray(x, np.float32)
    rows, n = x.shape
    dep = depth(n, impl)
    xd = x.astype(np.float64)
    s, a, exact = values(x, impl)
    mean = s / float(n)
    d = xd - mean[:, None]
    q = tree(d * d, impl)
    inv = _inv64(q, n, eps)
    fell = np.zeros(rows, bool)
    if check:
        c1, c2 = ln64_bound(mean, inv, a, q, n, dep, exact, eps)
        bad = ~np.all(out64_sure(d, d * inv[:, None], c1, c2), axis=1)
        ms = np.where(exact, mean, serial(xd) / float(n))
        ds = xd - ms[:, None]
        mean = np.where(bad, ms, mean)
        inv = np.where(bad, _inv64(serial(ds * ds), n, eps), inv)
        fell |= bad
    o = ((xd - mean[:, None]) * inv[:, None]).astype(np.float32)
    if w is not None:
        o = (o * np.asarray(w, np.float32)) + np.asarray(b, np.float32)
    return o, fell
