"""Write tests/golden/ln_boundary.npz: LayerNorm rows on which the GPU's
parallel float64 sums, taken alone, give other float32 results than the
reference's left-to-right sums (internal/kern/mathx.go:55-75 for the kern
form, pockettts/nn.go:27-49 for the float64 form), for both kernel forms
of the GPU (workgroup and one-wave trees, tests/_ln_tree.py).  The GPU must
reproduce the oracle on them, which it can only do through its in-order
pass.

    python tests/golden/make_ln_boundary.py

Two constructions, each checked against the oracle and the CPU model of
the trees before it is kept:
  inv path  - a row of D, -D and small +-e pairs (the mean is exactly 0,
              so d_i = x_i): in order, 2 D^2 absorbs every small square
              (each below half its unit in the last place), while the
              trees add many small squares together first and keep part of
              them.  A scan over D (kern form: inv rounded to float32) or
              over one pair's e (float64 form: an output rounded to
              float32) puts a float32 rounding boundary between the two.
  mean path - cancelling +-a pairs and a few tiny unpaired values t: the
              values' sum is inexact, the two orders' means differ by far
              more than the float32 unit of the tiny mean, and the tiny
              values' outputs (bias 0 there) show it.
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(HERE))

import oracle  # noqa: E402
import _ln_tree as L  # noqa: E402

N = 1024
EPS64 = 1e-5
OUT = os.path.join(HERE, "ln_boundary.npz")


def oracle_out(form, x, w, b):
    if form == "kern":
        return oracle.layernorm(x, w, b)
    return oracle.layernorm_f64(x, w, b, EPS64)


def model_out(form, x, w, b, impl, check):
    if form == "kern":
        return L.ln32(x, w, b, impl, check)
    return L.ln64(x, w, b, EPS64, impl, check)


def differs(a, b):
    return (np.asarray(a, np.float32).view(np.uint32) != np.asarray(b, np.float32).view(np.uint32)).any(axis=1)


def keeps(form, impl, x, w, b):
    """x's rows on which the tree alone differs from the oracle and the
    bound check sends the row to the in-order pass (which then agrees)."""
    want = oracle_out(form, x, w, b)
    tree, _ = model_out(form, x, w, b, impl, False)
    got, fell = model_out(form, x, w, b, impl, True)
    ok = differs(tree, want) & fell & ~differs(got, want)
    assert not (differs(tree, want) & ~fell).any(), "a row the check missed: the bound is wrong"
    return ok


def pair_row(rng, D, lo=2e-6, hi=6e-6):
    m = (N - 2) // 2
    e = (rng.uniform(lo, hi, m) * rng.choice([-1.0, 1.0], m)).astype(np.float32)
    x = np.concatenate([[D, -D], e, -e]).astype(np.float32)
    return x[rng.permutation(N)]


def inv_path_kern(rng, impl, want=2):
    w = rng.uniform(0.5, 1.5, N).astype(np.float32)
    b = (rng.standard_normal(N) * 0.1).astype(np.float32)
    rows = []
    for _ in range(20):
        base = pair_row(rng, np.float32(600.0))
        big = np.nonzero(np.abs(base) > 1)[0]
        sq = base.astype(np.float64) ** 2
        G = L.tree(sq[None], impl)[0] - 2.0 * 600.0 ** 2  # the small squares the tree keeps
        # every float32 D with 2 D^2 in [2^19, 2^20): the tree keeps the same G
        Ds = np.float32(512.0) + np.arange(0, (724 - 512) * 2 ** 14, dtype=np.int64).astype(np.float64) * 2.0 ** -14
        Ds = Ds.astype(np.float32)
        vs = 2.0 * Ds.astype(np.float64) ** 2
        a = (1.0 / np.sqrt(vs / N + 1e-5)).astype(np.float32)
        t = (1.0 / np.sqrt((vs + G) / N + 1e-5)).astype(np.float32)
        for Dc in Ds[a != t][:8]:
            x = base.copy()
            x[big[base[big] > 0]] = Dc
            x[big[base[big] < 0]] = -Dc
            if keeps("kern", impl, x[None], w, b)[0]:
                rows.append(x)
                break
        if len(rows) == want:
            return np.array(rows), w, b
    raise RuntimeError(f"kern {impl}: no inv-path row found")


def inv_path_f64(rng, impl, want=2):
    # squares just under half the unit in the last place of 2 D^2 in
    # [2^19, 2^20) (2^-34): the tree keeps as much of them as it can
    c_all = np.arange(np.float32(2.0 ** -19).view(np.int32), np.float32(7.5e-6).view(np.int32),
                      dtype=np.int32).view(np.float32)
    rows = []
    for _ in range(40):
        D = np.float32(rng.uniform(512.0, 723.0))
        x = pair_row(rng, D, 6e-6, 7.5e-6)
        xd = x.astype(np.float64)
        q_s = L.serial((xd ** 2)[None])[0]
        q_t = L.tree((xd ** 2)[None], impl)[0]
        if q_s == q_t:
            continue
        i_s, i_t = 1.0 / np.sqrt(q_s / N + EPS64), 1.0 / np.sqrt(q_t / N + EPS64)
        # one pair's value such that float32(e * inv) differs between the two
        hits = []
        for c in np.array_split(c_all, 8):
            cd = c.astype(np.float64)
            hits.extend(c[(cd * i_s).astype(np.float32) != (cd * i_t).astype(np.float32)][:8])
        small = np.nonzero((np.abs(x) < 1) & (x > 0))[0]
        for cv in hits[:16]:
            y = x.copy()
            k = small[0]
            partner = np.nonzero(y == -y[k])[0][0]
            y[k], y[partner] = cv, -cv
            if keeps("f64", impl, y[None], None, None)[0]:
                rows.append(y)
                break
        if len(rows) == want:
            return np.array(rows), None, None
    raise RuntimeError(f"f64 {impl}: no inv-path row found")


def mean_path(rng, form, impl, want=2):
    rows = []
    w = rng.uniform(0.5, 1.5, N).astype(np.float32)
    for _ in range(200):
        r = 6
        m = (N - r) // 2
        a = rng.standard_normal(m).astype(np.float32)
        tiny = (rng.uniform(1.0, 2.0, r) * 1e-12 * rng.choice([-1.0, 1.0], r)).astype(np.float32)
        x = np.concatenate([a, -a, tiny]).astype(np.float32)
        perm = rng.permutation(N)
        x = x[perm]
        b = (rng.standard_normal(N) * 0.1).astype(np.float32)
        b[np.abs(x) < 1e-9] = 0.0  # the tiny values' outputs stay tiny
        if keeps(form, impl, x[None], w, b)[0]:
            rows.append((x, b))
        if len(rows) == want:
            return rows, w
    raise RuntimeError(f"{form} {impl}: no mean-path row found")


def main():
    oracle.build()
    rng = np.random.default_rng(20261202)
    out = {}
    for impl in ("block", "wave"):
        x, w, b = inv_path_kern(rng, impl)
        out[f"kern_{impl}_inv_x"], out[f"kern_{impl}_inv_w"], out[f"kern_{impl}_inv_b"] = x, w, b
        x, _, _ = inv_path_f64(rng, impl)
        out[f"f64_{impl}_inv_x"] = x
        for form in ("kern", "f64"):
            rows, w = mean_path(rng, form, impl)
            for j, (x, b) in enumerate(rows):
                out[f"{form}_{impl}_mean{j}_x"] = x[None]
                out[f"{form}_{impl}_mean{j}_w"] = w
                out[f"{form}_{impl}_mean{j}_b"] = b
    # the oracle's outputs, for regression
    for k in [k for k in out if k.endswith("_x")]:
        form, base = k.split("_")[0], k[:-2]
        w, b = out.get(base + "_w"), out.get(base + "_b")
        out[base + "_y"] = oracle_out(form, out[k], w, b)
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT}: " + ", ".join(f"{k} {v.shape}" for k, v in out.items() if k.endswith("_x")))


if __name__ == "__main__":
    main()
