"""The GPU LayerNorms' order safety, on the CPU: the reference sums its
float64 statistics left to right (internal/kern/mathx.go:55-75,
pockettts/nn.go:27-49); the GPU sums them in a tree and, where a float32
result could differ, again in order (gorelaxor_amd/csrc/grx_ln.h).

tests/_ln_tree.py restates the GPU's trees and bound check; the GPU tests
(test_gpu_layernorm.py) pin that model to the device.  Here:
  - the boundary fixtures (tests/golden/ln_boundary.npz, written by
    tests/golden/make_ln_boundary.py) are rows on which the tree alone gives
    other float32 results than the oracle, so a pure tree sum fails them;
  - the bound check flags every row on which tree and oracle differ, over
    families of rows built to stress it (a missed row would be a wrong
    bound), and rarely flags ordinary rows.
"""
import os

import numpy as np
import pytest

import _ln_tree as L

FIX = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ln_boundary.npz")
EPS64 = 1e-5


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _cases():
    z = np.load(FIX)
    for k in sorted(z.files):
        if k.endswith("_x"):
            base = k[:-2]
            form, impl = base.split("_")[:2]
            yield base, form, impl, z[k], z.get(base + "_w"), z.get(base + "_b"), z[base + "_y"]


def _model(form, x, w, b, impl, check):
    if form == "kern":
        return L.ln32(x, w, b, impl, check)
    return L.ln64(x, w, b, EPS64, impl, check)


def _oracle(orc, form, x, w, b):
    if form == "kern":
        return orc.layernorm(x, w, b)
    return orc.layernorm_f64(x, w, b, EPS64)


def test_fixtures_are_the_oracles_outputs(orc):
    for base, form, impl, x, w, b, y in _cases():
        assert np.array_equal(_bits(_oracle(orc, form, x, w, b)), _bits(y)), base


def test_fixtures_fail_a_pure_tree_sum():
    """On every fixture row the tree alone is wrong and the check sends the
    row to the in-order pass, which is right."""
    kinds = set()
    for base, form, impl, x, w, b, y in _cases():
        tree, _ = _model(form, x, w, b, impl, False)
        got, fell = _model(form, x, w, b, impl, True)
        assert (_bits(tree) != _bits(y)).any(axis=1).all(), f"{base}: the tree alone is already right"
        assert fell.all(), f"{base}: not flagged"
        assert np.array_equal(_bits(got), _bits(y)), base
        kinds.add((form, impl, base.split("_")[2].rstrip("0123456789")))
    # both forms, both kernel forms, both the mean's and inv's paths
    assert kinds == {(f, i, p) for f in ("kern", "f64") for i in ("block", "wave") for p in ("inv", "mean")}


def _families(rng, n):
    """Rows that push the sums toward their bounds."""
    yield "normal", rng.standard_normal((400, n)).astype(np.float32)
    yield "offset", (rng.standard_normal((400, n)) * 0.01 + 30.0).astype(np.float32)
    # cancelling pairs plus tiny unpaired values: inexact, tiny means
    a = rng.standard_normal((400, (n - 6) // 2)).astype(np.float32)
    t = (rng.uniform(1, 2, (400, 6)) * 1e-12).astype(np.float32)
    x = np.concatenate([a, -a, t], axis=1)
    yield "cancel", np.take_along_axis(x, rng.permuted(np.tile(np.arange(n), (400, 1)), axis=1), axis=1)
    # two large values and many squares just under their half unit
    D = rng.uniform(512, 723, (400, 1)).astype(np.float32)
    e = (rng.uniform(6e-6, 7.5e-6, (400, (n - 2) // 2)) * rng.choice([-1, 1], (400, (n - 2) // 2))).astype(np.float32)
    x = np.concatenate([D, -D, e, -e], axis=1)
    yield "absorb", np.take_along_axis(x, rng.permuted(np.tile(np.arange(n), (400, 1)), axis=1), axis=1)
    # magnitudes spread over 40 binades
    yield "spread", (rng.standard_normal((400, n)) * np.exp2(rng.uniform(-30, 10, (400, n)))).astype(np.float32)


@pytest.mark.parametrize("n", [32, 512, 1024, 1280])
def test_check_flags_every_mismatch(orc, n):
    rng = np.random.default_rng(n)
    w = rng.uniform(0.5, 1.5, n).astype(np.float32)
    b = (rng.standard_normal(n) * 0.1).astype(np.float32)
    for name, x in _families(rng, n):
        for form in ("kern", "f64"):
            want = _oracle(orc, form, x, w, b)
            for impl in ("block", "wave"):
                tree, _ = _model(form, x, w, b, impl, False)
                got, fell = _model(form, x, w, b, impl, True)
                miss = (_bits(tree) != _bits(want)).any(axis=1) & ~fell
                assert not miss.any(), f"{name} {form} {impl} n={n}: rows {np.nonzero(miss)[0][:5]} missed"
                assert np.array_equal(_bits(got), _bits(want)), f"{name} {form} {impl} n={n}"


def test_in_order_pass_is_rare_on_ordinary_rows():
    rng = np.random.default_rng(3)
    n = 1024
    x = rng.standard_normal((4000, n)).astype(np.float32)
    w = np.ones(n, np.float32)
    b = np.zeros(n, np.float32)
    for impl in ("block", "wave"):
        assert L.ln32(x, w, b, impl)[1].sum() <= 4
        assert L.ln64(x, w, b, EPS64, impl)[1].sum() <= 60  # ~0.4 % of rows: each output rounds


def test_tree_model_matches_the_oracle_on_ordinary_rows(orc):
    """The tree model is not a trivial restatement of the oracle, but it
    agrees with it wherever no rounding boundary interferes."""
    rng = np.random.default_rng(4)
    x = rng.standard_normal((500, 768)).astype(np.float32)
    w = rng.standard_normal(768).astype(np.float32)
    b = rng.standard_normal(768).astype(np.float32)
    for impl in ("block", "wave"):
        assert np.array_equal(_bits(L.ln32(x, w, b, impl, False)[0]), _bits(orc.layernorm(x, w, b)))
        assert np.array_equal(_bits(L.ln64(x, None, None, EPS64, impl, False)[0]),
                              _bits(orc.layernorm_f64(x, None, None, EPS64)))
