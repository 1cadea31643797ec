"""The path's LayerNorms on the GPU (grx_layernorm_dev: the workgroup and
one-wave forms every model kernel uses) against the oracle, bit for bit:
kern's layerNorm (internal/kern/mathx.go:55-75) and pockettts' float64 one
(pockettts/nn.go:27-49).

The boundary fixtures (tests/golden/ln_boundary.npz) are rows on which the
GPU's tree sums alone round to other float32 results: with GRX_LN_TREE_ONLY
the device gives exactly what the CPU model of its trees (tests/
_ln_tree.py) predicts - so the model is the device's order - and differs
from the oracle; without it the device gives the oracle's results.
"""
import os

import numpy as np
import pytest

import _ln_tree as L
from gorelaxor_amd import GrxError

pytestmark = pytest.mark.gpu

FIX = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ln_boundary.npz")
EPS64 = 1e-5
IMPL = {"block": 0, "wave": 1}


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _run(kern, form, impl, x, w, b, eps=EPS64, flags=0):
    from gorelaxor_amd import hiprt

    x = np.ascontiguousarray(x, np.float32)
    rows, n = x.shape
    dx = hiprt.DeviceBuffer.from_array(x)
    dy = hiprt.DeviceBuffer(x.nbytes)
    dw = hiprt.DeviceBuffer.from_array(np.ascontiguousarray(w, np.float32)) if w is not None else None
    db = hiprt.DeviceBuffer.from_array(np.ascontiguousarray(b, np.float32)) if b is not None else None
    kern.layernorm_dev(kern.LN_KERN if form == "kern" else kern.LN_F64, IMPL[impl], dy, dx, rows, n, dw, db, eps,
                       flags)
    kern.default_context().sync()
    return dy.download(np.float32, (rows, n))


def _oracle(orc, form, x, w, b, eps=EPS64):
    if form == "kern":
        return orc.layernorm(x, w, b)
    return orc.layernorm_f64(x, w, b, eps)


def _model(form, x, w, b, impl, check, eps=EPS64):
    if form == "kern":
        return L.ln32(x, w, b, impl, check)[0]
    return L.ln64(x, w, b, eps, impl, check)[0]


def test_boundary_rows_need_and_get_the_in_order_pass(kern, orc):
    z = np.load(FIX)
    seen = 0
    for k in sorted(z.files):
        if not k.endswith("_x"):
            continue
        base = k[:-2]
        form, impl = base.split("_")[:2]
        x, w, b, y = z[k], z.get(base + "_w"), z.get(base + "_b"), z[base + "_y"]
        print(f"ln boundary {base} rows {x.shape[0]}", flush=True)
        tree = _run(kern, form, impl, x, w, b, flags=kern.LN_TREE_ONLY)
        assert np.array_equal(_bits(tree), _bits(_model(form, x, w, b, impl, False))), f"{base}: tree order"
        assert (_bits(tree) != _bits(y)).any(axis=1).all(), f"{base}: the tree alone is right"
        got = _run(kern, form, impl, x, w, b)
        assert np.array_equal(_bits(got), _bits(y)), f"{base}: differs from the oracle"
        seen += 1
    assert seen == 12  # 2 forms x 2 kernel forms x (inv, mean0, mean1)


@pytest.mark.parametrize("form", ["kern", "f64"])
@pytest.mark.parametrize("impl", ["block", "wave"])
@pytest.mark.parametrize("n", [32, 68, 512, 1024, 1280])
def test_random_rows_bit_exact(kern, orc, form, impl, n):
    rng = np.random.default_rng(n + 7 * len(form) + IMPL[impl])
    x = np.concatenate([rng.standard_normal((300, n)),
                        rng.standard_normal((100, n)) * 0.01 + 30.0,
                        rng.standard_normal((100, n)) * np.exp2(rng.uniform(-30, 10, (100, n)))]).astype(np.float32)
    w = rng.uniform(0.5, 1.5, n).astype(np.float32)
    b = (rng.standard_normal(n) * 0.1).astype(np.float32)
    for ww, bb, eps in ((w, b, 1e-5), (None, None, 1e-6)) if form == "f64" else ((w, b, 1e-5),):
        want = _oracle(orc, form, x, ww, bb, eps)
        got = _run(kern, form, impl, x, ww, bb, eps)
        assert np.array_equal(_bits(got), _bits(want)), f"{form} {impl} n={n}"
        tree = _run(kern, form, impl, x, ww, bb, eps, flags=kern.LN_TREE_ONLY)
        assert np.array_equal(_bits(tree), _bits(_model(form, x, ww, bb, impl, False, eps))), "tree order"


def test_wide_rows_workgroup_form(kern, orc):
    rng = np.random.default_rng(11)
    for n in (2048, 4096, 5120):
        x = rng.standard_normal((64, n)).astype(np.float32)
        w = rng.uniform(0.5, 1.5, n).astype(np.float32)
        b = rng.standard_normal(n).astype(np.float32)
        assert np.array_equal(_bits(_run(kern, "kern", "block", x, w, b)), _bits(orc.layernorm(x, w, b))), n
        assert np.array_equal(_bits(_run(kern, "f64", "block", x, w, b)),
                              _bits(orc.layernorm_f64(x, w, b, EPS64))), n


def test_errors(kern):
    x = np.zeros((1, 64), np.float32)
    with pytest.raises(GrxError, match="needs w and b"):
        _run(kern, "kern", "block", x, None, None)
    with pytest.raises(GrxError, match="go together"):
        _run(kern, "f64", "block", x, np.ones(64, np.float32), None)
    with pytest.raises(GrxError, match="one-wave form"):
        _run(kern, "kern", "wave", np.zeros((1, 1284), np.float32), np.ones(1284, np.float32),
             np.ones(1284, np.float32))
