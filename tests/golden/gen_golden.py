"""Writes the committed golden fixtures from the CPU oracle.

    python tests/golden/gen_golden.py

The reference holds no golden vectors for this path (no testdata/), so these
fixtures pin the oracle's own outputs: a later change to the oracle or to the
product that moves a bit fails test_oracle_golden.py / test_gpu_kern.py.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from gorelaxor_amd.synth import q8_weight  # noqa: E402


def gemv_fixture():
    rng = np.random.default_rng(2024)
    n, k = 64, 1024
    w = q8_weight(rng, n, k)
    x = rng.standard_normal((2, k)).astype(np.float32)
    x[1, :32] = 0
    bias = rng.standard_normal(n).astype(np.float32)
    y = oracle.matmul_q8_int(x, w, n, k, bias)
    qa, sa = oracle.quant_act_i8(x)
    s = oracle.block_dots(qa, w, n, k)
    np.savez_compressed(os.path.join(HERE, "q8_gemv_64x1024.npz"), n=n, k=k, w=w, x=x, bias=bias, y=y,
                        qa=qa, sa=sa, s=s)


if __name__ == "__main__":
    oracle.build()
    gemv_fixture()
    print("fixtures written to", HERE)
