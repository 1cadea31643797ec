"""Writes rnnt_softmax_boundary.npy: joint logits (97 tokens, the last one
blank) whose softmax probability of the first maximal token, float32(1/s)
with s the in-order float64 sum of e^(x - max), has a float32 rounding
boundary within a quarter of the device's error interval (2^-52 (V + 4)
relative) of 1/s, so the decoder must form s in order.  Found by search
with numpy's exp, then checked with the oracle's exp and in-order sum."""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

V = 97


def main():
    from oracle import oracle as O
    rng = np.random.default_rng(2024)
    delta = (V + 4) * 2.0 ** -52
    for rnd in range(400):
        x = (rng.standard_normal((200000, V)) * 2).astype(np.float32)
        x[:, V - 1] = -30.0  # blank never wins
        x[:, 0] = 9.0        # token 0 the maximum
        d = (x - x[:, :1]).astype(np.float32).astype(np.float64)
        s = np.exp(d).sum(1)
        q = 1.0 / s
        f = q.astype(np.float32)
        # the float32 rounding boundary nearest to q
        up = np.nextafter(f, np.float32(np.inf)).astype(np.float64)
        dn = np.nextafter(f, np.float32(-np.inf)).astype(np.float64)
        fb = f.astype(np.float64)
        mid = np.where(q >= fb, (fb + up) / 2, (fb + dn) / 2)
        near = np.abs(mid - q) <= q * delta / 4
        for i in np.nonzero(near)[0]:
            row = x[i]
            sq = 0.0
            for v in row:
                sq += O.fd_exp(float(np.float32(v - row[0])))
            qq = 1.0 / sq
            if abs(((float(np.float32(qq)) + float(np.float32(np.nextafter(np.float32(qq), np.float32(
                    np.inf if qq >= float(np.float32(qq)) else -np.inf))))) / 2) - qq) <= qq * delta / 4:
                np.save(os.path.join(HERE, "rnnt_softmax_boundary.npy"), row)
                print("found after", rnd, "rounds: 1/s =", qq)
                return
    raise SystemExit("none found")


if __name__ == "__main__":
    main()
