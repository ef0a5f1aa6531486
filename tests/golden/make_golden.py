"""Writes tests/golden/q8_small_case.npz from the CPU oracle.

The case is small and seeded: W [40, 320] ~ N(0, 0.02) (K = 320 is 10 blocks,
so the device pass layout pads its single pass), x [3, 320] ~ N(0, 1) with
the last block of row 1 zeroed.  Stored: weights, arena (p4) bytes, Q8_1
activations and both epilogue variants of y = x . W^T.  Run from the repo
root: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle import q8_oracle as o  # noqa: E402


def main():
    rng = np.random.default_rng(20261201)
    n, k, m = 40, 320, 3
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[1, -32:] = 0.0
    p4 = o.pack_q8_0_p4(w)
    qa, sa = o.quantize_act_q8_1(x)
    y_scalar = o.linear(x, p4, n, epilogue="scalar")
    y_fma = o.linear(x, p4, n, epilogue="fma")
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "q8_small_case.npz")
    np.savez_compressed(out, w=w, x=x, p4=p4, qa=qa, sa=sa, y_scalar=y_scalar,
                        y_fma=y_fma)
    print(out)


if __name__ == "__main__":
    main()
