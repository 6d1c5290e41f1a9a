"""Writes the GEMV golden fixtures of tests/golden from the CPU oracle (brute force cross-checked).

The reference holds no golden vectors for this path (its tests compute brute-force truth on the fly), so these
fixtures are the oracle's, each checked against an independent numpy product before it is written. Run from the repo
root: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import oracle  # noqa: E402

CASES = [
    # name, rows, cols, trit seed, act seed, weight scale, act scale
    ("gemv_64x320", 64, 320, 11, 12, 0.05, 1.0),
    ("gemv_96x3072", 96, 3072, 21, 22, 0.02, 0.3),
    ("gemv_130x161", 130, 161, 31, 32, 0.7, 2.5),
    ("gemv_65x23040", 65, 23040, 41, 42, 0.013, 0.09),
]


def main():
    for name, rows, cols, ts, as_, ws, scale in CASES:
        t = oracle.gen_trits(ts, (rows, cols))
        a = oracle.gen_i8(as_, cols, -128, 127)
        planar = oracle.pack_matrix(t)
        acc = oracle.gemv_lut_planar(planar, rows, cols, a)
        assert np.array_equal(acc.astype(np.int64), t.astype(np.int64) @ a.astype(np.int64))
        y = oracle.epilogue_f32(acc, ws, scale)
        np.savez_compressed(os.path.join(HERE, name + ".npz"), shape=np.array([rows, cols]), planar=planar, acts=a,
                            acc=acc, y=y, weight_scale=np.float32(ws), act_scale=np.float32(scale))
        print(name, acc[:4])
    # config 0: store the inputs' seeds and a checksum of the exact outputs.
    t = oracle.gen_trits(0xC0FFEE, (2560, 2560))
    a = oracle.gen_i8(0xBEEF, 2560, -127, 127)
    acc = t.astype(np.int64) @ a.astype(np.int64)
    y = oracle.epilogue_f32(acc.astype(np.int32), 0.02, 1.0)
    np.savez_compressed(os.path.join(HERE, "config0_2560.npz"), acc=acc.astype(np.int32), y=y,
                        trit_seed=np.uint64(0xC0FFEE), act_seed=np.uint64(0xBEEF))


if __name__ == "__main__":
    main()
