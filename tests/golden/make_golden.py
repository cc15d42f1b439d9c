"""Write tests/golden/int_products.npz: exact known-answer matmul vectors.

The reference ships no golden vectors (its parity test draws unseeded
torch.randn, tests/test_matmul.py:36-37), so the known answers here come from
arithmetic: integer-valued inputs in [-8, 8], whose products and partial sums
stay below 2**24, are represented exactly in float32 and bfloat16, so every
correct fp32-accumulating matmul must reproduce the integer product bit for
bit.  Expected outputs are computed with Python/numpy int64 arithmetic.

Shapes: the reference's parity shapes (tests/test_matmul.py:33) that keep the
file small, plus ragged shapes whose every tile edge is partial and K tails
that are not multiples of any K step.

    python tests/golden/make_golden.py
"""

import os

import numpy as np

SHAPES = [(1, 1, 1), (5, 7, 3), (65, 17, 63), (128, 300, 130),
          (3, 4097, 5), (17, 33, 65), (257, 129, 255), (16, 1000, 131)]


def main():
    rng = np.random.Generator(np.random.PCG64(20261201))
    out = {"shapes": np.array(SHAPES, dtype=np.int64)}
    for i, (m, k, n) in enumerate(SHAPES):
        a = rng.integers(-8, 9, size=(m, k), dtype=np.int64)
        b = rng.integers(-8, 9, size=(k, n), dtype=np.int64)
        c = a @ b
        assert np.abs(c).max() < 2 ** 24
        out[f"x1_{i}"] = a.astype(np.int8)
        out[f"x2_{i}"] = b.astype(np.int8)
        out[f"out_{i}"] = c.astype(np.int32)
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "int_products.npz")
    np.savez_compressed(path, **out)
    print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
