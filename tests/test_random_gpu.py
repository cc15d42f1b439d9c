"""Seeded random parity sweep on the GPU: (variant, split) drawn from every
config `ext.hip_configs` offers for a random shape, operand layout and dtype,
against the fp64 oracle.  The error is taken per element relative to
|x1| |x2| (the bound fp32 summation in any order meets), so dot products
that cancel do not inflate it the way a plain relative error would."""

import random

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tilec import ext

pytestmark = pytest.mark.gpu

MS = [1, 2, 3, 4, 7, 15, 16, 17, 33, 64, 100, 127, 129, 200, 257, 513, 1024]
NS = [1, 3, 7, 16, 33, 63, 64, 65, 127, 128, 129, 200, 257, 513]
KS = [1, 2, 5, 15, 16, 17, 63, 64, 65, 127, 128, 129, 255, 333, 1000, 1025, 2048, 3001, 4097]


def _device(h, col_major):
    """A (rows x cols) host matrix on the GPU, row-major or as the transposed
    view of a contiguous (cols x rows) tensor; uint16 = bf16 bit patterns."""
    src = np.ascontiguousarray(h.T if col_major else h)
    t = torch.from_numpy(src.view(np.int16) if h.dtype == np.uint16 else src).cuda()
    if h.dtype == np.uint16:
        t = t.view(torch.bfloat16)
    return t.T if col_major else t


@pytest.mark.parametrize("block", range(3))
def test_random_configs(block):
    rng = random.Random(1000 + block)
    for i in range(100):
        dtype = rng.choice(["f32", "f32", "bf16"])
        M, N, K = rng.choice(MS), rng.choice(NS), rng.choice(KS)
        if M * K * N > 5e7:
            K = max(1, int(5e7 // (M * N)))
        layout = rng.choice([0, 0, 1, 2, 3])
        cfg = rng.choice(ext.hip_configs(M, K, N, dtype, layout))
        seed = 10000 * block + 10 * i
        a, b = O.normal((M, K), seed), O.normal((K, N), seed + 1)
        if dtype == "bf16":
            a, b = O.bf16_round(a), O.bf16_round(b)
            ref, af, bf = O.matmul_bf16_f64(a, b), O.bf16_to_f32(a), O.bf16_to_f32(b)
        else:
            ref, af, bf = O.matmul_f64(a, b), a, b
        print(f"random {block}.{i}: {dtype} {(M, K, N)} layout {layout} {cfg}", flush=True)
        got = ext.matrix_mul(_device(a, layout & 1), _device(b, layout & 2), cfg)
        torch.cuda.synchronize()
        bound = np.abs(af.astype(np.float64)) @ np.abs(bf.astype(np.float64))
        err = np.abs(got.cpu().numpy().astype(np.float64) - ref) / np.maximum(bound, 1e-30)
        assert float(err.max()) <= 1e-5, (dtype, (M, K, N), layout, cfg, float(err.max()))
