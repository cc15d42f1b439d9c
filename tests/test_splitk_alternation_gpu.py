"""Split-K combines under changing inputs, on an MI355X.

Every kernel that splits a reduction across workgroups publishes partials in
a workspace and lets the last workgroup of a cell add them (agent-coherent
stores and loads, a relaxed agent-scope counter).  A stale cache line — a
partial of an earlier call still held somewhere the combining workgroup
reads from — would only show when the same workspace slots receive different
values from one call to the next, so each case here alternates two seeded
small-integer inputs through the same shape, variant, split and workspace,
32 times, and checks every result bit for bit against its exact integer
product (integer sums below 2^24 are exact in fp32 in any order).  The first
mismatch fails the case.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tilec import ext

pytestmark = pytest.mark.gpu

ROUNDS = 32


def say(msg):
    print(msg, flush=True)


def _pair(shape_a, shape_b, seed, lo=-4, hi=4):
    a = [O.small_ints(shape_a, seed + 2 * i, lo, hi) for i in range(2)]
    b = [O.small_ints(shape_b, seed + 2 * i + 1, lo, hi) for i in range(2)]
    return a, b


def _exact(a, b):
    """The integer product, in int64, as fp32 (every entry below 2^24)."""
    p = a.astype(np.int64) @ b.astype(np.int64)
    assert np.abs(p).max() < 1 << 24
    return p.astype(np.float32)


# (kernel family, config, (M, K, N), dtype): each one splits K.
MATMUL_CASES = [
    ("streaming", ("skinny_f32_w8_b1", 8), (16, 4096, 1024), torch.float32),
    ("panel", ("skinny_f32_p_v1_w8", 8), (1, 4096, 4096), torch.float32),
    ("panel bf16", ("skinny_bf16_p_v1_w8", 16), (1, 4096, 4096), torch.bfloat16),
    ("panel, M <= 4", ("skinny_f32_p_v4_w8", 8), (3, 4096, 4096), torch.float32),
    ("direct", ("direct_f32_32x64_w4_db", 8), (127, 1000, 513), torch.float32),
    ("tile GEMM", ("gemm_f32_64x64x16_w2x2", 8), (100, 4096, 200), torch.float32),
    ("streaming bf16", ("skinny_bf16_w8_b1", 8), (16, 4096, 1024), torch.bfloat16),
]


@pytest.mark.parametrize("case", range(len(MATMUL_CASES)))
def test_alternating_inputs_matmul(case):
    fam, cfg, (M, K, N), dt = MATMUL_CASES[case]
    say(f"alternation {fam}: {cfg} at {(M, K, N)} {dt}")
    a, b = _pair((M, K), (K, N), 900 + 10 * case)
    x1 = [torch.from_numpy(v).to("cuda").to(dt) for v in a]
    x2 = [torch.from_numpy(v).to("cuda").to(dt) for v in b]
    want = [torch.from_numpy(_exact(a[i], b[i])).to("cuda") for i in range(2)]
    assert not torch.equal(want[0], want[1])
    for r in range(ROUNDS):
        i = r & 1
        got = ext.matrix_mul(x1[i], x2[i], cfg)
        torch.cuda.synchronize()
        if not torch.equal(got, want[i]):
            bad = (got != want[i]).nonzero()[:4].tolist()
            pytest.fail(f"{fam}: round {r} (input {i}) differs from the exact product at {bad}")
    say(f"alternation {fam}: {ROUNDS} rounds exact")


# (axis, shape, dtype): splits the reduced dimension across workgroups.
SUM_CASES = [
    (1, (4, 1 << 20), torch.float32),
    (0, (1 << 18, 64), torch.float32),
    (1, (8, 1 << 19), torch.bfloat16),
]


@pytest.mark.parametrize("case", range(len(SUM_CASES)))
def test_alternating_inputs_sum(case):
    axis, shape, dt = SUM_CASES[case]
    say(f"alternation sum axis {axis}: {shape} {dt}")
    xs = [O.small_ints(shape, 950 + 10 * case + i, -8, 8) for i in range(2)]
    x = [torch.from_numpy(v).to("cuda").to(dt) for v in xs]
    want = [torch.from_numpy(v.astype(np.int64).sum(axis).astype(np.float32)).to("cuda") for v in xs]
    assert not torch.equal(want[0], want[1])
    for r in range(ROUNDS):
        i = r & 1
        got = ext.sum(x[i], axis=axis)
        torch.cuda.synchronize()
        if not torch.equal(got, want[i]):
            bad = (got != want[i]).nonzero()[:4].tolist()
            pytest.fail(f"sum axis {axis}: round {r} (input {i}) differs from the exact sum at {bad}")
    say(f"alternation sum axis {axis}: {ROUNDS} rounds exact")
