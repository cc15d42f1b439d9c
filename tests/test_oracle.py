"""Pins the CPU oracle (oracle/) before it is trusted as the parity checker.

Each oracle function is checked against something that does not share its
code: torch.matmul (the reference's own oracle, tests/test_matmul.py:40),
brute-force Python loops, exact integer arithmetic, closed forms and
invariants.  Several checks are chosen so a plausible slip (a dropped K step,
a transposed operand, a wrong mask) fails them; `test_planted_mistakes_are_caught`
confirms that on deliberately broken oracles.
"""

import math
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O

REF_SHAPES = [(1, 1, 1), (5, 7, 3), (65, 17, 63), (128, 300, 130), (512, 1024, 256)]
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "int_products.npz")


def brute_f64(a, b):
    M, K = a.shape
    N = b.shape[1]
    c = [[0.0] * N for _ in range(M)]
    for i in range(M):
        for j in range(N):
            s = 0.0
            for k in range(K):
                s += float(a[i, k]) * float(b[k, j])
            c[i][j] = s
    return np.array(c, dtype=np.float64).reshape(M, N)


@pytest.mark.parametrize("shape", REF_SHAPES)
def test_tiled_f32_matches_torch_matmul(shape):
    m, k, n = shape
    a, b = O.normal((m, k), 1), O.normal((k, n), 2)
    got = O.matmul_tiled_f32(a, b)
    ref = (torch.from_numpy(a) @ torch.from_numpy(b)).numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-3, atol=1e-2)  # the reference's tolerance
    assert O.rel_l2(got, ref) < 1e-6
    assert O.rel_l2(got, O.matmul_f64(a, b)) < 1e-6


@pytest.mark.parametrize("shape", [(1, 1, 1), (5, 7, 3), (65, 17, 63)])
def test_f64_equals_bruteforce(shape):
    # fp32*fp32 is exact in fp64 and both sum in increasing k, so bit-exact.
    m, k, n = shape
    a, b = O.normal((m, k), 3), O.normal((k, n), 4)
    np.testing.assert_array_equal(O.matmul_f64(a, b), brute_f64(a, b))


@pytest.mark.parametrize("shape", [(1, 1, 1), (5, 7, 3), (65, 17, 63), (70, 40, 33)])
def test_tiled_f32_equals_stepwise_fp32_loop(shape):
    # Brute-force fp32 emulation of `acc = acc + dot(x, y)` per BK step.
    m, k, n = shape
    a, b = O.normal((m, k), 5), O.normal((k, n), 6)
    BK = 16
    acc = np.zeros((m, n), np.float32)
    for k0 in range(0, k, BK):
        d = np.zeros((m, n), np.float32)
        for kk in range(k0, min(k, k0 + BK)):
            d = (d + (a[:, kk:kk + 1] * b[kk:kk + 1, :]).astype(np.float32)).astype(np.float32)
        acc = (acc + d).astype(np.float32)
    np.testing.assert_array_equal(O.matmul_tiled_f32(a, b, 64, 64, BK), acc)


def test_golden_integer_products():
    g = np.load(GOLDEN)
    for i, (m, k, n) in enumerate(g["shapes"]):
        a = g[f"x1_{i}"].astype(np.float32)
        b = g[f"x2_{i}"].astype(np.float32)
        want = g[f"out_{i}"]
        np.testing.assert_array_equal(O.matmul_tiled_f32(a, b), want.astype(np.float32))
        np.testing.assert_array_equal(O.matmul_f64(a, b), want.astype(np.float64))
        a16, b16 = O.bf16_round(a), O.bf16_round(b)
        np.testing.assert_array_equal(O.bf16_to_f32(a16), a)  # small ints are exact in bf16
        np.testing.assert_array_equal(O.matmul_tiled_bf16(a16, b16), want.astype(np.float32))
        np.testing.assert_array_equal(O.matmul_bf16_f64(a16, b16), want.astype(np.float64))


def test_closed_forms():
    a = O.normal((37, 53), 7)
    eye = np.eye(53, dtype=np.float32)
    np.testing.assert_array_equal(O.matmul_tiled_f32(a, eye), a)
    np.testing.assert_array_equal(O.matmul_tiled_f32(np.eye(37, dtype=np.float32), a), a)
    ones_a, ones_b = np.ones((9, 1234), np.float32), np.ones((1234, 11), np.float32)
    np.testing.assert_array_equal(O.matmul_tiled_f32(ones_a, ones_b), np.full((9, 11), 1234.0, np.float32))
    # K == 0: the accumulator never leaves zero.
    np.testing.assert_array_equal(O.matmul_tiled_f32(np.zeros((3, 0), np.float32), np.zeros((0, 4), np.float32)),
                                  np.zeros((3, 4), np.float32))


def test_invariants():
    a, b = O.normal((70, 90), 8), O.normal((90, 50), 9)
    c = O.matmul_tiled_f32(a, b)
    # Scaling by a power of two is exact.
    np.testing.assert_array_equal(O.matmul_tiled_f32(4 * a, b), 4 * c)
    # (AB)^T = B^T A^T with the same products in the same order: bit-exact.
    np.testing.assert_array_equal(O.matmul_tiled_f32(b.T, a.T), c.T)
    # Zero padding of K (masked loads with other=0) changes nothing.
    ap = np.concatenate([a, np.zeros((70, 13), np.float32)], 1)
    bp = np.concatenate([b, np.zeros((13, 50), np.float32)], 0)
    np.testing.assert_array_equal(O.matmul_f64(ap, bp), O.matmul_f64(a, b))
    # K-split additivity.
    lo = O.matmul_f64(a[:, :37], b[:37]) + O.matmul_f64(a[:, 37:], b[37:])
    assert O.rel_l2(lo, O.matmul_f64(a, b)) < 1e-14
    # Linearity in the first operand.
    a2 = O.normal((70, 90), 10)
    assert O.rel_l2(O.matmul_f64(a + a2, b), O.matmul_f64(a, b) + O.matmul_f64(a2, b)) < 1e-6


def test_tile_sizes_do_not_change_masked_results():
    # Ragged shape; every tile edge partial for every tile size.
    a, b = O.small_ints((127, 1000), 11), O.small_ints((1000, 513), 12)
    want = (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32)
    for BM, BN, BK in [(64, 64, 16), (32, 16, 8), (128, 64, 64), (7, 5, 3)]:
        np.testing.assert_array_equal(O.matmul_tiled_f32(a, b, BM, BN, BK), want)


def test_bf16_rounding_known_answers():
    x = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -2.5, 0.0, -0.0, np.inf, -np.inf,
                  3.0e38, 1e-40], np.float32)
    got = O.bf16_round(x)
    assert got[0] == 0x3F80
    assert got[1] == 0x3F80          # tie -> even
    assert got[2] == 0x3F82          # tie -> even (up)
    assert got[3] == 0xC020
    assert got[4] == 0x0000 and got[5] == 0x8000
    assert got[6] == 0x7F80 and got[7] == 0xFF80
    nan = O.bf16_round(np.array([np.nan], np.float32))[0]
    assert (nan & 0x7F80) == 0x7F80 and (nan & 0x7F) != 0


def test_bf16_rounding_matches_torch():
    x = O.normal((100000,), 13) * np.float32(1e3)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(O.bf16_round(x), want)


def test_bf16_f64_matches_torch():
    a, b = O.normal((64, 300), 14), O.normal((300, 40), 15)
    a16, b16 = O.bf16_round(a), O.bf16_round(b)
    ta = torch.from_numpy(O.bf16_to_f32(a16)).double()
    tb = torch.from_numpy(O.bf16_to_f32(b16)).double()
    assert O.rel_l2(O.matmul_bf16_f64(a16, b16), (ta @ tb).numpy()) < 1e-14
    assert O.rel_l2(O.matmul_tiled_bf16(a16, b16), (ta @ tb).numpy()) < 1e-6


def test_planted_mistakes_are_caught():
    """Broken oracles (planted here, on the CPU) fail the checks above."""
    g = np.load(GOLDEN)
    a = g["x1_3"].astype(np.float32)
    b = g["x2_3"].astype(np.float32)
    want = g["out_3"].astype(np.float32)
    dropped_tail = O.matmul_tiled_f32(a[:, :-1], b[:-1])          # last k step lost
    transposed = O.matmul_tiled_f32(a, b[::-1].copy())             # B rows reversed
    sign = -O.matmul_tiled_f32(a, b)
    unmasked_edge = O.matmul_tiled_f32(a, b)
    unmasked_edge[-1, -1] += 1.0                                   # one edge element wrong
    for bad in (dropped_tail, transposed, sign, unmasked_edge):
        assert not np.array_equal(bad, want)
    # and the rel-L2 gate would reject them
    for bad in (dropped_tail, transposed, sign):
        assert O.rel_l2(bad, want) > O.TOL_F32


def test_rel_l2():
    assert O.rel_l2(np.zeros(3), np.zeros(3)) == 0.0
    assert O.rel_l2([1.0, 0.0], [0.0, 0.0]) == math.inf
    assert abs(O.rel_l2([3.0, 4.0], [3.0, 0.0]) - 4.0 / 3.0) < 1e-15


# ---------------------------------------------------------------------------
# Host integer helpers
# ---------------------------------------------------------------------------

def test_cdiv_known_answer():
    assert O.cdiv(5000, 4096) == 2  # tilec/language.py:17
    for a in range(0, 200):
        for b in range(1, 20):
            assert O.cdiv(a, b) == math.ceil(a / b)


def test_plan_known_answers():
    assert O.plan(300) == (1024, 1)
    assert O.plan(4096) == (4096, 1)
    assert O.plan(5000) == (4096, 2)
    assert O.plan(1) == (1, 1)
    assert O.plan(2) == (4, 1)
    assert O.plan(256) == (256, 1)
    assert O.plan(257) == (1024, 1)
    assert O.plan(100, block=64) == (64, 2)


def test_plan_characterisation():
    for n in range(1, 20000, 7):
        block, chunks = O.plan(n)
        # the smallest power of 4 that is >= n, capped at MAX_BLOCK
        p = 1
        while p < n:
            p *= 4
        assert block == min(p, O.MAX_BLOCK)
        assert chunks == math.ceil(n / block)


def test_mm_configs_characterisation():
    for M1, N, M2 in [(129, 256, 32), (1000, 4096, 100), (8, 48, 3), (1, 31, 1), (7, 20000, 9)]:
        got = set(O.mm_configs(M1, N, M2))
        want = set()
        for p in O.SPLITS:
            if p != 1 and N // p < 32:
                continue
            for r in O.JOINS:
                if r != 1 and M1 < r:
                    continue
                n = math.ceil(N / p)
                top = O.plan(n)[0]
                for b in list(O.BLOCKS) + [top]:
                    if b == top or (b < top and math.ceil(n / b) <= 16):
                        want.add((p, r, b))
        assert got == want
        assert len(got) == len(O.mm_configs(M1, N, M2))  # no duplicates


# Hand-derived known answers for the legacy config space (tilec/ext.py:29-51):
# blocks(n) keeps the BLOCKS below plan(n)'s block that cut n into at most 16
# chunks, then that block; mm_configs crosses the splits p with N // p >= 32,
# the joins r <= M1 and the blocks of cdiv(N, p).
BLOCKS_KNOWN = {
    1: [1],                      # plan(1) = (1, 1)
    31: [64],                    # plan(31): 64; no BLOCKS entry below 64
    300: [256, 1024],            # plan(300): 1024; 256 cuts 300 into 2
    4096: [256, 1024, 4096],     # 256 cuts 4096 into exactly 16
    5000: [1024, 4096],          # 256 would take 20 chunks; 1024 takes 5
    8192: [1024, 4096],          # block capped at 4096; 256 would take 32 chunks
}
MM_CONFIGS_KNOWN = {
    (1, 31, 1): [(1, 1, 64)],    # 31 // 2 < 32: no split; M1 = 1: no join
    (8, 48, 3): [(1, 1, 64), (1, 2, 64), (1, 4, 64), (1, 8, 64)],
}
MM_CONFIGS_COUNT = {
    (129, 256, 32): 16,          # p in 1, 2, 4, 8 (256 // 16 < 32) x 4 joins x one block each
    (4, 4096, 64): 39,           # 7 splits with 3 + 3 + 2 + 2 + 1 + 1 + 1 blocks, x joins 1, 2, 4
}


@pytest.mark.parametrize("impl", ["oracle", "ext"])
def test_blocks_and_mm_configs_known_answers(impl):
    from tilec import ext
    blocks = O.blocks if impl == "oracle" else ext._blocks
    mm_configs = O.mm_configs if impl == "oracle" else ext.mm_configs
    for n, want in BLOCKS_KNOWN.items():
        assert blocks(n) == want, n
    for args, want in MM_CONFIGS_KNOWN.items():
        assert mm_configs(*args) == want, args
    for args, count in MM_CONFIGS_COUNT.items():
        assert len(mm_configs(*args)) == count, args
    # (4, 4096, 64): the largest split keeps one 64-element block
    assert (64, 4, 64) in mm_configs(4, 4096, 64) and (64, 8, 64) not in mm_configs(4, 4096, 64)


# ---------------------------------------------------------------------------
# Sums (tl.sum, kernel1.py:8-15)
# ---------------------------------------------------------------------------

def test_sum_reference_example_known_answer():
    """kernel1.py:18-27 sums the rows of arange(32).reshape(4, 8) and checks
    them against numpy's x.sum(axis=1): row r holds 8r .. 8r+7, so its sum
    is 64r + 28; column c holds c, 8+c, 16+c, 24+c, so its sum is 48 + 4c."""
    x = np.arange(32, dtype=np.float32).reshape(4, 8)
    np.testing.assert_array_equal(O.sum_f64(x, 1), [28, 92, 156, 220])
    np.testing.assert_array_equal(O.sum_f64(x, 0), [48 + 4 * c for c in range(8)])
    np.testing.assert_array_equal(O.row_sum_f32_seq(x), [28, 92, 156, 220])


def test_sum_matches_brute_force_loops():
    for i, (r, c) in enumerate([(1, 1), (3, 7), (5, 1), (1, 33), (17, 65)]):
        x = O.normal((r, c), 900 + i)
        rows = [math.fsum(float(x[a, b]) for b in range(c)) for a in range(r)]
        cols = [math.fsum(float(x[a, b]) for a in range(r)) for b in range(c)]
        np.testing.assert_allclose(O.sum_f64(x, 1), rows, rtol=1e-13, atol=1e-13)
        np.testing.assert_allclose(O.sum_f64(x, 0), cols, rtol=1e-13, atol=1e-13)
        seq = O.row_sum_f32_seq(x)
        for a in range(r):  # the fp32 loop, element by element
            acc = np.float32(0)
            for b in range(c):
                acc = np.float32(acc + x[a, b])
            assert seq[a] == acc


def test_sum_invariants_and_error_bound():
    x = O.normal((300, 257), 910)
    assert math.isclose(O.sum_f64(x, 1).sum(), O.sum_f64(x, 0).sum(), rel_tol=1e-12, abs_tol=1e-9)
    y = O.normal((300, 257), 911)
    np.testing.assert_allclose(O.sum_f64(x + y, 1), O.sum_f64(x, 1) + O.sum_f64(y, 1), rtol=1e-6, atol=1e-5)
    assert O.sum_error_ok(O.row_sum_f32_seq(x), x, 1)
    # the bound rejects a dropped element (a plausible off-by-one)
    assert not O.sum_error_ok(O.row_sum_f32_seq(x[:, :-1]), x, 1)
    assert not O.sum_error_ok(O.sum_f64(x, 1) + 1e-3, x, 1)
