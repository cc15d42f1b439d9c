"""GPU parity: tilec.ext.matrix_mul on an MI355X against the CPU oracle.

The reference's own GPU test (tests/test_matmul.py:32-40) compares
`ext.matrix_mul` with `x1 @ x2` on five shapes at rtol=1e-3, atol=1e-2; that
is kept as a floor.  On top: rel-L2 <= 1e-5 (fp32) / 1e-2 (bf16) against the
fp64 oracle (oracle/matmul_oracle.c) for every BASELINE config, every
compiled variant on ragged shapes, bit-exact integer known answers, and
size-independent properties at full size.  Inputs are seeded numpy draws
made on the CPU, so the GPU and the oracle see identical values.
"""

import math

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tilec import _lib, ext
import tilec

pytestmark = pytest.mark.gpu

GOLDEN = __import__("os").path.join(__import__("os").path.dirname(__file__), "golden", "int_products.npz")


def say(msg):
    print(msg, flush=True)


def dev(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda").to(dtype)


def dev_bf16(h):
    """uint16 bf16 bit patterns -> bf16 device tensor."""
    return torch.from_numpy(np.ascontiguousarray(h).view(np.int16)).to("cuda").view(torch.bfloat16)


def run(x1, x2, config=None):
    out = ext.matrix_mul(x1, x2, config)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def f32_variants():
    return [v["name"] for v in _lib.variants() if v["dtype"] == _lib.F32]


def bf16_variants():
    return [v["name"] for v in _lib.variants() if v["dtype"] == _lib.BF16]


# ---------------------------------------------------------------------------
# The reference's parity test, kept as the floor
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("shape", [(1, 1, 1), (5, 7, 3), (65, 17, 63), (128, 300, 130), (512, 1024, 256)])
def test_matrix_mul_reference_shapes(shape):
    m, k, n = shape
    say(f"reference shape {shape}")
    a, b = O.normal((m, k), 100), O.normal((k, n), 101)
    got = tilec.ext.matrix_mul(dev(a), dev(b))
    torch.cuda.synchronize()
    got = got.cpu().numpy()
    assert got.dtype == np.float32 and got.shape == (m, n)
    ref = (torch.from_numpy(a) @ torch.from_numpy(b)).numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-3, atol=1e-2)  # tests/test_matmul.py:40
    assert O.rel_l2(got, O.matmul_f64(a, b)) <= O.TOL_F32


# ---------------------------------------------------------------------------
# Exact known answers, every variant
# ---------------------------------------------------------------------------

def test_golden_integer_products_every_variant():
    g = np.load(GOLDEN)
    for i, (m, k, n) in enumerate(g["shapes"]):
        a = g[f"x1_{i}"].astype(np.float32)
        b = g[f"x2_{i}"].astype(np.float32)
        want = g[f"out_{i}"].astype(np.float32)
        for cfg in ext.hip_configs(int(m), int(k), int(n), "f32"):
            say(f"golden {i} {(m, k, n)} f32 {cfg}")
            np.testing.assert_array_equal(run(dev(a), dev(b), cfg), want)
        a16, b16 = O.bf16_round(a), O.bf16_round(b)
        for cfg in ext.hip_configs(int(m), int(k), int(n), "bf16"):
            say(f"golden {i} {(m, k, n)} bf16 {cfg}")
            np.testing.assert_array_equal(run(dev_bf16(a16), dev_bf16(b16), cfg), want)


# ---------------------------------------------------------------------------
# Every variant on ragged shapes
# ---------------------------------------------------------------------------

RAGGED = [(1, 1, 1), (3, 5, 7), (16, 64, 64), (17, 31, 65), (33, 100, 257), (127, 1000, 513),
          (200, 129, 63), (257, 300, 129), (64, 4097, 33)]


@pytest.mark.parametrize("name", f32_variants())
def test_f32_variant_ragged(name):
    v = _lib.variants()[_lib.variant_id(name)]
    for i, (m, k, n) in enumerate(RAGGED):
        if v["max_m"] and m > v["max_m"]:
            continue
        a, b = O.normal((m, k), 200 + 2 * i), O.normal((k, n), 201 + 2 * i)
        ref = O.matmul_f64(a, b)
        splits = [1] if v["family"] == _lib.FAMILY_GEMM else [1, 2, 3, 8]
        for s in splits:
            say(f"{name} split {s} shape {(m, k, n)}")
            got = run(dev(a), dev(b), (name, s))
            assert O.rel_l2(got, ref) <= O.TOL_F32, (name, s, (m, k, n))


@pytest.mark.parametrize("name", bf16_variants())
def test_bf16_variant_ragged(name):
    v = _lib.variants()[_lib.variant_id(name)]
    for i, (m, k, n) in enumerate(RAGGED):
        if v["max_m"] and m > v["max_m"]:
            continue
        a16 = O.bf16_round(O.normal((m, k), 300 + 2 * i))
        b16 = O.bf16_round(O.normal((k, n), 301 + 2 * i))
        say(f"{name} shape {(m, k, n)}")
        got = run(dev_bf16(a16), dev_bf16(b16), (name, 1))
        # fp32 accumulation of exact bf16 inputs: far inside the 1e-2 gate
        assert O.rel_l2(got, O.matmul_bf16_f64(a16, b16)) <= 1e-5, (name, (m, k, n))


def _splittable(dtype_code):
    return [v["name"] for v in _lib.variants()
            if v["family"] == _lib.FAMILY_GEMM and v["dtype"] == dtype_code and ext.tile_can_split(v)]


SPLIT_SHAPES = [(1, 1000, 65), (17, 4097, 33), (64, 1024, 64), (127, 1000, 513), (200, 3001, 129), (520, 2048, 300)]


@pytest.mark.parametrize("name", _splittable(_lib.F32) + _splittable(_lib.BF16))
def test_gemm_split_k(name):
    """K split across workgroups of a tile GEMM: partial tiles combined by the
    last split in split order — oracle parity, bit-exact integers, and the
    same bits on a repeat call."""
    v = _lib.variants()[_lib.variant_id(name)]
    bf16 = v["dtype"] == _lib.BF16
    for i, (m, k, n) in enumerate(SPLIT_SHAPES):
        if bf16:
            a16 = O.bf16_round(O.normal((m, k), 700 + 2 * i))
            b16 = O.bf16_round(O.normal((k, n), 701 + 2 * i))
            x1, x2, ref, tol = dev_bf16(a16), dev_bf16(b16), O.matmul_bf16_f64(a16, b16), 1e-5
        else:
            a, b = O.normal((m, k), 700 + 2 * i), O.normal((k, n), 701 + 2 * i)
            x1, x2, ref, tol = dev(a), dev(b), O.matmul_f64(a, b), O.TOL_F32
        for s in (2, 3, 8):
            say(f"{name} split {s} shape {(m, k, n)}")
            got = run(x1, x2, (name, s))
            assert O.rel_l2(got, ref) <= tol, (name, s, (m, k, n))
            np.testing.assert_array_equal(run(x1, x2, (name, s)), got)
    rng = np.random.default_rng(5)
    a = rng.integers(-3, 4, (70, 1500)).astype(np.float32)
    b = rng.integers(-3, 4, (1500, 90)).astype(np.float32)
    want = (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32)
    if bf16:
        x1, x2 = dev(a).to(torch.bfloat16), dev(b).to(torch.bfloat16)  # small integers are exact in bf16
    else:
        x1, x2 = dev(a), dev(b)
    for s in (1, 4, 7):
        np.testing.assert_array_equal(run(x1, x2, (name, s)), want)


def test_skinny_shapes_and_splits():
    for m in (1, 2, 4, 7, 15, 16):
        for k, n in [(1, 1), (5, 63), (1000, 65), (4096, 130), (4097, 4096)]:
            a, b = O.normal((m, k), 7 * m + k), O.normal((k, n), 7 * m + k + 1)
            ref = O.matmul_f64(a, b)
            for cfg in ext.hip_configs(m, k, n, "f32"):
                if not cfg[0].startswith("skinny"):
                    continue
                got = run(dev(a), dev(b), cfg)
                assert O.rel_l2(got, ref) <= O.TOL_F32, (cfg, (m, k, n))
            say(f"skinny m={m} k={k} n={n} ok")


def test_skinny_bf16():
    """bf16 inputs on the streaming kernel (widened to fp32 in registers):
    aligned and unaligned shapes, every split the tuner may pick."""
    for m in (1, 4, 16):
        for k, n in [(64, 128), (1000, 136), (4096, 4096), (4097, 130), (333, 1000)]:
            a16 = O.bf16_round(O.normal((m, k), 11 * m + k))
            b16 = O.bf16_round(O.normal((k, n), 11 * m + k + 1))
            ref = O.matmul_bf16_f64(a16, b16)
            cfgs = [c for c in ext.hip_configs(m, k, n, "bf16") if c[0].startswith("skinny")]
            assert cfgs
            for cfg in cfgs:
                got = run(dev_bf16(a16), dev_bf16(b16), cfg)
                assert O.rel_l2(got, ref) <= 1e-5, (cfg, (m, k, n))
            say(f"skinny bf16 m={m} k={k} n={n}: {len(cfgs)} configs ok")
    rng = np.random.default_rng(3)
    a = rng.integers(-3, 4, (9, 2000)).astype(np.float32)
    b = rng.integers(-3, 4, (2000, 300)).astype(np.float32)
    want = (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32)
    for cfg in [("skinny_bf16_w4_b1", 1), ("skinny_bf16_w8_b2", 8), ("skinny_bf16_w4_b2", 3)]:
        np.testing.assert_array_equal(run(dev(a).to(torch.bfloat16), dev(b).to(torch.bfloat16), cfg), want)


def test_skinny_fma_path():
    """The FMA variants (M <= 1 or 4, row-major x2; a column-major x2 runs the
    MFMA path): every M up to the variant's bound, ragged and aligned K and
    N, row- and column-major x1, split K, against the fp64 oracle; small
    integers bit-exact."""
    # (the row-tile variants for x @ W.T, M <= 16, are covered by test_gemv_rows_kernel)
    fma = [v for v in _lib.variants() if v["family"] == _lib.FAMILY_SKINNY and v["max_m"] in (1, 4)
           and not v["name"].endswith(("_c128", "_c256"))]
    # 8 streaming FMA variants, 8 row-dot variants for x @ W.T, 6 panel variants
    assert len(fma) == 22
    for v in fma:
        bf = v["dtype"] == _lib.BF16
        for m in range(1, v["max_m"] + 1):
            for i, (k, n) in enumerate([(1, 1), (5, 63), (1000, 65), (4096, 136), (4097, 130), (333, 1000)]):
                a, b = O.normal((m, k), 40 * m + i), O.normal((k, n), 40 * m + i + 20)
                if bf:
                    a, b = O.bf16_round(a), O.bf16_round(b)
                ref = O.matmul_bf16_f64(a, b) if bf else O.matmul_f64(a, b)
                mk = dev_bf16 if bf else dev
                for layout in (0, _lib.X1_COL_MAJOR, _lib.X2_COL_MAJOR):
                    for s in (1, 3, 8):
                        say(f"{v['name']} m={m} k={k} n={n} layout {layout} split {s}")
                        got = run_layout(mk(a), mk(b), layout, (v["name"], s))
                        assert O.rel_l2(got, ref) <= (1e-5 if bf else O.TOL_F32), (v["name"], m, k, n, layout, s)
    rng = np.random.default_rng(21)
    for m in (1, 3, 4):
        a = rng.integers(-3, 4, (m, 3001)).astype(np.float32)
        b = rng.integers(-3, 4, (3001, 260)).astype(np.float32)
        want = (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32)
        for v in fma:
            if m > v["max_m"]:
                continue
            conv = (lambda x: dev(x).to(torch.bfloat16)) if v["dtype"] == _lib.BF16 else dev
            for s in (1, 5):
                np.testing.assert_array_equal(run(conv(a), conv(b), (v["name"], s)), want)


def panel_variants():
    return [v for v in _lib.variants() if ext.panel_variant(v)]


def test_panel_kernel():
    """The panel kernel (512-byte pieces of each x2 row, M <= 4, row-major
    x2): every M up to each variant's bound, K ragged (odd, not a multiple
    of 16) and aligned, N a multiple of the 16-byte group with a partial last
    panel, row- and column-major x1, unsplit and split K, against the fp64
    oracle.  Shapes it does not take (N % group != 0) run the streaming
    fallback and are checked the same way."""
    pv = panel_variants()
    assert len(pv) == 6
    shapes = [(16, 8), (36, 136), (1004, 264), (4096, 4096), (4097, 520), (333, 1000), (100, 4), (1, 256)]
    for v in pv:
        bf = v["dtype"] == _lib.BF16
        for m in range(1, v["max_m"] + 1):
            for i, (k, n) in enumerate(shapes):
                a, b = O.normal((m, k), 60 * m + i), O.normal((k, n), 60 * m + i + 30)
                if bf:
                    a, b = O.bf16_round(a), O.bf16_round(b)
                ref = O.matmul_bf16_f64(a, b) if bf else O.matmul_f64(a, b)
                mk = dev_bf16 if bf else dev
                for layout in (0, _lib.X1_COL_MAJOR):
                    for s in (1, 3, 8, 64):
                        say(f"{v['name']} m={m} k={k} n={n} layout {layout} split {s}")
                        got = run_layout(mk(a), mk(b), layout, (v["name"], s))
                        assert O.rel_l2(got, ref) <= (1e-5 if bf else O.TOL_F32), (v["name"], m, k, n, layout, s)


def test_panel_exact_and_deterministic():
    """Small integers: every partial sum is exact in fp32, so any split and
    summation order gives the int64 product bit for bit; a repeat call gives
    the same bits; the counters are zero again after every call."""
    rng = np.random.default_rng(31)
    L = _lib.lib()
    for m in (1, 3, 4, 9, 16):
        a = rng.integers(-3, 4, (m, 3008)).astype(np.float32)
        b = rng.integers(-3, 4, (3008, 392)).astype(np.float32)
        want = (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32)
        for v in panel_variants():
            if m > v["max_m"]:
                continue
            conv = (lambda x: dev(x).to(torch.bfloat16)) if v["dtype"] == _lib.BF16 else dev
            x1, x2 = conv(a), conv(b)
            for s in (1, 2, 7, 16):
                say(f"{v['name']} exact m={m} split {s}")
                got = run(x1, x2, (v["name"], s))
                np.testing.assert_array_equal(got, want)
                np.testing.assert_array_equal(run(x1, x2, (v["name"], s)), got)
                stream = torch.cuda.current_stream().cuda_stream
                cnt = ext._COUNTERS.get((x1.device.index, stream))
                if cnt is not None:
                    assert torch.count_nonzero(cnt).item() == 0, (v["name"], m, s)
    # config 1 size with every panel variant, against the oracle
    for m in (1, 4, 16):
        a, b = O.normal((m, 4096), 900 + m), O.normal((4096, 4096), 901)
        ref = O.matmul_f64(a, b)
        for v in panel_variants():
            if m > v["max_m"] or v["dtype"] != _lib.F32:
                continue
            for s in (0, 8, 16):
                say(f"{v['name']} config-1 m={m} split {s}")
                assert O.rel_l2(run(dev(a), dev(b), (v["name"], s)), ref) <= O.TOL_F32


def direct_variants():
    return [v for v in _lib.variants() if v["family"] == _lib.FAMILY_DIRECT]


DIRECT_SHAPES = [(1, 4096, 4096), (4, 4096, 4096), (16, 4096, 4096), (7, 1000, 65), (16, 37, 3001),
                 (513, 3001, 127), (127, 1000, 513), (512, 4096, 64), (100, 4097, 33), (33, 16, 1),
                 (1024, 1024, 1024), (1100, 333, 1500)]


def test_direct_kernel():
    """The direct-operand MFMA kernel (operands loaded straight into MFMA
    registers, K split over waves and workgroups): the GEMV, small-output and
    1024^3 BASELINE shapes plus ragged ones (K and N not multiples of 4, M
    past a tile), every layout, unsplit and split K, against the fp64
    oracle."""
    dv = direct_variants()
    assert len(dv) == 11
    for i, (m, k, n) in enumerate(DIRECT_SHAPES):
        a, b = O.normal((m, k), 1100 + 2 * i), O.normal((k, n), 1101 + 2 * i)
        ref = O.matmul_f64(a, b)
        x1, x2 = dev(a), dev(b)
        for v in dv:
            for layout in (0, *LAYOUTS):
                for s in (1, 5, 16):
                    say(f"{v['name']} {(m, k, n)} layout {layout} split {s}")
                    got = run_layout(x1, x2, layout, (v["name"], s))
                    assert O.rel_l2(got, ref) <= O.TOL_F32, (v["name"], (m, k, n), layout, s)


def test_direct_exact_unaligned_and_deterministic():
    """Small integers (every partial sum exact in fp32): any split and
    summation order gives the int64 product bit for bit, also from operands
    whose base is only 4-byte aligned (views at flat[1:]) and with padded
    row strides; a repeat call gives the same bits; the counters are zero
    again after every call."""
    rng = np.random.default_rng(41)
    for m, k, n in [(1, 3008, 392), (9, 777, 131), (16, 2051, 260), (70, 1500, 90), (513, 301, 127)]:
        a = rng.integers(-3, 4, (m, k)).astype(np.float32)
        b = rng.integers(-3, 4, (k, n)).astype(np.float32)
        want = (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32)
        fa = torch.zeros(m * k + 1, device="cuda")
        fa[1:] = dev(a).flatten()
        fb = torch.zeros(k * (n + 3) + 1, device="cuda")
        fb[1:].view(k, n + 3)[:, :n] = dev(b)
        x1s = [dev(a), fa[1:].view(m, k)]
        x2s = [dev(b), fb[1:].view(k, n + 3)[:, :n]]
        assert x1s[1].data_ptr() % 16 == 4 and x2s[1].data_ptr() % 16 == 4
        for v in direct_variants():
            for x1, x2 in zip(x1s, x2s):
                for s in (1, 3, 16, 64):
                    say(f"{v['name']} exact {(m, k, n)} split {s} base %16 = {x1.data_ptr() % 16}")
                    got = run(x1, x2, (v["name"], s))
                    np.testing.assert_array_equal(got, want)
                    np.testing.assert_array_equal(run(x1, x2, (v["name"], s)), got)
                    stream = torch.cuda.current_stream().cuda_stream
                    cnt = ext._COUNTERS.get((x1.device.index, stream))
                    if cnt is not None:
                        assert torch.count_nonzero(cnt).item() == 0, (v["name"], (m, k, n), s)


def test_skinny_row_blocks():
    """M > 16 on the streaming kernel: one grid row block per 16 rows of x1,
    each with its own partial slots and counters (every skinny config the
    tuner may pick for these small outputs)."""
    for i, (m, k, n) in enumerate([(17, 64, 64), (40, 1000, 65), (127, 1000, 513), (513, 3001, 127),
                                   (512, 4096, 64)]):
        a, b = O.normal((m, k), 500 + 2 * i), O.normal((k, n), 501 + 2 * i)
        ref = O.matmul_f64(a, b)
        cfgs = [c for c in ext.hip_configs(m, k, n, "f32") if c[0].startswith("skinny")]
        assert cfgs, (m, k, n)
        for cfg in cfgs:
            got = run(dev(a), dev(b), cfg)
            assert O.rel_l2(got, ref) <= O.TOL_F32, (cfg, (m, k, n))
        say(f"skinny row blocks m={m} k={k} n={n}: {len(cfgs)} configs ok")
    # Bit-exact on small integers (every partial sum exact in fp32), ragged
    # last row block and slab.
    rng = np.random.default_rng(11)
    a = rng.integers(-3, 4, (37, 777)).astype(np.float32)
    b = rng.integers(-3, 4, (777, 131)).astype(np.float32)
    want = (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32)
    for cfg in [("skinny_f32_w4_b1", 3), ("skinny_f32_w8_b2", 8), ("skinny_f32_w16_b1", 1)]:
        np.testing.assert_array_equal(run(dev(a), dev(b), cfg), want)


# ---------------------------------------------------------------------------
# BASELINE.json configs (seeds 2i / 2i+1 for config i)
# ---------------------------------------------------------------------------

def test_config0_readme_example():
    say("config 0: [512,4096] @ [4096,64]")
    a, b = O.normal((512, 4096), 0), O.normal((4096, 64), 1)
    got = run(dev(a), dev(b))
    assert O.rel_l2(got, O.matmul_f64(a, b)) <= O.TOL_F32
    assert O.rel_l2(got, O.matmul_tiled_f32(a, b)) <= O.TOL_F32
    ref = (torch.from_numpy(a) @ torch.from_numpy(b)).numpy()
    assert O.rel_l2(got, ref) <= O.TOL_F32


@pytest.mark.parametrize("m", [1, 4, 16])
def test_config1_skinny(m):
    say(f"config 1: M={m} K=N=4096")
    a, b = O.normal((m, 4096), 2), O.normal((4096, 4096), 3)
    got = run(dev(a), dev(b))
    assert O.rel_l2(got, O.matmul_f64(a, b)) <= O.TOL_F32
    ref = (torch.from_numpy(a) @ torch.from_numpy(b)).numpy()
    assert O.rel_l2(got, ref) <= O.TOL_F32


@pytest.mark.parametrize("n", [1024, 2048])
def test_config2_square_full(n):
    say(f"config 2: {n}^3 fp32")
    a, b = O.uniform((n, n), 4), O.uniform((n, n), 5)
    got = run(dev(a), dev(b))
    assert O.rel_l2(got, O.matmul_f64(a, b)) <= O.TOL_F32


def _sample_rows(M, count, seed):
    rng = np.random.default_rng(seed)
    rows = np.unique(np.concatenate([[0, M - 1], rng.choice(M, size=count, replace=False)]))
    return rows


def test_config2_square_4096():
    say("config 2: 4096^3 fp32 (sampled rows + properties)")
    n = 4096
    a, b = O.uniform((n, n), 4), O.uniform((n, n), 5)
    da, db = dev(a), dev(b)
    got = ext.matrix_mul(da, db)
    rows = _sample_rows(n, 192, 0)
    ref = O.matmul_f64(a[rows], b)
    assert O.rel_l2(got[torch.from_numpy(rows).cuda()].cpu().numpy(), ref) <= O.TOL_F32
    # deterministic and exactly linear under power-of-two scaling
    again = ext.matrix_mul(da, db)
    scaled = ext.matrix_mul(da * 2, db)
    torch.cuda.synchronize()
    assert torch.equal(got, again)
    assert torch.equal(scaled, got * 2)
    # column block consistency: a column slice of B gives the same columns,
    # bit for bit with the full product's config (an output tile's K order
    # does not depend on N), and to fp32 accuracy with the slice's own pick
    # (which may be another kernel with another summation order)
    full_cfg = ext._tuned(n, n, n, "f32", 0)
    db_sub = db[:, :1024].contiguous()
    same = ext.matrix_mul(da, db_sub, full_cfg)
    sub = ext.matrix_mul(da, db_sub)
    torch.cuda.synchronize()
    assert torch.equal(same, got[:, :1024])
    assert O.rel_l2(sub.cpu().numpy(), got[:, :1024].cpu().numpy()) <= O.TOL_F32


@pytest.mark.parametrize("shape", [(127, 1000, 513), (513, 3001, 127), (1000, 4097, 3001), (3001, 513, 1000)])
def test_config3_ragged(shape):
    m, k, n = shape
    say(f"config 3: ragged {shape}")
    a, b = O.normal((m, k), 6), O.normal((k, n), 7)
    got = run(dev(a), dev(b))
    assert O.rel_l2(got, O.matmul_f64(a, b)) <= O.TOL_F32


def test_config4_bf16_8192():
    say("config 4: bf16 8192^3 (sampled rows + properties)")
    n = 8192
    sigma = n ** -0.25  # sigma^2 = K^-1/2
    a16 = O.bf16_round(O.normal((n, n), 8, std=sigma))
    b16 = O.bf16_round(O.normal((n, n), 9, std=sigma))
    da, db = dev_bf16(a16), dev_bf16(b16)
    got = ext.matrix_mul(da, db)
    torch.cuda.synchronize()
    assert got.dtype == torch.float32 and got.shape == (n, n)
    rows = _sample_rows(n, 62, 1)
    g = got[torch.from_numpy(rows).cuda()].cpu().numpy()
    ref64 = O.matmul_bf16_f64(a16[rows], b16)
    assert O.rel_l2(g, ref64) <= O.TOL_BF16
    assert O.rel_l2(g, ref64) <= 1e-5  # what fp32 accumulation actually achieves
    # the north star's oracle: fp32 CPU matmul of the same bf16-rounded inputs
    ref32 = (torch.from_numpy(O.bf16_to_f32(a16[rows])) @ torch.from_numpy(O.bf16_to_f32(b16))).numpy()
    assert O.rel_l2(g, ref32) <= O.TOL_BF16
    again = ext.matrix_mul(da, db)
    torch.cuda.synchronize()
    assert torch.equal(got, again)


# ---------------------------------------------------------------------------
# Edge cases
# ---------------------------------------------------------------------------

def test_empty_and_zero_k():
    for m, k, n in [(0, 5, 7), (5, 7, 0), (0, 0, 0), (4, 0, 6), (40, 0, 300)]:
        for dt in (torch.float32, torch.bfloat16):
            x1 = torch.randn(m, k, device="cuda").to(dt)
            x2 = torch.randn(k, n, device="cuda").to(dt)
            out = ext.matrix_mul(x1, x2)
            torch.cuda.synchronize()
            assert out.shape == (m, n) and out.dtype == torch.float32
            assert torch.count_nonzero(out).item() == 0
    say("empty / K=0 ok")


def test_nonfinite_stays_local():
    # An Inf in the last row/column must not leak into other outputs through
    # masked (padded) lanes: edge handling selects zeros, never reads garbage.
    for m, k, n in [(3, 37, 70), (100, 37, 70), (300, 129, 300)]:
        a, b = O.normal((m, k), 11), O.normal((k, n), 12)
        a[-1, -1] = np.inf
        b[-1, -1] = np.nan
        for cfg in ext.hip_configs(m, k, n, "f32"):
            got = run(dev(a), dev(b), cfg)
            ref = O.matmul_f64(a, b)
            finite = np.isfinite(ref)
            assert np.array_equal(np.isfinite(got), finite), cfg
            assert O.rel_l2(got[finite], ref[finite]) <= O.TOL_F32, cfg
    say("non-finite locality ok")


def test_strided_and_transposed_inputs():
    a, b = O.normal((300, 200), 13), O.normal((200, 150), 14)
    ref = O.matmul_f64(a, b)
    da, db = dev(a), dev(b)
    # row-strided and transposed views are read in place
    big_a = torch.zeros(300, 260, device="cuda")
    big_a[:, :200] = da
    big_b = torch.zeros(200, 170, device="cuda")
    big_b[:, :150] = db
    for x1, x2 in [(big_a[:, :200], big_b[:, :150]), (da.t().contiguous().t(), db),
                   (da, db.t().contiguous().t()), (big_a[:, :200], db.t().contiguous().t())]:
        assert O.rel_l2(run(x1, x2), ref) <= O.TOL_F32
    # skinny path with a strided x2
    a1 = O.normal((4, 200), 15)
    assert O.rel_l2(run(dev(a1), big_b[:, :150]), O.matmul_f64(a1, b)) <= O.TOL_F32
    # a view that is neither row- nor column-major ([300, 100], strides (260, 2)) is copied first
    b2 = O.normal((100, 150), 16)
    assert O.rel_l2(run(big_a[:, :200][:, ::2], dev(b2)), O.matmul_f64(np.ascontiguousarray(a[:, ::2]), b2)) <= O.TOL_F32
    say("strided ok")


# ---------------------------------------------------------------------------
# Column-major operands (transposed views), read in place by every variant
# ---------------------------------------------------------------------------

LAYOUTS = [_lib.X1_COL_MAJOR, _lib.X2_COL_MAJOR, _lib.X1_COL_MAJOR | _lib.X2_COL_MAJOR]


def laid_out(x, col, pad=0):
    """The [r, c] device matrix x as a column-major view (x.T of a [c, r + pad]
    row-major buffer, leading dimension r + pad) when col, else as is."""
    if not col:
        return x
    r, c = x.shape
    buf = torch.zeros((c, r + pad), dtype=x.dtype, device=x.device)
    buf[:, :r] = x.t()
    return buf[:, :r].t()


def run_layout(x1, x2, layout, config=None, pad=0):
    v1 = laid_out(x1, layout & _lib.X1_COL_MAJOR, pad)
    v2 = laid_out(x2, layout & _lib.X2_COL_MAJOR, pad)
    # a vector is both row- and column-major (ext takes row-major): check
    # the layout bits of the operands that are matrices
    got = ext.layout_of(v1, v2)
    for bit, x in ((_lib.X1_COL_MAJOR, x1), (_lib.X2_COL_MAJOR, x2)):
        if min(x.shape) > 1:
            assert got & bit == layout & bit, (layout, got, tuple(x.shape))
    return run(v1, v2, config)


LAYOUT_SHAPES = RAGGED + [(64, 256, 256), (200, 516, 132), (256, 512, 256), (264, 200, 392), (8, 1032, 520)]


@pytest.mark.parametrize("name", f32_variants())
def test_f32_variant_layouts(name):
    v = _lib.variants()[_lib.variant_id(name)]
    for layout in LAYOUTS:
        for i, (m, k, n) in enumerate(LAYOUT_SHAPES):
            if v["max_m"] and m > v["max_m"]:
                continue
            a, b = O.normal((m, k), 500 + 2 * i), O.normal((k, n), 501 + 2 * i)
            ref = O.matmul_f64(a, b)
            splits = [1] if v["family"] == _lib.FAMILY_GEMM else [1, 3, 8]
            for s in splits:
                say(f"{name} layout {layout} split {s} shape {(m, k, n)}")
                got = run_layout(dev(a), dev(b), layout, (name, s))
                assert O.rel_l2(got, ref) <= O.TOL_F32, (name, layout, s, (m, k, n))


@pytest.mark.parametrize("name", bf16_variants())
def test_bf16_variant_layouts(name):
    v = _lib.variants()[_lib.variant_id(name)]
    for layout in LAYOUTS:
        for i, (m, k, n) in enumerate(LAYOUT_SHAPES):
            if v["max_m"] and m > v["max_m"]:
                continue
            a16 = O.bf16_round(O.normal((m, k), 600 + 2 * i))
            b16 = O.bf16_round(O.normal((k, n), 601 + 2 * i))
            ref = O.matmul_bf16_f64(a16, b16)
            splits = [1] if v["family"] == _lib.FAMILY_GEMM else [1, 3, 8]
            for s in splits:
                say(f"{name} layout {layout} split {s} shape {(m, k, n)}")
                got = run_layout(dev_bf16(a16), dev_bf16(b16), layout, (name, s))
                assert O.rel_l2(got, ref) <= 1e-5, (name, layout, s, (m, k, n))


# (M, K steps, N): K = steps x the variant's K step
M16_STEP_SHAPES = [(300, 1, 260), (300, 3, 260), (257, 5, 513), (300, 6, 260), (520, 33, 264), (64, 10, 600)]


@pytest.mark.parametrize("name", [v["name"] for v in _lib.variants() if "_m16" in v["name"]])
def test_bf16_m16_step_counts(name):
    """The 16x16x32 tile kernels with K a multiple of their K step: odd and
    even step counts (a 32-deep step runs an odd count as the next even one,
    the extra step on zeros) and the remainder after the unrolled ring, in
    every layout: the fp64 oracle on bf16 inputs, and the exact integer
    product on small integers."""
    v = _lib.variants()[_lib.variant_id(name)]
    for i, (m, steps, n) in enumerate(M16_STEP_SHAPES):
        k = steps * v["bk"]
        a16 = O.bf16_round(O.normal((m, k), 640 + 2 * i))
        b16 = O.bf16_round(O.normal((k, n), 641 + 2 * i))
        ref = O.matmul_bf16_f64(a16, b16)
        ai = O.small_ints((m, k), 660 + 2 * i, -3, 3)
        bi = O.small_ints((k, n), 661 + 2 * i, -3, 3)
        want = (ai.astype(np.int64) @ bi.astype(np.int64)).astype(np.float32)
        for layout in [0] + LAYOUTS:
            say(f"{name} layout {layout} shape {(m, k, n)}")
            got = run_layout(dev_bf16(a16), dev_bf16(b16), layout, (name, 1))
            assert O.rel_l2(got, ref) <= 1e-5, (name, layout, (m, k, n))
            got = run_layout(dev(ai, torch.bfloat16), dev(bi, torch.bfloat16), layout, (name, 1))
            np.testing.assert_array_equal(got, want)


def test_f32_lds_copies_strides_and_fallbacks():
    """The fp32 tiles with direct-to-LDS copies (*_lds) against the fp64
    oracle and, where the library has one, the register-staged variant of
    the same tile, bit for bit: row strides padded to a multiple of 4 (the copies' path), strides
    and bases that are not (a flat[1:] view, a stride of N + 3: the
    register-staged fallback), K tails, partial edge tiles, every layout, and
    K splits for the tiles that split."""
    lds = [v for v in _lib.variants() if v["name"].endswith("_lds")]
    assert len(lds) == 5
    names = {v["name"] for v in _lib.variants()}
    shapes = [(256, 512, 256), (300, 260, 196), (130, 1004, 72), (64, 32, 64), (520, 4100, 264)]
    for i, (m, k, n) in enumerate(shapes):
        a, b = O.normal((m, k), 1300 + 2 * i), O.normal((k, n), 1301 + 2 * i)
        ref = O.matmul_f64(a, b)
        fa = torch.zeros(m * k + 1, device="cuda")
        fa[1:] = dev(a).flatten()
        views = {"aligned": (dev(a), dev(b)), "unaligned x1 base": (fa[1:].view(m, k), dev(b))}
        for v in lds:
            base = v["name"][:-4]
            splits = [1, 3] if ext.tile_can_split(v) else [1]
            for s in splits:
                for label in ("aligned", "unaligned x1 base"):
                    x1, x2 = views[label]
                    say(f"{v['name']} split {s} {label} shape {(m, k, n)}")
                    got = ext.matrix_mul(x1, x2, (v["name"], s))
                    if base in names:  # the 64x64 tiles have no register-staged variant of their own
                        assert torch.equal(got, ext.matrix_mul(x1, x2, (base, s))), (v["name"], s, label, (m, k, n))
                    assert O.rel_l2(got.cpu().numpy(), ref) <= O.TOL_F32, (v["name"], s, label, (m, k, n))
                for layout in [0] + LAYOUTS:
                    for pad in (4, 3):
                        say(f"{v['name']} split {s} layout {layout} pad {pad} shape {(m, k, n)}")
                        got = run_layout(dev(a), dev(b), layout, (v["name"], s), pad=pad)
                        if base in names:
                            np.testing.assert_array_equal(got, run_layout(dev(a), dev(b), layout, (base, s), pad=pad))
                        assert O.rel_l2(got, ref) <= O.TOL_F32, (v["name"], s, layout, pad, (m, k, n))


def _view_at(x, col, off, extra):
    """The [r, c] device matrix x copied into a flat buffer at element offset
    `off`, row-major (or column-major when col) with a leading dimension
    `extra` elements longer than needed."""
    r, c = x.shape
    ld = (r if col else c) + extra
    flat = torch.zeros(off + ld * (c if col else r) + 1, dtype=x.dtype, device=x.device)
    v = flat[off:].as_strided((r, c), (1, ld) if col else (ld, 1))
    v.copy_(x)
    return v


def test_pad_variants_any_alignment():
    """The pad variants (operands copied into the workspace with 16-byte rows,
    every row's bytes shifted into place; with K a whole number of K steps an
    aligned operand is read in place) on operands at every element
    misalignment of base and row stride, in every layout, K splits where the
    tile splits: the fp64 oracle, and small integers exactly."""
    pads = [v for v in _lib.variants() if v["name"].endswith("_pad")]
    assert len(pads) == 5
    # K a whole number of K steps (64 and 32 divide 512 and 1024): operands
    # whose rows are already whole 16-byte groups are read in place
    shapes = [(67, 1001, 93), (130, 515, 264), (5, 77, 9), (300, 200, 131), (130, 512, 261), (67, 1024, 96)]
    for i, (m, k, n) in enumerate(shapes):
        a, b = O.normal((m, k), 1400 + 2 * i), O.normal((k, n), 1401 + 2 * i)
        ai, bi = O.small_ints((m, k), 1420 + 2 * i, -3, 3), O.small_ints((k, n), 1421 + 2 * i, -3, 3)
        want = (ai.astype(np.int64) @ bi.astype(np.int64)).astype(np.float32)
        for v in pads:
            bf16 = v["dtype"] == _lib.BF16
            if bf16:
                a16, b16 = O.bf16_round(a), O.bf16_round(b)
                x1, x2, ref, tol = dev_bf16(a16), dev_bf16(b16), O.matmul_bf16_f64(a16, b16), 1e-5
                y1, y2 = dev(ai, torch.bfloat16), dev(bi, torch.bfloat16)
            else:
                x1, x2, ref, tol = dev(a), dev(b), O.matmul_f64(a, b), O.TOL_F32
                y1, y2 = dev(ai), dev(bi)
            splits = [1, 3] if ext.tile_can_split(v) and i == 0 else [1]
            for layout in [0] + LAYOUTS:
                c1, c2 = bool(layout & _lib.X1_COL_MAJOR), bool(layout & _lib.X2_COL_MAJOR)
                for off, extra in ((1, 3), (3, 0), (0, 5), (2, 1)):
                    for s in splits:
                        say(f"{v['name']} split {s} layout {layout} offset {off} extra {extra} shape {(m, k, n)}")
                        got = run(_view_at(x1, c1, off, extra), _view_at(x2, c2, off + 1, extra), (v["name"], s))
                        assert O.rel_l2(got, ref) <= tol, (v["name"], s, layout, off, extra, (m, k, n))
                        got = run(_view_at(y1, c1, off, extra), _view_at(y2, c2, off + 1, extra), (v["name"], s))
                        np.testing.assert_array_equal(got, want)


def test_row_dot_any_alignment():
    """The row-dot kernel (x @ W.T, M <= 4) at every element misalignment of
    K, of both row strides and of both bases: its own kernel runs (no
    scratch) and matches the fp64 oracle, and small integers exactly.  Past
    K a row's last 16-byte chunk holds the row stride's padding, NaN here,
    which must not leak in."""
    rows = [v for v in _lib.variants() if ext.rows_variant(v) and not v["name"].endswith(("_c128", "_c256"))]
    assert len(rows) == 8
    shapes = [(1, 1001, 37), (4, 517, 300), (3, 4099, 64), (1, 3, 9), (2, 2053, 129)]
    for i, (m, k, n) in enumerate(shapes):
        a, b = O.normal((m, k), 1500 + 2 * i), O.normal((k, n), 1501 + 2 * i)
        ai, bi = O.small_ints((m, k), 1520 + 2 * i, -3, 3), O.small_ints((k, n), 1521 + 2 * i, -3, 3)
        want = (ai.astype(np.int64) @ bi.astype(np.int64)).astype(np.float32)
        for v in rows:
            if m > v["max_m"]:
                continue
            bf16 = v["dtype"] == _lib.BF16
            if bf16:
                a16, b16 = O.bf16_round(a), O.bf16_round(b)
                x1, x2, ref, tol = dev_bf16(a16), dev_bf16(b16), O.matmul_bf16_f64(a16, b16), 1e-5
                y1, y2 = dev(ai, torch.bfloat16), dev(bi, torch.bfloat16)
            else:
                x1, x2, ref, tol = dev(a), dev(b), O.matmul_f64(a, b), O.TOL_F32
                y1, y2 = dev(ai), dev(bi)
            for off, extra in ((0, 0), (1, 3), (3, 1), (5, 2)):
                say(f"{v['name']} offset {off} extra {extra} shape {(m, k, n)}")
                views = []
                for p1, p2 in ((x1, x2), (y1, y2)):
                    v1 = _view_at(p1, False, off, extra)
                    v2 = _view_at(p2, True, off + 2, extra)
                    # the padding between rows of x1 and of W (and past the last) is NaN
                    if extra:
                        v1.as_strided((m, extra), (k + extra, 1), v1.storage_offset() + k).fill_(float("nan"))
                        v2.as_strided((n, extra), (k + extra, 1), v2.storage_offset() + k).fill_(float("nan"))
                    views.append((v1, v2))
                wv = views[0][1]
                assert ext.layout_of(views[0][0], wv) == _lib.X2_COL_MAJOR
                got = run(*views[0], (v["name"], 1))
                assert O.rel_l2(got, ref) <= tol, (v["name"], off, extra, (m, k, n))
                np.testing.assert_array_equal(run(*views[1], (v["name"], 1)), want)


def test_layouts_padded_strides_and_splits():
    """Column strides above the row count, and K splits of the tile GEMMs,
    in every layout."""
    cases = [((33, 1000, 65), "f32"), ((520, 2048, 300), "f32"), ((16, 4096, 512), "f32"),
             ((520, 2048, 304), "bf16"), ((16, 4096, 512), "bf16")]
    for (m, k, n), dt in cases:
        a, b = O.normal((m, k), 700), O.normal((k, n), 701)
        if dt == "bf16":
            a, b = O.bf16_round(a), O.bf16_round(b)
            x1, x2, ref, tol = dev_bf16(a), dev_bf16(b), O.matmul_bf16_f64(a, b), 1e-5
        else:
            x1, x2, ref, tol = dev(a), dev(b), O.matmul_f64(a, b), O.TOL_F32
        for layout in LAYOUTS:
            for cfg in ext.hip_configs(m, k, n, dt):
                for pad in (0, 8, 3):
                    say(f"padded {(m, k, n)} {dt} layout {layout} pad {pad} {cfg}")
                    got = run_layout(x1, x2, layout, cfg, pad)
                    assert O.rel_l2(got, ref) <= tol, ((m, k, n), dt, layout, pad, cfg)


def test_golden_integer_products_layouts():
    """Exact small-integer products are exact in every layout and variant."""
    g = np.load(GOLDEN)
    for i, (m, k, n) in enumerate(g["shapes"]):
        m, k, n = int(m), int(k), int(n)
        a = g[f"x1_{i}"].astype(np.float32)
        b = g[f"x2_{i}"].astype(np.float32)
        want = g[f"out_{i}"].astype(np.float32)
        a16, b16 = O.bf16_round(a), O.bf16_round(b)
        for layout in LAYOUTS:
            for cfg in ext.hip_configs(m, k, n, "f32"):
                say(f"golden {i} {(m, k, n)} f32 layout {layout} {cfg}")
                np.testing.assert_array_equal(run_layout(dev(a), dev(b), layout, cfg), want)
            for cfg in ext.hip_configs(m, k, n, "bf16"):
                say(f"golden {i} {(m, k, n)} bf16 layout {layout} {cfg}")
                np.testing.assert_array_equal(run_layout(dev_bf16(a16), dev_bf16(b16), layout, cfg), want)


@pytest.mark.parametrize("m", [1, 4, 16])
def test_gemv_weight_transposed(m):
    """x @ W.T with W [N, K] row-major (a linear layer's weight), at the
    config-1 size, with the tuned pick: the weight is read in place."""
    k = n = 4096
    x, w = O.normal((m, k), 800 + m), O.normal((n, k), 801 + m)
    ref = O.matmul_f64(x, np.ascontiguousarray(w.T))
    dx, dw = dev(x), dev(w)
    assert ext.layout_of(dx, dw.t()) == _lib.X2_COL_MAJOR
    got = run(dx, dw.t())
    assert O.rel_l2(got, ref) <= O.TOL_F32
    x16, w16 = O.bf16_round(x), O.bf16_round(w)
    got16 = run(dev_bf16(x16), dev_bf16(w16).t())
    assert O.rel_l2(got16, O.matmul_bf16_f64(x16, np.ascontiguousarray(w16.T))) <= 1e-5
    say(f"gemv x @ W.T m={m} ok")


def test_gemv_rows_kernel():
    """The kernels for x @ W.T (x2 column-major: W [N, K] row-major, no K
    split): the row-dot kernel (one wave per one or two rows of W over all of
    K, M <= 4) and the row-tile kernel (16 rows of W per workgroup, 8 or 16
    waves, MFMAs fed through LDS, M <= 16).  Many M up to the variant's bound, N ragged
    against the rows per workgroup, K a multiple of the 16-byte group but not
    of the wave chunk, row strides of W and x1 past K whose padding holds NaN
    (both are masked at K, so it must not leak), against the fp64 oracle;
    small integers bit-exact; other layouts run the streaming kernel."""
    rows = [v for v in _lib.variants() if ext.rows_variant(v)]
    assert len(rows) == 14
    for v in rows:
        bf = v["dtype"] == _lib.BF16
        ms = range(1, v["max_m"] + 1) if v["max_m"] <= 4 else (1, 2, 5, 8, 13, 16)
        for m in ms:
            for i, (k, n) in enumerate([(8, 1), (1000, 37), (4096, 513), (2056, 130)]):
                a, w = O.normal((m, k), 60 * m + i), O.normal((n, k), 60 * m + i + 30)
                if bf:
                    a, w = O.bf16_round(a), O.bf16_round(w)
                ref = (O.matmul_bf16_f64 if bf else O.matmul_f64)(a, np.ascontiguousarray(w.T))
                if bf:
                    wp = np.full((n, k + 24), 0x7FC0, dtype=np.uint16)  # bf16 NaN
                    wp[:, :k] = w
                    ap = np.full((m, k + 8), 0x7FC0, dtype=np.uint16)
                    ap[:, :k] = a
                    dw, dx = dev_bf16(wp)[:, :k], dev_bf16(ap)[:, :k]
                else:
                    wp = np.full((n, k + 24), np.nan, dtype=np.float32)
                    wp[:, :k] = w
                    ap = np.full((m, k + 8), np.nan, dtype=np.float32)
                    ap[:, :k] = a
                    dw, dx = dev(wp)[:, :k], dev(ap)[:, :k]
                assert dw.stride() == (k + 24, 1) and (m == 1 or dx.stride() == (k + 8, 1))
                say(f"{v['name']} m={m} k={k} n={n}")
                got = run(dx, dw.t(), (v["name"], 1))
                assert O.rel_l2(got, ref) <= (1e-5 if bf else O.TOL_F32), (v["name"], m, k, n)
                assert np.isfinite(got).all()
    rng = np.random.default_rng(33)
    for m in (1, 3, 4, 9, 16):
        a = rng.integers(-3, 4, (m, 3000)).astype(np.float32)
        w = rng.integers(-3, 4, (260, 3000)).astype(np.float32)
        want = (a.astype(np.int64) @ w.T.astype(np.int64)).astype(np.float32)
        for v in rows:
            if m > v["max_m"]:
                continue
            conv = (lambda x: dev(x).to(torch.bfloat16)) if v["dtype"] == _lib.BF16 else dev
            np.testing.assert_array_equal(run(conv(a), conv(w).t(), (v["name"], 1)), want)
            for layout in (0, _lib.X1_COL_MAJOR, _lib.X1_COL_MAJOR | _lib.X2_COL_MAJOR):
                got = run_layout(conv(a), conv(np.ascontiguousarray(w.T)), layout, (v["name"], 2))
                np.testing.assert_array_equal(got, want)


def test_gemv_rows_unaligned_base_and_scratch():
    """x @ W.T through base pointers that are only 4-byte (fp32) or 2- and
    8-byte (bf16) aligned, with K and the strides aligned: every row-dot and
    row-tile variant, AUTO and the tuned pick then run the streaming
    fallback, at split 1 and at the automatic split, against the fp64
    oracle.  With aligned operands the row kernels' own path needs no
    scratch: the C ABI accepts the call with no workspace or counters."""
    L = _lib.lib()
    k, n = 4096, 520
    for bf, offsets in ((False, (1,)), (True, (1, 4))):
        dt = torch.bfloat16 if bf else torch.float32
        rows = [v for v in _lib.variants() if ext.rows_variant(v) and v["dtype"] == (_lib.BF16 if bf else _lib.F32)]
        for m in (1, 4, 16):
            a, w = O.normal((m, k), 80 + m), O.normal((n, k), 81 + m)
            if bf:
                a, w = O.bf16_round(a), O.bf16_round(w)
            ref = (O.matmul_bf16_f64 if bf else O.matmul_f64)(a, np.ascontiguousarray(w.T))
            mk = dev_bf16 if bf else dev
            for off in offsets:
                fa = torch.zeros(m * k + off, dtype=dt, device="cuda")
                fa[off:] = mk(a).flatten()
                fw = torch.zeros(n * k + off, dtype=dt, device="cuda")
                fw[off:] = mk(w).flatten()
                x1, x2 = fa[off:].view(m, k), fw[off:].view(n, k).t()
                assert x1.data_ptr() % 16 != 0 and x2.data_ptr() % 16 != 0
                cfgs = [(v["name"], s) for v in rows if m <= v["max_m"] for s in (1, 0)] + [None, "auto"]
                for cfg in cfgs:
                    say(f"unaligned x @ W.T {'bf16' if bf else 'f32'} m={m} offset {off} {cfg}")
                    got = run(x1, x2, _lib.VARIANT_AUTO if cfg == "auto" else cfg)
                    assert O.rel_l2(got, ref) <= (1e-5 if bf else O.TOL_F32), (bf, m, off, cfg)
            # aligned operands: the row kernel itself runs, without scratch
            dx, dw = mk(a), mk(w)
            out = torch.empty((m, n), dtype=torch.float32, device="cuda")
            for v in rows:
                if m > v["max_m"]:
                    continue
                rc = L.tilec_matmul(dx.data_ptr(), dw.data_ptr(), out.data_ptr(), m, n, k, k, k, n,
                                    _lib.X2_COL_MAJOR, _lib.BF16 if bf else _lib.F32, v["id"], 0,
                                    None, 0, None, 0, torch.cuda.current_stream().cuda_stream)
                assert rc == _lib.OK, (v["name"], _lib.last_error())
                torch.cuda.synchronize()
                assert O.rel_l2(out.cpu().numpy(), ref) <= (1e-5 if bf else O.TOL_F32), v["name"]


def test_non_default_stream_and_ordering():
    a, b = O.normal((16, 2048), 16), O.normal((2048, 1024), 17)
    ref = O.matmul_f64(a, b)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        da, db = dev(a), dev(b)
        out = ext.matrix_mul(da, db)
        out2 = ext.matrix_mul(da, db)
    s.synchronize()
    assert O.rel_l2(out.cpu().numpy(), ref) <= O.TOL_F32
    assert torch.equal(out, out2)
    say("stream ok")


def test_workspace_counters_return_to_zero():
    a, b = O.normal((16, 4096), 18), O.normal((4096, 4096), 19)
    da, db = dev(a), dev(b)
    ref = O.matmul_f64(a, b)
    L = _lib.lib()
    for cfg in [("skinny_f32_w8_b1", 8), ("skinny_f32_w4_b2", 16), ("skinny_f32_w16_b1", 4), ("skinny_f32_w8_b2", 64)]:
        for _ in range(3):
            got = run(da, db, cfg)
            assert O.rel_l2(got, ref) <= O.TOL_F32, cfg
        v = _lib.variant_id(cfg[0])
        cb = L.tilec_matmul_counter_bytes(16, 4096, 4096, 0, v, cfg[1])
        stream = torch.cuda.current_stream().cuda_stream
        cnt = ext._COUNTERS[(da.device.index, stream)]
        assert cb > 0 and torch.count_nonzero(cnt).item() == 0, cfg
    # calls of different shapes share the buffers: layouts must not collide
    for m, k, n in [(1, 4096, 130), (16, 4096, 4096), (3, 4000, 65), (16, 65536, 64), (2, 4096, 130)]:
        a1, b1 = O.normal((m, k), m + k), O.normal((k, n), n)
        for cfg in ext.hip_configs(m, k, n, "f32"):
            if cfg[0].startswith("skinny"):
                assert O.rel_l2(run(dev(a1), dev(b1), cfg), O.matmul_f64(a1, b1)) <= O.TOL_F32, (cfg, (m, k, n))
    say("workspace counters ok")


def test_bf16_skinny_and_tiled_api():
    a16 = O.bf16_round(O.normal((4, 1000), 20))
    b16 = O.bf16_round(O.normal((1000, 300), 21))
    got = run(dev_bf16(a16), dev_bf16(b16))
    assert O.rel_l2(got, O.matmul_bf16_f64(a16, b16)) <= 1e-5
    a, b = O.normal((100, 70), 22), O.normal((70, 90), 23)
    got = ext._matrix_mul_tiled(dev(a), dev(b))  # the reference default BM=BN=64, BK=16
    torch.cuda.synchronize()
    assert O.rel_l2(got.cpu().numpy(), O.matmul_f64(a, b)) <= O.TOL_F32
    with pytest.raises(ValueError):
        ext._matrix_mul_tiled(dev(a), dev(b), BM=48, BN=48, BK=16)
    say("bf16 skinny / tiled api ok")


def test_graph_capture_replays():
    # Captured skinny calls (split K, reused workspace) replayed several times,
    # with eager work between replays; every replay must match eager.
    a, b = O.normal((16, 4096), 24), O.normal((4096, 2048), 25)
    da, db = dev(a), dev(b)
    eager = ext.matrix_mul(da, db, ("skinny_f32_w8_b1", 8))
    eager2 = ext.matrix_mul(da, db)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        # the workspace for this stream is allocated (and zeroed) before capture
        ext.matrix_mul(da, db, ("skinny_f32_w8_b1", 8))
        ext.matrix_mul(da, db)
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            out = ext.matrix_mul(da, db, ("skinny_f32_w8_b1", 8))
            out2 = ext.matrix_mul(da, db)
    torch.cuda.current_stream().wait_stream(s)
    for i in range(4):
        out.zero_()
        g.replay()
        junk = ext.matrix_mul(da[:4], db)  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(out, eager), i
        assert torch.equal(out2, eager2), i
        del junk
    say("graph replay ok")


def test_graph_capture_row_dot_and_bf16_rings():
    """The kernels without a K split in a captured graph: the row-dot and
    row-tile kernels for x @ W.T and the bf16 LDS-DMA GEMM with a ring of four
    stage buffers (fence-free step barrier), replayed several times with eager
    work between replays; every replay must match the eager result bit for
    bit."""
    x, w = O.normal((1, 2048), 70), O.normal((1536, 2048), 71)
    x12 = O.normal((12, 2048), 74)
    a16, b16 = O.bf16_round(O.normal((512, 1024), 72)), O.bf16_round(O.normal((1024, 512), 73))
    dx, dw, dx12 = dev(x), dev(w), dev(x12)
    da, db = dev_bf16(a16), dev_bf16(b16)
    cfg_rows, cfg_ring = ("skinny_f32_t1_r1_w8_u2", 1), ("gemm_bf16_256x256x32_r4w8", 1)
    cfg_tile = ("skinny_f32_t16_r16_w8_c128", 1)
    eager = ext.matrix_mul(dx, dw.t(), cfg_rows)
    eager2 = ext.matrix_mul(da, db, cfg_ring)
    eager3 = ext.matrix_mul(dx12, dw.t(), cfg_tile)
    torch.cuda.synchronize()
    assert O.rel_l2(eager.cpu().numpy(), O.matmul_f64(x, np.ascontiguousarray(w.T))) <= O.TOL_F32
    assert O.rel_l2(eager2.cpu().numpy(), O.matmul_bf16_f64(a16, b16)) <= 1e-5
    assert O.rel_l2(eager3.cpu().numpy(), O.matmul_f64(x12, np.ascontiguousarray(w.T))) <= O.TOL_F32
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ext.matrix_mul(dx, dw.t(), cfg_rows)
        ext.matrix_mul(da, db, cfg_ring)
        ext.matrix_mul(dx12, dw.t(), cfg_tile)
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            out = ext.matrix_mul(dx, dw.t(), cfg_rows)
            out2 = ext.matrix_mul(da, db, cfg_ring)
            out3 = ext.matrix_mul(dx12, dw.t(), cfg_tile)
    torch.cuda.current_stream().wait_stream(s)
    for i in range(4):
        out.zero_()
        out2.zero_()
        out3.zero_()
        g.replay()
        junk = ext.matrix_mul(da[:64], db)  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(out, eager), i
        assert torch.equal(out2, eager2), i
        assert torch.equal(out3, eager3), i
        del junk
    say("graph replay (row-dot, row-tile, bf16 ring of 4) ok")
