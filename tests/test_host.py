"""Host logic and the C ABI, without a GPU.

Covers what the reference's host code decides before it launches
(tilec/ext.py:54-63, tilec/jit.py:34-39): shape and dtype errors, the legacy
config-space helpers, the MI355X config space and tuner plumbing, and that
libtilec_hip.so loads and exports every symbol include/tilec.h declares, with
argument validation that fails before any kernel would be enqueued.
"""

import ctypes
import math
import os
import re

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tilec import _lib, ext, tune
import tilec

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


# ---------------------------------------------------------------------------
# The drop-in surface
# ---------------------------------------------------------------------------

def test_reference_names_are_available():
    assert tilec.ext.matrix_mul is ext.matrix_mul
    assert tilec.ext._matrix_mul_tiled is ext._matrix_mul_tiled
    for name in ("plan", "mm_configs", "cdiv", "MAX_BLOCK", "SPLITS", "JOINS", "BLOCKS", "_blocks"):
        assert hasattr(tilec.ext, name)
    assert tilec.language.cdiv(5000, 4096) == 2
    assert callable(tilec.tune.pick)


def test_legacy_helpers_match_oracle():
    for n in list(range(1, 300)) + [1000, 4095, 4096, 4097, 5000, 16384, 65537]:
        assert ext.plan(n) == O.plan(n)
        assert ext._blocks(n) == O.blocks(n)
    for M1, N, M2 in [(129, 256, 32), (1000, 4096, 100), (8, 48, 3), (8081, 16384, 3857)]:
        assert ext.mm_configs(M1, N, M2) == O.mm_configs(M1, N, M2)


def test_shape_mismatch_raises_value_error():
    with pytest.raises(ValueError, match=r"matrix_mul: shapes \(3, 4\) and \(5, 6\) don't match"):
        ext.matrix_mul(torch.zeros(3, 4), torch.zeros(5, 6))


def test_non_2d_raises_value_error():
    with pytest.raises(ValueError):
        ext.matrix_mul(torch.zeros(3), torch.zeros(3, 4))
    with pytest.raises(ValueError):
        ext.matrix_mul(torch.zeros(2, 3, 4), torch.zeros(4, 4))


@pytest.mark.parametrize("dt", [torch.float64, torch.float16, torch.int32])
def test_unsupported_dtype_raises_type_error(dt):
    with pytest.raises(TypeError):
        ext.matrix_mul(torch.zeros(3, 4, dtype=dt), torch.zeros(4, 5, dtype=dt))


def test_mixed_dtype_raises_type_error():
    with pytest.raises(TypeError):
        ext.matrix_mul(torch.zeros(3, 4), torch.zeros(4, 5, dtype=torch.bfloat16))


def test_cpu_tensors_raise_not_fallback():
    # No CPU fallback: host tensors are rejected, never computed on the CPU.
    with pytest.raises(TypeError, match="ROCm GPU"):
        ext.matrix_mul(torch.zeros(3, 4), torch.zeros(4, 5))


# ---------------------------------------------------------------------------
# Config space and tuner
# ---------------------------------------------------------------------------

def test_hip_configs_rules():
    names = {v["name"]: v for v in _lib.variants()}
    # the direct family past the small-output rule: up to four 64x64 tiles per CU, fp32 only
    assert ext.direct_regime(1024, 1024, "f32") and ext.direct_regime(2048, 2048, "f32")
    assert not ext.direct_regime(2049, 2048, "f32") and not ext.direct_regime(1024, 1024, "bf16")
    assert any(c[0].startswith("direct_") for c in ext.hip_configs(1024, 1024, 1024, "f32"))
    assert not any(c[0].startswith("direct_") for c in ext.hip_configs(4096, 4096, 4096, "f32"))
    # 2048 x 2048 x 16384: 1024 64x64 tiles (2048 of 32x64): at 256 CUs the 8-per-CU cap leaves the
    # direct kernel a K split of 2 at most, where a split of 64 would launch 131 072 workgroups
    big = [c for c in ext.hip_configs(2048, 16384, 2048, "f32") if c[0].startswith("direct_")]
    if ext.device_cus() == 256:
        assert big and max(ext._direct_splits(16384, s) for _, s in big) == 2
    # no direct config past the library's 2 GiB partials limit is offered
    names = {v["name"]: v for v in _lib.variants()}
    for M, K, N in [(2048, 4096, 2048), (1024, 1024, 1024), (513, 3001, 127), (1, 65536, 4096)]:
        for name, s in ext.hip_configs(M, K, N, "f32"):
            if name.startswith("direct_"):
                assert ext.direct_workspace_bytes(names[name], M, N, ext._direct_splits(K, s)) < 1 << 31
    for M, K, N, dt in [(1, 4096, 4096, "f32"), (16, 4096, 4096, "f32"), (17, 4096, 4096, "f32"),
                        (4096, 4096, 4096, "f32"), (8192, 8192, 8192, "bf16"), (3, 100, 7, "f32"),
                        (1, 4096, 4096, "bf16"), (1024, 1024, 1024, "f32"), (520, 8192, 1648, "bf16")]:
        cfgs = ext.hip_configs(M, K, N, dt)
        assert cfgs and len(cfgs) == len(set(cfgs))
        for name, s in cfgs:
            v = names[name]
            assert v["dtype"] == (_lib.F32 if dt == "f32" else _lib.BF16)
            if v["family"] == _lib.FAMILY_SKINNY:
                assert v["max_m"] == 0 or M <= v["max_m"]
                eff = ext._skinny_splits(K, s, v["bk"])
                assert eff == 1 or K // eff >= 16 * v["waves"]
            elif v["family"] == _lib.FAMILY_DIRECT:
                eff = ext._direct_splits(K, s)
                assert dt == "f32" and v["bm"] < 2 * max(M, 16)
                assert ext.skinny_regime(M, N, dt) or ext.direct_regime(M, N, dt)
                assert eff == 1 or ext.cdiv(K, eff) >= 16 * v["waves"]
                # a K split keeps the grid within 8 workgroups per CU
                tiles = ext.cdiv(M, v["bm"]) * ext.cdiv(N, v["bn"])
                assert eff == 1 or tiles * eff <= 8 * ext.device_cus()
            else:
                tiles = ext.cdiv(M, v["bm"]) * ext.cdiv(N, v["bn"])
                eff = ext._gemm_splits(K, s, v["bk"])
                assert eff == 1 or (ext.tile_can_split(v) and tiles < ext.device_cus()
                                    and ext.cdiv(K, v["bk"]) >= 4 * eff)
        has_skinny = any(names[n]["family"] == _lib.FAMILY_SKINNY for n, _ in cfgs)
        assert has_skinny == ext.skinny_regime(M, N, dt)
    # Few tiles: the tile GEMMs that can split are offered split configs.
    assert ("gemm_bf16_128x128x64_r4", 8) in ext.hip_configs(1, 4096, 4096, "bf16")
    assert ("gemm_f32_128x64x16_w2x2", 4) in ext.hip_configs(1024, 1024, 1024, "f32")
    assert all(s == 1 for _, s in ext.hip_configs(8192, 8192, 8192, "bf16"))


def test_direct_split_geometry_matches_the_library():
    """Direct kernel: K chunks of a multiple of 16 rows, none empty; scratch =
    splits * tiles * (16-byte values per thread after the waves meet) *
    threads, counters = one 256-byte line per tile, none when unsplit."""
    L = _lib.lib()
    for v in [v for v in _lib.variants() if v["family"] == _lib.FAMILY_DIRECT]:
        items = 4 * (v["bm"] // 16) * (v["bn"] // 64)
        nv = ext.cdiv(items, v["waves"])
        for M, N, K in [(1, 4096, 4096), (513, 127, 3001), (127, 513, 1000), (16, 64, 16), (5, 7, 1)]:
            tiles = ext.cdiv(M, v["bm"]) * ext.cdiv(N, v["bn"])
            for s in (1, 2, 3, 8, 16, 64, 5000):
                eff = ext._direct_splits(K, s)
                kc = ext.cdiv(ext.cdiv(K, s), 16) * 16
                assert eff == ext.cdiv(K, kc) and (eff - 1) * kc < K
                ws = L.tilec_matmul_workspace_bytes(M, N, K, _lib.F32, v["id"], s)
                cnt = L.tilec_matmul_counter_bytes(M, N, K, _lib.F32, v["id"], s)
                assert ws == (ext.direct_workspace_bytes(v, M, N, eff) if eff > 1 else 0)
                if eff == 1:
                    assert ws == 0 and cnt == 0, (v["name"], M, N, K, s)
                else:
                    assert ws == eff * tiles * nv * v["waves"] * 64 * 16, (v["name"], M, N, K, s)
                    assert cnt == tiles * 64 * 4, (v["name"], M, N, K, s)


def test_gemm_split_geometry_matches_the_library():
    """Workspace the C ABI asks for a split tile GEMM = splits * tiles *
    BM * BN floats; counters = one 256-byte line per tile; unsplittable
    tiles are refused."""
    L = _lib.lib()
    v = _lib.variants()[_lib.variant_id("gemm_f32_64x64x16_w2x2")]
    for M, N, K, s in [(1024, 1024, 1024, 4), (100, 70, 1000, 3), (64, 64, 4096, 16), (64, 64, 40, 8)]:
        eff = ext._gemm_splits(K, s, v["bk"])
        tiles = ext.cdiv(M, 64) * ext.cdiv(N, 64)
        ws = L.tilec_matmul_workspace_bytes(M, N, K, _lib.F32, v["id"], s)
        cnt = L.tilec_matmul_counter_bytes(M, N, K, _lib.F32, v["id"], s)
        assert ws == (eff * tiles * 64 * 64 * 4 if eff > 1 else 0), (M, N, K, s)
        assert cnt == (tiles * 256 if eff > 1 else 0)
    big = _lib.variant_id("gemm_bf16_256x256x64_r2")
    assert _call(M=256, N=256, K=4096, dtype=_lib.BF16, variant=big, split=4) == _lib.ERR_UNSUPPORTED
    assert L.tilec_auto_split_k(256, 256, 4096, _lib.BF16, big) == 1
    small = _lib.variant_id("gemm_bf16_128x128x64_r4")
    assert L.tilec_auto_split_k(1, 4096, 4096, _lib.BF16, small) > 1


def test_row_dot_configs_only_where_the_kernel_runs():
    """The x @ W.T variants (row-dot, M <= 4; row-tile, M <= 16) are offered
    unsplit, for x2 column-major, the row-tile kernel only for K a multiple
    of the 16-byte group (the row-dot kernel takes any K); elsewhere they
    would run the streaming kernel unsplit."""
    rows = lambda cfgs: [c for c in cfgs if ext.rows_variant(_lib.variants()[_lib.variant_id(c[0])])]
    f32 = rows(ext.hip_configs(1, 4096, 4096, "f32", _lib.X2_COL_MAJOR))
    assert f32 and all(s == 1 for _, s in f32)
    assert rows(ext.hip_configs(4, 4096, 4096, "bf16", _lib.X2_COL_MAJOR))
    assert not rows(ext.hip_configs(1, 4096, 4096, "f32", 0))
    assert not rows(ext.hip_configs(1, 4096, 4096, "f32", _lib.X1_COL_MAJOR | _lib.X2_COL_MAJOR))
    odd = rows(ext.hip_configs(1, 4094, 4096, "f32", _lib.X2_COL_MAJOR))
    assert odd and not any(c.endswith(("_c128", "_c256")) for c, _ in odd)
    assert rows(ext.hip_configs(4, 4092, 4096, "bf16", _lib.X2_COL_MAJOR))
    assert not rows(ext.hip_configs(5, 4092, 4096, "bf16", _lib.X2_COL_MAJOR))  # row-tile only, K % 8
    m5 = rows(ext.hip_configs(5, 4096, 4096, "f32", _lib.X2_COL_MAJOR))
    assert m5 and all(c.endswith(("_c128", "_c256")) for c, _ in m5)  # only the row-tile kernel above M = 4
    assert rows(ext.hip_configs(16, 4096, 4096, "bf16", _lib.X2_COL_MAJOR))
    assert not rows(ext.hip_configs(17, 4096, 4096, "f32", _lib.X2_COL_MAJOR))  # M above every bound


def test_tune_features_and_shapes():
    f = tune.features(16, 4096, 4096, 256, "f32", "skinny_f32_w8_b1", 8)
    assert len(f) == 34 and all(math.isfinite(x) for x in f) and f[16:18] == [0.0, 0.0] and f[28:30] == [1.0, 1.0]
    # alignment of each operand's contiguous extent: x1 row-major runs along K, x2 column-major along K
    assert tune.features(5, 4097, 4096, 256, "f32", "skinny_f32_w8_b1", 1)[28:30] == [0.0, 1.0]
    assert tune.features(5, 4096, 4100, 256, "bf16", "skinny_bf16_w8_b1", 1)[28:30] == [1.0, 0.0]
    assert tune.features(6, 4096, 4100, 256, "bf16", "skinny_bf16_w8_b1", 1, layout=3)[28:30] == [0.0, 1.0]
    # variant properties beyond the descriptor: 16x16 MFMA blocks, transposing and padding prepasses
    assert f[30:33] == [0.0, 0.0, 0.0]
    assert tune.features(4096, 4096, 4096, 256, "bf16", "gemm_bf16_256x256x64_r2_m16", 1)[30:33] == [1.0, 0.0, 0.0]
    assert tune.features(4096, 4096, 4096, 256, "bf16", "gemm_bf16_256x256x64_r2_kc", 1)[30:33] == [0.0, 1.0, 0.0]
    assert tune.features(1000, 4097, 3001, 256, "f32", "gemm_f32_64x64x32_w2x2_pad", 1)[30:33] == [0.0, 0.0, 1.0]
    # whether the config runs its tile's slower fallback for these operands
    fb = lambda *a: tune.features(*a)[33]
    assert fb(1000, 4097, 3001, 256, "f32", "gemm_f32_128x128x32_w2x4_lds", 1, 0) == 1.0
    assert fb(1000, 4097, 3001, 256, "f32", "gemm_f32_128x128x32_w2x4_pad", 1, 0) == 0.0
    assert fb(1000, 4097, 3001, 256, "f32", "gemm_f32_128x128x32_w2x4", 1, 0) == 0.0  # register-staged: its own kernel
    assert fb(1024, 4096, 1020, 256, "bf16", "gemm_bf16_128x128x64_r4_m16", 1, 0) == 1.0  # N % 8
    assert fb(1024, 4096, 1020, 256, "bf16", "gemm_bf16_128x128x64_r4_m16", 1, 1) == 1.0
    assert fb(1020, 4096, 1024, 256, "bf16", "gemm_bf16_128x128x64_r4_m16", 1, 0) == 0.0  # M is no row extent here
    assert fb(1020, 4096, 1024, 256, "bf16", "gemm_bf16_128x128x64_r4_m16", 1, 1) == 1.0  # ... but is here
    # kc transposes only when M, N and K are multiples of 8, else runs the plain tile
    assert fb(1024, 4096, 1020, 256, "bf16", "gemm_bf16_128x128x64_r4_kc", 1, 0) == 1.0
    assert fb(1020, 4096, 1024, 256, "bf16", "gemm_bf16_128x128x64_r4_kc", 1, 0) == 0.0
    assert fb(1024, 4096, 1024, 256, "bf16", "gemm_bf16_128x128x64_r4_kc", 1, 3) == 0.0
    assert fb(1020, 4096, 1024, 256, "bf16", "gemm_bf16_64x64x64_w2x2", 1, 1) == 0.0
    assert fb(16, 4097, 4096, 256, "f32", "skinny_f32_w8_b1", 1, 0) == 0.0
    # the row-dot kernel's shifted form for K past whole 16-byte groups; the row-tile kernel never runs there
    assert fb(4, 5429, 11110, 256, "bf16", "skinny_bf16_t4_r2_w4", 1, 2) == 1.0
    assert fb(4, 5432, 11110, 256, "bf16", "skinny_bf16_t4_r2_w4", 1, 2) == 0.0
    assert fb(4, 5432, 11110, 256, "bf16", "skinny_bf16_t16_r16_w8_c128", 1, 2) == 0.0
    # copies before the GEMM enter the analytic time: a launch each and their bytes
    assert tune.prepass(1000, 4097, 3001, "f32", "gemm_f32_64x64x32_w2x2_pad") == (2, 8 * (1000 * 4097 + 4097 * 3001))
    assert tune.prepass(1024, 512, 640, "bf16", "gemm_bf16_128x128x64_r4_kc", 1) == (2, 4 * (1024 * 512 + 512 * 640))
    assert tune.prepass(1024, 512, 640, "bf16", "gemm_bf16_128x128x64_r4_kc", 2) == (0, 0)
    assert tune.prepass(1024, 512, 640, "bf16", "gemm_bf16_128x128x64_r4_kc", 0) == (1, 4 * 512 * 640)
    assert tune.prepass(1020, 512, 640, "bf16", "gemm_bf16_128x128x64_r4_kc", 0) == (0, 0)
    assert tune.prepass(1024, 512, 640, "bf16", "gemm_bf16_128x128x64_r4", 1) == (0, 0)
    m16, plain = (tune.features(4096, 4096, 4096, 256, "bf16", k, 1) for k in
                  ("gemm_bf16_256x256x64_r2_m16", "gemm_bf16_256x256x64_r2"))
    assert m16[:30] == plain[:30] and m16 != plain
    assert tune.features(16, 4096, 4096, 256, "f32", "skinny_f32_w8_b1", 8, layout=3)[16:18] == [1.0, 1.0]
    assert tune.features(1, 4096, 4096, 256, "f32", "skinny_f32_v1_w4_b2", 4)[18] == 1.0
    s = tune.shapes(120, seed=0, n_layout=40, n_rows=10, n_tile=6, n_medium=0, n_narrow=0, n_bf16=0)
    assert s == tune.shapes(120, seed=0, n_layout=40, n_rows=10, n_tile=6, n_medium=0, n_narrow=0, n_bf16=0)
    rm = [x for x in s if x[4] == 0]
    lay = [x for x in s if x[4] != 0]
    assert len(rm) == 120 + len(tune.CONFIG_SHAPES) and len(lay) == 40 + len(tune.LAYOUT_CONFIG_SHAPES) + 10 + 6
    # the x @ W.T streams (M <= 4 and 5 <= M <= 16, x2 column-major) add to, and do not change, the others
    no_rows = tune.shapes(120, seed=0, n_layout=40, n_rows=0, n_tile=6, n_medium=0, n_narrow=0, n_bf16=0)
    assert set(no_rows) <= set(s) and all(x[0] <= 4 and x[4] == 2 for x in set(s) - set(no_rows))
    no_tile = tune.shapes(120, seed=0, n_layout=40, n_rows=10, n_tile=0, n_medium=0, n_narrow=0, n_bf16=0)
    assert set(no_tile) <= set(s) and all(5 <= x[0] <= 16 and x[4] == 2 for x in set(s) - set(no_tile))
    assert {x + (0,) for x in tune.CONFIG_SHAPES} <= set(rm) and set(tune.LAYOUT_CONFIG_SHAPES) <= set(lay)
    assert {x[4] for x in lay} == {1, 2, 3}
    assert any(m <= 16 for m, *_ in s) and any(d == "bf16" for _, _, _, d, _ in s)
    # the row-major draws do not depend on the layout stream
    assert rm == [x for x in tune.shapes(120, seed=0, n_layout=5, n_medium=0, n_narrow=0, n_bf16=0) if x[4] == 0]
    # the medium and narrow streams add row-major shapes in their ranges, and
    # never a shape the tuner must leave unseen
    full = tune.shapes(120, seed=0, n_layout=40, n_rows=10, n_tile=6, n_bf16=0)
    more = set(full) - set(s)
    assert set(s) <= set(full) and 100 <= len(more) <= 140 and all(x[4] == 0 for x in more)
    for M, K, N, d, _ in more:
        small, large = min(M, N), max(M, N)
        assert (48 <= small <= 600 and 500 <= large <= 6000 and 500 <= K <= 4096) or \
            (48 <= small <= 400 and 500 <= large <= 5000 and 2048 <= K <= 16384), (M, K, N)
    assert {d for *_, d, _ in more} == {"f32", "bf16"}
    # the bf16 stream adds bf16 tile GEMMs in every layout, within its ranges
    with_bf16 = tune.shapes(120, seed=0, n_layout=40, n_rows=10, n_tile=6)
    extra = set(with_bf16) - set(full)
    assert set(full) <= set(with_bf16) and 70 <= len(extra) <= 80 and {x[4] for x in extra} == {0, 1, 2, 3}
    assert all(d == "bf16" and 64 <= M <= 8192 and 256 <= K <= 8192 and 64 <= N <= 8192 for M, K, N, d, _ in extra)
    assert not {u + (0,) for u in tune.UNSEEN_SHAPES} & set(tune.shapes(400))


def test_tune_roofline_known_answers():
    # 4096^3 fp32 on the 256x256 tile: 256 tiles, one round of one workgroup
    # per CU, no padding; the matrix-peak time 2 * 4096^3 / 157.3e12 bounds it
    t_est, t_c, t_m, t_r, pad, tail, fill, kpw, rounds = tune.roofline(
        4096, 4096, 4096, 256, "f32", "gemm_f32_256x256x32_w2x4_lds", 1)
    assert (pad, tail, fill, rounds) == (1.0, 1.0, 1.0, 1.0)
    assert t_c == pytest.approx(2 * 4096 ** 3 / 157.3e12)
    assert t_m == pytest.approx(3 * 4 * 4096 ** 2 / 8e12)
    assert t_r == pytest.approx(4 * 2 * 4096 ** 2 * 16 / 20e12)
    assert t_est == pytest.approx(t_c + 3e-6) and kpw == 4096 / 8
    # 1 x 4096 @ 4096 x 4096 on the streaming kernel, split 8: 64 slabs of 16 x 64
    # (1/16 of each used), 512 workgroups of 8 waves = 2 rounds; HBM-bound
    t_est, t_c, t_m, t_r, pad, tail, fill, kpw, rounds = tune.roofline(
        1, 4096, 4096, 256, "f32", "skinny_f32_w8_b1", 8)
    assert (pad, rounds, fill) == (1 / 16, 2.0, 1.0)
    assert t_m == pytest.approx((4 * (4096 + 4096 ** 2) + 4 * 4096 + 8 * 64 * 16 * 64 * 8) / 8e12)
    assert t_est == pytest.approx(max(t_c, t_m, t_r) + 3e-6 + 1.5e-6)


def test_tune_rotating_operands():
    """Streaming-regime timings cycle x2 over copies that together exceed the
    Infinity Cache (at most 16); tile-GEMM shapes and tiny x2 use x2 alone."""
    import torch
    x2 = torch.ones(1024, 1024)                      # 4 MiB
    ops = tune.operands_for(1, 1024, 1024, x2)
    assert len(ops) == 16 and ops[0] is x2 and all(o.data_ptr() != x2.data_ptr() for o in ops[1:])
    assert all(torch.equal(o, x2) for o in ops)
    big = torch.empty(8192, 8192, dtype=torch.bfloat16)   # 128 MiB: 4 copies reach 512 MiB
    assert len(tune.operands_for(8, 8192, 8192, big)) == 4
    ops = tune.operands_for(4096, 1024, 1024, x2)                   # 256 tiles: tile-GEMM regime
    assert len(ops) == 1 and ops[0] is x2
    small = torch.ones(64, 64)                                        # under 1 MiB
    ops = tune.operands_for(1, 64, 64, small)
    assert len(ops) == 1 and ops[0] is small


def test_exported_trees_match_sklearn(tmp_path):
    from sklearn.ensemble import GradientBoostingRegressor
    rng = np.random.default_rng(0)
    X = rng.normal(size=(400, 6))
    y = np.sin(X[:, 0]) + X[:, 1] * X[:, 2] + 0.1 * rng.normal(size=400)
    m = GradientBoostingRegressor(n_estimators=50, max_depth=3, learning_rate=0.1, random_state=0).fit(X, y)
    path = tmp_path / "m.json"
    tune.export(m, str(path))
    import json
    tm = tune.TreeModel(json.loads(path.read_text()))
    Xt = rng.normal(size=(100, 6))
    np.testing.assert_allclose(tm.predict(Xt), m.predict(Xt), rtol=1e-12, atol=1e-12)


def test_pick_returns_a_valid_config_or_none():
    for M, K, N, dt in [(16, 4096, 4096, "f32"), (4096, 4096, 4096, "f32"), (8192, 8192, 8192, "bf16")]:
        p = tune.pick(M, K, N, dt)
        assert p is None or p in ext.hip_configs(M, K, N, dt)
    assert tune.pick(0, 5, 5) is None


def test_pick_uses_measured_best_for_benchmarked_shapes():
    if not os.path.exists(tune.DATA) or not os.path.exists(tune.MODEL):
        pytest.skip("no MI355X tuning data committed yet")
    best = tune.best_table(tune.load())
    for shape in [s + (0,) for s in tune.CONFIG_SHAPES] + tune.LAYOUT_CONFIG_SHAPES:
        key = ",".join(map(str, shape))
        if key not in best:
            continue  # not benchmarked in this layout yet
        assert tune.pick(*shape) == tuple(best[key]), shape


def test_committed_tuning_data_schema():
    if not os.path.exists(tune.DATA):
        pytest.skip("no MI355X tuning data committed yet")
    rows = tune.load()
    assert rows and set(rows[0]) == set(tune.FIELDS)
    assert all(r["ms"] > 0 for r in rows)


# ---------------------------------------------------------------------------
# C ABI
# ---------------------------------------------------------------------------

def _declared_functions():
    src = open(os.path.join(ROOT, "include", "tilec.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(tilec_\w+)\s*\(", src)))


def test_header_declares_what_the_binding_binds():
    declared = _declared_functions()
    assert declared == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    L = ctypes.CDLL(_lib.LIB_PATH)
    for name in _declared_functions():
        assert hasattr(L, name), name


def test_version_and_variants():
    L = _lib.lib()
    assert L.tilec_version() == 10100
    vs = _lib.variants()
    assert len(vs) == L.tilec_num_variants() > 0
    assert len({v["name"] for v in vs}) == len(vs)
    fams = {(v["family"], v["dtype"]) for v in vs}
    assert (_lib.FAMILY_SKINNY, _lib.F32) in fams
    assert (_lib.FAMILY_GEMM, _lib.F32) in fams and (_lib.FAMILY_GEMM, _lib.BF16) in fams
    assert _lib.lib().tilec_variant_info(len(vs), None, None) == _lib.ERR_UNSUPPORTED


def _call(M=8, N=8, K=8, ldx1=None, ldx2=None, ldo=None, dtype=0, variant=-1, split=0,
          ws=None, ws_bytes=0, cnt=None, cnt_bytes=0, x1=16, x2=16, out=16, layout=0):
    # Non-null dummy pointers: every case below must fail validation before launch.
    L = _lib.lib()
    c1, c2 = layout & _lib.X1_COL_MAJOR, layout & _lib.X2_COL_MAJOR
    return L.tilec_matmul(x1, x2, out, M, N, K, ldx1 if ldx1 is not None else (M if c1 else K),
                          ldx2 if ldx2 is not None else (K if c2 else N), ldo if ldo is not None else N,
                          layout, dtype, variant, split, ws, ws_bytes, cnt, cnt_bytes, None)


def test_abi_rejects_bad_arguments_before_launch():
    assert _call(dtype=7) == _lib.ERR_TYPE
    assert _call(M=-1) == _lib.ERR_VALUE
    assert _call(K=1 << 40) == _lib.ERR_VALUE
    assert _call(split=-2) == _lib.ERR_VALUE
    assert _call(ldx1=3) == _lib.ERR_VALUE
    assert _call(ldx2=3) == _lib.ERR_VALUE
    assert _call(ldo=3) == _lib.ERR_VALUE
    # Column-major operands: the stride runs over columns and covers the rows.
    assert _call(M=8, K=4, ldx1=4, layout=_lib.X1_COL_MAJOR) == _lib.ERR_VALUE
    assert "ldx1=4 < M=8" in _lib.last_error()
    assert _call(K=8, N=4, ldx2=4, layout=_lib.X2_COL_MAJOR) == _lib.ERR_VALUE
    assert "ldx2=4 < K=8" in _lib.last_error()
    assert _call(layout=4) == _lib.ERR_VALUE
    assert "layout" in _lib.last_error()
    assert _call(out=None) == _lib.ERR_VALUE
    assert _call(x1=None) == _lib.ERR_VALUE
    assert _call(variant=10 ** 6) == _lib.ERR_UNSUPPORTED
    skinny = _lib.variant_id("skinny_f32_w8_b1")
    gemm = _lib.variant_id("gemm_f32_128x128x16_w2x2")
    bf16 = _lib.variant_id("gemm_bf16_128x128x64_r4")
    # The streaming kernel takes any M in 16-row blocks, up to 65535 of them.
    assert _call(M=16 * 65535 + 1, variant=skinny) == _lib.ERR_UNSUPPORTED
    assert "M <=" in _lib.last_error()
    # Its 32-bit block offsets bound the strides: column-major x2 spans a
    # slab of 64 columns, so its column stride stays below 2^23.
    assert _call(M=4, N=64, K=64, ldx2=1 << 23, variant=skinny, layout=_lib.X2_COL_MAJOR) == _lib.ERR_UNSUPPORTED
    assert "2^23" in _lib.last_error()
    assert _call(M=4, N=64, K=64, ldx2=1 << 25, variant=skinny) == _lib.ERR_UNSUPPORTED
    assert _call(variant=bf16, dtype=0) == _lib.ERR_UNSUPPORTED
    # Tile GEMMs split K (workspace required) unless a thread's tile is too big to.
    assert _call(M=64, N=64, K=4096, variant=gemm, split=2) == _lib.ERR_WORKSPACE
    assert _call(K=4096, variant=_lib.variant_id("gemm_f32_256x256x16_w2x2"), split=2) == _lib.ERR_UNSUPPORTED
    # Split K needs a workspace.
    assert _call(M=4, N=256, K=4096, variant=skinny, split=4) == _lib.ERR_WORKSPACE
    assert "workspace" in _lib.last_error()
    # ... and zeroed counters
    assert _call(M=4, N=256, K=4096, variant=skinny, split=4, ws=16, ws_bytes=1 << 30) == _lib.ERR_WORKSPACE
    assert "counters" in _lib.last_error()
    with pytest.raises(ValueError):
        _lib.check(_call(M=-1))
    with pytest.raises(TypeError):
        _lib.check(_call(dtype=9))
    with pytest.raises(RuntimeError):
        _lib.check(_call(variant=10 ** 6))


def test_noalloc_rejects_oversized_scratch_before_launch():
    # A call whose split K needs more than the static scratch fails before
    # anything touches a device (dummy pointers, no GPU needed).
    L = _lib.lib()
    prep = _lib.variant_id("gemm_bf16_256x256x64_r2_kc")
    n = 8192
    assert L.tilec_matmul_workspace_bytes(n, n, n, _lib.BF16, prep, 1) > 16 << 20
    rc = L.tilec_matmul_noalloc(16, 16, 16, n, n, n, n, n, n, 0, _lib.BF16, prep, 1, None)
    assert rc == _lib.ERR_WORKSPACE
    assert "tilec_matmul_noalloc has" in _lib.last_error()
    # Argument errors are reported as by tilec_matmul.
    assert L.tilec_matmul_noalloc(16, 16, 16, -1, 8, 8, 8, 8, 8, 0, 0, -1, 0, None) == _lib.ERR_VALUE
    assert L.tilec_matmul_noalloc(16, 16, 16, 8, 8, 8, 8, 8, 8, 0, 7, -1, 0, None) == _lib.ERR_TYPE
    # M == 0: nothing to do, no device access.
    assert L.tilec_matmul_noalloc(None, None, None, 0, 8, 8, 8, 8, 8, 0, 0, -1, 0, None) == _lib.OK


def test_panel_variants_check_their_own_split_geometry():
    # The panel kernel takes at least K / KC splits (KC = 512 fp32 / 256 bf16
    # rows) and addresses its partials with 32-bit offsets: shapes whose
    # partials reach 2 GiB, or whose splits pass the grid's 65535, are
    # rejected before launch, and the size queries answer 0 for them.
    L = _lib.lib()
    pb = _lib.variant_id("skinny_bf16_p_v1_w8")
    pf = _lib.variant_id("skinny_f32_p_v1_w8")
    for v, dt, K in [(pb, _lib.BF16, 1 << 22), (pf, _lib.F32, 1 << 22)]:
        assert L.tilec_matmul_workspace_bytes(1, 4096, K, dt, v, 0) == 0, (v, K)
        assert _call(M=1, N=4096, K=K, dtype=dt, variant=v, split=0, ws=16, ws_bytes=1 << 40,
                     cnt=16, cnt_bytes=1 << 30) == _lib.ERR_UNSUPPORTED
        assert "2 GiB" in _lib.last_error()
    assert _call(M=1, N=64, K=1 << 24, dtype=_lib.BF16, variant=pb, split=0) == _lib.ERR_VALUE
    assert "65535" in _lib.last_error()
    # the config-1 size still resolves: 8 splits x 32 panels of 16-row x 128-column partial slots
    assert L.tilec_matmul_workspace_bytes(1, 4096, 4096, _lib.F32, pf, 8) == 8 * 32 * 16 * 128 * 4


def _scratch(M, N, K, ldx1, ldx2, layout, dtype=0, variant=-1, split=0):
    ws, cnt = ctypes.c_size_t(7), ctypes.c_size_t(7)
    rc = _lib.lib().tilec_matmul_scratch_bytes(M, N, K, ldx1, ldx2, layout, dtype, variant, split,
                                               ctypes.byref(ws), ctypes.byref(cnt))
    return rc, ws.value, cnt.value


def test_scratch_query_follows_layout_and_strides():
    L = _lib.lib()
    # M=8, K=200, N=64 with a row stride of x2 past the streaming kernel's
    # 2^25 bound: the automatic pick is the direct kernel, whose split K
    # needs scratch; the layout-blind query (contiguous strides) sees the
    # streaming kernel instead.
    ld = (1 << 25) + 64
    rc, ws, cnt = _scratch(8, 64, 200, 0, ld, 0)
    assert rc == _lib.OK and ws > 0 and cnt > 0
    assert _lib.variants()[L.tilec_select_variant_layout(8, 64, 200, 0, 0, 0, ld)]["name"].startswith("direct_")
    # the same answer as the layout-blind queries for contiguous row-major operands
    for M, N, K in [(1, 4096, 4096), (16, 4096, 4096), (200, 3000, 1500), (4096, 4096, 4096)]:
        assert _scratch(M, N, K, 0, 0, 0)[1:] == (L.tilec_matmul_workspace_bytes(M, N, K, 0, -1, 0),
                                                   L.tilec_matmul_counter_bytes(M, N, K, 0, -1, 0))
    # errors come back as tilec_matmul's status, with zero sizes
    assert _scratch(-1, 8, 8, 0, 0, 0) == (_lib.ERR_VALUE, 0, 0)
    assert _scratch(8, 8, 8, 0, 0, 4) == (_lib.ERR_VALUE, 0, 0)
    assert _scratch(8, 8, 8, 0, 0, 0, dtype=5) == (_lib.ERR_TYPE, 0, 0)
    assert _scratch(0, 8, 8, 0, 0, 0) == (_lib.OK, 0, 0)
    # ext sizes a call with the same query
    assert ext._scratch_sizes(8, 64, 200, 200, ld, 0, 0, -1, 0) == (ws, cnt)


def test_pad_variants_offered_for_unaligned_rows_and_sized():
    """The fp32 *_pad variants (both operands copied into the workspace with
    rows padded to 16 bytes and K to the K step) are offered only where an
    operand's rows are not whole 16-byte groups, and their scratch is the two
    padded copies (each 256-byte aligned) plus the split-K partials."""
    pads = lambda M, K, N, layout=0: {c for c in ext.hip_configs(M, K, N, "f32", layout) if c[0].endswith("_pad")}
    assert pads(1000, 4097, 3001) and pads(3001, 513, 1000) and pads(1024, 1024, 1022)
    assert not pads(1024, 1024, 1024) and not pads(4096, 4096, 4096)
    # bf16: 16-byte groups are 8 elements
    bpads = lambda M, K, N, layout=0: {c for c in ext.hip_configs(M, K, N, "bf16", layout) if c[0].endswith("_pad")}
    assert bpads(1000, 4097, 3001) and bpads(1024, 1024, 1020) and not pads(1024, 1024, 1020)
    assert not bpads(1024, 1024, 1024) and not bpads(8192, 8192, 8192) and not bpads(1024, 1020, 1024, _lib.X1_COL_MAJOR)
    assert ext.needs_pad(1024, 1020, 1024, 0, "bf16") and not ext.needs_pad(1024, 1020, 1024, 0, "f32")
    # layout: a column-major x1 is contiguous along M, a column-major x2 along K
    assert ext.needs_pad(1001, 1024, 1024, _lib.X1_COL_MAJOR) and not ext.needs_pad(1001, 1024, 1024)
    assert ext.needs_pad(1024, 1024, 1001) and not ext.needs_pad(1024, 1024, 1001, _lib.X2_COL_MAJOR)
    vid = _lib.variant_id("gemm_f32_128x128x32_w2x4_pad")
    M, N, K = 1000, 3001, 4097
    kp, m4, n4 = 4128, 1000, 3004
    copies = -(-m4 * kp * 4 // 256) * 256 + -(-n4 * kp * 4 // 256) * 256
    rc, ws, cnt = _scratch(M, N, K, 0, 0, 0, variant=vid, split=1)
    assert rc == _lib.OK and (ws, cnt) == (copies, 0)
    tiles = 8 * 24
    rc, ws, cnt = _scratch(M, N, K, 0, 0, 0, variant=vid, split=4)
    assert rc == _lib.OK and ws == copies + 4 * tiles * 128 * 128 * 4 and cnt == tiles * 64 * 4
    vid = _lib.variant_id("gemm_bf16_128x128x64_r4_m16_pad")
    kp, m8, n8 = 4160, 1000, 3008
    copies = -(-m8 * kp * 2 // 256) * 256 + -(-n8 * kp * 2 // 256) * 256
    rc, ws, cnt = _scratch(M, N, K, 0, 0, 0, dtype=_lib.BF16, variant=vid, split=1)
    assert rc == _lib.OK and (ws, cnt) == (copies, 0)
    rc, ws, cnt = _scratch(M, N, K, 0, 0, 0, dtype=_lib.BF16, variant=vid, split=4)
    assert rc == _lib.OK and ws == copies + 4 * tiles * 128 * 128 * 4 and cnt == tiles * 64 * 4


def test_hip_configs_of_empty_outputs():
    for M, K, N in [(0, 64, 64), (4, 64, 0), (0, 0, 0)]:
        for dt in ("f32", "bf16"):
            cfgs = ext.hip_configs(M, K, N, dt)
            assert isinstance(cfgs, list)
            assert not any(c[0].startswith("direct_") for c in cfgs)


def test_read_floor_rejects_bad_arguments_before_launch():
    L = _lib.lib()
    assert L.tilec_read_floor(16, 16384 + 16, 16, 0, None) == _lib.ERR_VALUE
    assert "16 KiB" in _lib.last_error()
    assert L.tilec_read_floor(8, 16384, 16, 0, None) == _lib.ERR_VALUE  # not 16-byte aligned
    assert L.tilec_read_floor(None, 16384, 16, 0, None) == _lib.ERR_VALUE
    assert L.tilec_read_floor(16, 16384, None, 0, None) == _lib.ERR_VALUE
    assert L.tilec_read_floor(16, 16384, 16, -1, None) == _lib.ERR_VALUE
    assert L.tilec_read_floor(None, 0, None, 0, None) == _lib.OK  # nothing to read


def test_abi_empty_outputs_enqueue_nothing():
    # M == 0 or N == 0: nothing to do, no device access (null pointers are fine).
    assert _call(M=0, x1=None, x2=None, out=None) == _lib.OK
    assert _call(N=0, x1=None, x2=None, out=None) == _lib.OK


def test_workspace_geometry():
    L = _lib.lib()
    v = _lib.variant_id("skinny_f32_w8_b1")
    part = 16 * 64 * 4  # partial sums per split and 64-column slab
    assert L.tilec_matmul_workspace_bytes(16, 1000, 1000, 0, v, 1) == 0
    assert L.tilec_matmul_counter_bytes(16, 1000, 1000, 0, v, 1) == 0
    # a workgroup takes at most 1024 rows of K: K=4096 runs at least 4 splits
    assert L.tilec_matmul_workspace_bytes(16, 4096, 4096, 0, v, 1) == 4 * 64 * part
    # 64 slabs, 8 splits; one counter per slab, each on its own 256-byte line
    assert L.tilec_matmul_counter_bytes(16, 4096, 4096, 0, v, 8) == 64 * 256
    assert L.tilec_matmul_workspace_bytes(16, 4096, 4096, 0, v, 8) == 8 * 64 * part
    # splits are recomputed so that none is empty: K=100 in 16-row chunks -> 7 splits
    assert L.tilec_matmul_workspace_bytes(1, 64, 100, 0, v, 8) == 7 * part
    assert L.tilec_matmul_workspace_bytes(1, 64, 10, 0, v, 8) == 0  # one 16-row chunk
    # Python's view of the split rule agrees with the library's
    for K, s in [(4096, 1), (4096, 8), (100, 8), (10, 8), (5000, 3), (65536, 2)]:
        nbytes = L.tilec_matmul_workspace_bytes(1, 64, K, 0, v, s)
        eff = ext._skinny_splits(K, s, 1024)
        assert nbytes == (0 if eff == 1 else eff * part), (K, s)
    assert L.tilec_matmul_workspace_bytes(16, 4096, 4096, 0, _lib.variant_id("gemm_f32_128x128x16_w2x2"), 1) == 0
    s = L.tilec_auto_split_k(16, 4096, 4096, 0, v)
    assert 1 <= s <= 4096 // (4 * 8 * 4)
    # tile GEMMs: 32 tiles of 128 x 128 split K to fill the CUs; 1024 tiles do not split
    g = _lib.variant_id("gemm_f32_128x128x16_w2x2")
    assert L.tilec_auto_split_k(16, 4096, 4096, 0, g) == 8
    assert L.tilec_auto_split_k(4096, 4096, 4096, 0, g) == 1


def test_select_variant_rules():
    L = _lib.lib()
    names = [v["name"] for v in _lib.variants()]
    assert names[L.tilec_select_variant(1, 4096, 4096, 0)].startswith("skinny_f32")
    assert names[L.tilec_select_variant(4096, 4096, 4096, 0)].startswith("gemm_f32")
    # medium fp32 outputs: the direct-to-LDS 64x64 tile where its tiles give each CU one or two, else the
    # direct kernel's two-register-set 32x64 tile, unless 128x128 tiles fill the CUs
    assert names[L.tilec_select_variant(1024, 1024, 1024, 0)] == "gemm_f32_64x64x32_w2x2_lds"
    assert names[L.tilec_select_variant(3001, 1000, 513, 0)] == "direct_f32_32x64_w4_db"  # M, N, K
    assert names[L.tilec_select_variant(2048, 2048, 2048, 0)].startswith("gemm_f32")
    assert names[L.tilec_select_variant(8192, 8192, 8192, 1)].startswith("gemm_bf16")
    assert names[L.tilec_select_variant(4, 4096, 4096, 1)].startswith("skinny_bf16")
    assert names[L.tilec_select_variant(17, 4096, 4096, 1)].startswith("gemm_bf16")
    assert L.tilec_select_variant(4, 4, 4, 5) == -_lib.ERR_TYPE
    # layout-aware: x @ W.T takes the row-dot (M = 1) / row-tile kernels
    wt = _lib.X2_COL_MAJOR
    assert names[L.tilec_select_variant_layout(1, 4096, 4096, 0, wt, 0, 0)] == "skinny_f32_t1_r1_w8_u2"
    assert names[L.tilec_select_variant_layout(16, 4096, 4096, 1, wt, 0, 0)] == "skinny_bf16_t16_r16_w8_c128"
    assert L.tilec_select_variant_layout(1, 4096, 4096, 0, 0, 0, 0) == L.tilec_select_variant(1, 4096, 4096, 0)
    # unaligned K or strides: the row-dot kernel takes them, the row-tile kernel does not
    assert names[L.tilec_select_variant_layout(1, 4096, 4097, 0, wt, 0, 4099)] == "skinny_f32_t1_r1_w8_u2"
    assert names[L.tilec_select_variant_layout(1, 4096, 4095, 1, wt, 4095, 4095)] == "skinny_bf16_t1_r1_w8_u2"
    assert not names[L.tilec_select_variant_layout(8, 4096, 4097, 0, wt, 0, 4099)].endswith("_c128")
    assert L.tilec_select_variant_layout(4, 4, 4, 0, 8, 0, 0) == -_lib.ERR_VALUE


def test_operand_layouts_read_in_place():
    """Row-strided and transposed views go to the kernels as they are (layout
    bits and leading dimensions), everything else is copied to row-major."""
    a = torch.zeros(6, 10)
    t, ld, col = ext._operand(a, 6, 10)
    assert (t.data_ptr(), ld, col) == (a.data_ptr(), 10, False)
    v = a[:, 2:7]                                   # row stride 10 >= 5 columns
    t, ld, col = ext._operand(v, 6, 5)
    assert (t.data_ptr(), ld, col) == (v.data_ptr(), 10, False)
    at = a.t()                                      # [10, 6] column-major, column stride 10
    t, ld, col = ext._operand(at, 10, 6)
    assert (t.data_ptr(), ld, col) == (a.data_ptr(), 10, True)
    sub = a[1:5, :].t()                             # [10, 4] column-major, column stride 10 >= 10 rows
    t, ld, col = ext._operand(sub, 10, 4)
    assert (t.data_ptr(), ld, col) == (sub.data_ptr(), 10, True)
    # vectors: size-1 dimensions impose no stride, row-major preferred
    row = a[2:3, :]
    assert ext._operand(row, 1, 10)[1:] == (10, False)
    colv = a[:, 3:4]
    assert ext._operand(colv, 6, 1)[1:] == (10, False)
    colt = a[3:4, :].t()                            # [10, 1]: stride (1, 10)
    assert ext._operand(colt, 10, 1)[1:] == (1, False)  # element (r, 0) at r * 1
    # neither layout: every other element, broadcast -> contiguous copies
    every_other = a.t()[:, ::2]                     # [10, 3], strides (1, 20): column-major, ld 20
    t, ld, col = ext._operand(every_other, 10, 3)
    assert (t.data_ptr(), ld, col) == (a.data_ptr(), 20, True)
    for x, (r, c) in ((a[:, ::2], (6, 5)), (torch.zeros(1, 10).expand(6, 10), (6, 10)), (a[::2, ::2], (3, 5))):
        t, ld, col = ext._operand(x, r, c)
        assert t.is_contiguous() and ld == c and col is False
        assert torch.equal(t, x)
    assert ext.layout_of(a, a.t()) == _lib.X2_COL_MAJOR
    assert ext.layout_of(a.t(), a) == _lib.X1_COL_MAJOR
    assert ext.layout_of(a.t(), a.t().t()) == _lib.X1_COL_MAJOR


# ---------------------------------------------------------------------------
# Sums: C ABI validation and split geometry (no device calls)
# ---------------------------------------------------------------------------

def _sum_call(R=8, C=8, ldx=None, layout=0, dtype=0, axis=1, ws=None, ws_bytes=0, cnt=None, cnt_bytes=0,
              x=16, out=16):
    # Non-null dummy pointers: every case must fail (or finish) before launch.
    L = _lib.lib()
    return L.tilec_sum(x, out, R, C, ldx if ldx is not None else (R if layout else C), layout, dtype, axis,
                       ws, ws_bytes, cnt, cnt_bytes, None)


def test_sum_abi_rejects_bad_arguments_before_launch():
    assert _sum_call(dtype=5) == _lib.ERR_TYPE
    assert _sum_call(axis=2) == _lib.ERR_VALUE and "axis" in _lib.last_error()
    assert _sum_call(layout=_lib.X2_COL_MAJOR) == _lib.ERR_VALUE
    assert _sum_call(R=-1) == _lib.ERR_VALUE
    assert _sum_call(ldx=3) == _lib.ERR_VALUE and "ldx=3 < C=8" in _lib.last_error()
    assert _sum_call(C=4, ldx=3, layout=_lib.X1_COL_MAJOR) == _lib.ERR_VALUE and "ldx=3 < R=8" in _lib.last_error()
    assert _sum_call(out=None) == _lib.ERR_VALUE
    assert _sum_call(x=None) == _lib.ERR_VALUE
    # no outputs: nothing to do, no device access
    assert _sum_call(R=0, x=None, out=None) == _lib.OK
    assert _sum_call(C=0, axis=0, x=None, out=None) == _lib.OK
    # a few long rows split their columns: workspace, then zeroed counters
    assert _sum_call(R=4, C=1 << 20) == _lib.ERR_WORKSPACE and "workspace" in _lib.last_error()
    assert _sum_call(R=4, C=1 << 20, ws=16, ws_bytes=1 << 30) == _lib.ERR_WORKSPACE
    assert "counters" in _lib.last_error()
    # rows too long for 32-bit offsets
    assert _sum_call(R=1, C=(1 << 29) + 1, ldx=(1 << 29) + 1) == _lib.ERR_UNSUPPORTED


def test_sum_geometry():
    L = _lib.lib()
    ws = L.tilec_sum_workspace_bytes
    cnt = L.tilec_sum_counter_bytes
    # 4096 rows of 4096: a wave per row, 1024 workgroups: no split
    assert ws(4096, 4096, 0, 0, 1) == 0 and cnt(4096, 4096, 0, 0, 1) == 0
    # 4 long rows: one workgroup of rows, columns split; partials of 256 floats
    # per workgroup and split, one counter line per workgroup
    w = ws(4, 1 << 20, 0, 0, 1)
    assert w > 0 and w % (256 * 4) == 0 and cnt(4, 1 << 20, 0, 0, 1) == 256
    # column sums of 4096 x 4096: 64 slabs of 64 columns, rows split 8 ways
    assert ws(4096, 4096, 0, 0, 0) == 8 * 64 * 256 * 4 and cnt(4096, 4096, 0, 0, 0) == 64 * 256
    # bf16 slabs are 128 columns wide
    assert cnt(4096, 4096, 0, 1, 0) == 32 * 256
    # a column-major matrix sums like the row-major transpose along the other axis
    assert ws(1 << 20, 4, _lib.X1_COL_MAJOR, 0, 0) == w
    assert ws(4096, 4096, _lib.X1_COL_MAJOR, 0, 1) == ws(4096, 4096, 0, 0, 0)
    # short rows (C <= 16 fp32): one lane per row, 256 rows per workgroup
    assert ws(1 << 20, 8, 0, 0, 1) == 0
    # invalid arguments size nothing
    assert ws(4, 1 << 20, 0, 0, 7) == 0


def test_prep_variants_workspace_and_splits():
    """*_kc variants hold transposed copies of both operands in the workspace
    (256-byte aligned, sized for any layout) and never split K."""
    L = _lib.lib()
    v = _lib.variant_id("gemm_bf16_256x256x64_r2_kc")
    M, N, K = 1000, 520, 3000
    a = (M * K * 2 + 255) // 256 * 256
    b = (K * N * 2 + 255) // 256 * 256
    assert L.tilec_matmul_workspace_bytes(M, N, K, _lib.BF16, v, 1) == a + b
    assert L.tilec_matmul_counter_bytes(M, N, K, _lib.BF16, v, 1) == 0
    assert L.tilec_matmul_workspace_bytes(M, N, 0, _lib.BF16, v, 1) == 0
    assert L.tilec_auto_split_k(64, 64, 4096, _lib.BF16, v) == 1
    assert _call(M=64, N=64, K=4096, dtype=_lib.BF16, variant=v, split=2) == _lib.ERR_UNSUPPORTED
    assert _call(M=64, N=64, K=4096, dtype=_lib.BF16, variant=v, split=1) == _lib.ERR_WORKSPACE
    kc = [c for c in ext.hip_configs(64, 4096, 64, "bf16") if c[0].endswith("_kc")]
    assert kc and all(s == 1 for _, s in kc)
