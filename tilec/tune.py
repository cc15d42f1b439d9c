"""Shape → kernel-config model for MI355X, after the reference's tuner
(tilec/tune.py).

    python -m tilec.tune bench [n]   # time every config on random shapes → CSV
    python -m tilec.tune train       # fit the model, report held-out quality, export JSON

Same method as the reference: benchmark every valid config of every shape
into a resumable CSV (tilec/tune.py:68-87), fit a gradient-boosted regressor
on log(ms) (tilec/tune.py:99-132), and let `pick` take the argmin of the
predicted time over the configs valid for a shape (tilec/tune.py:143-151).
What differs:
  * the configs are the compiled gfx950 variants × split_k (`ext.hip_configs`);
  * `machine()` queries the ROCm device instead of macOS `sysctl`;
  * shapes include the skinny M <= 16 regime and bf16;
  * short calls are timed from replayed HIP graphs, and streaming-regime
    shapes cycle x2 over copies larger than the Infinity Cache;
  * the fitted trees are exported to JSON and evaluated here with numpy, so
    `pick` needs neither scikit-learn nor a pickle at run time;
  * the export also carries the measured best config of every benchmarked
    shape, which `pick` returns for those exact shapes (the model predicts
    the rest).
"""

import csv
import json
import math
import os
import random
import re
import sys
from functools import lru_cache

from . import _lib
from .language import cdiv

HERE = os.path.dirname(os.path.abspath(__file__))
DATA = os.path.join(HERE, "mm_bench_mi355x.csv")
MODEL = os.path.join(HERE, "mm_model_mi355x.json")
FIELDS = ["chip", "cus", "M", "K", "N", "dtype", "layout", "kernel", "BM", "BN", "BK", "split_k", "ms"]


@lru_cache(None)
def machine():
    """(chip name, compute units) of GPU 0 — replaces the macOS query of
    tilec/tune.py:19-26."""
    import torch
    p = torch.cuda.get_device_properties(0)
    arch = getattr(p, "gcnArchName", "") or ""
    return f"{p.name} {arch.split(':')[0]}".strip(), int(p.multi_processor_count)


@lru_cache(None)
def _variant_by_name():
    return {v["name"]: v for v in _lib.variants()}


PEAK_FLOPS = {"f32": 157.3e12, "bf16": 2516.6e12}  # MI355X dense matrix peaks
PEAK_HBM = 8e12        # bytes/s
PEAK_L2_READ = 20e12   # bytes/s, operand re-reads served by the L2s and the Infinity Cache (order of magnitude)
LAUNCH_S = 3e-6        # a launch's fixed cost on MI355X (the 1x1x1 product's device time)
COMBINE_S = 1.5e-6     # a split-K count-and-combine after the last row


def prepass(M, K, N, dtype, kernel, layout=0):
    """(launches, bytes moved) of the copies a variant makes before its GEMM:
    the transposing variants (`*_kc`) transpose each operand that is not
    k-contiguous (none when M, N or K is not a multiple of 8: the plain tile
    runs), the pad variants (`*_pad`) copy both operands."""
    esz = 4 if dtype == "f32" else 2
    if kernel.endswith("_pad"):
        return 2, 2 * esz * (M * K + K * N)
    if kernel.endswith("_kc") and M % 8 == 0 and N % 8 == 0 and K % 8 == 0:
        t1, t2 = bool(layout & _lib.X1_COL_MAJOR), not layout & _lib.X2_COL_MAJOR
        if t1 or t2:
            return int(t1) + int(t2), 2 * esz * (M * K * t1 + K * N * t2)
    return 0, 0


def roofline(M, K, N, cus, dtype, kernel, split_k, layout=0):
    """Analytic estimate for one (shape, config), the terms the trees cannot
    derive from sizes alone: the time at the matrix peak scaled by the share
    of CUs the grid fills and by the tile padding, the algorithmic HBM bytes
    (plus split-K partials written and read back), the operand re-reads of
    the tile grid, a launch and a combine, and any copies of the operands
    before the GEMM (`prepass`: a launch each, their bytes at half the HBM
    rate); also the padding efficiency, the fill of the last round of
    workgroups and the K rows each wave takes.  Returns (t_est, t_compute,
    t_hbm, t_reread, pad, tail, fill, k_per_wave, rounds)."""
    v = _variant_by_name()[kernel]
    esz = 4 if dtype == "f32" else 2
    bm, bn = v["bm"], v["bn"]
    tiles = cdiv(M, bm) * cdiv(N, bn)
    wgs = tiles * split_k
    slots = cus * (1 if v["waves"] >= 8 else 2)
    rounds = max(1, cdiv(wgs, slots))
    tail = wgs / (rounds * slots)
    fill = min(1.0, wgs / cus)
    pad = (M * N) / max(1, tiles * bm * bn)
    t_c = 2.0 * M * N * K / (PEAK_FLOPS[dtype] * max(fill * pad, 1e-9))
    t_m = (esz * (M * K + K * N) + 4 * M * N + (8.0 * tiles * bm * bn * split_k if split_k > 1 else 0)) / PEAK_HBM
    t_r = esz * (M * K * cdiv(N, bn) + K * N * cdiv(M, bm)) / PEAK_L2_READ
    launches, moved = prepass(M, K, N, dtype, kernel, layout)
    t_est = (max(t_c, t_m, t_r) + LAUNCH_S * (1 + launches) + 2.0 * moved / PEAK_HBM +
             (COMBINE_S if split_k > 1 else 0))
    return t_est, t_c, t_m, t_r, pad, tail, fill, max(1.0, K / split_k / v["waves"]), float(rounds)


def features(M, K, N, cus, dtype, kernel, split_k, layout=0):
    """Model inputs for one (shape, config); the role of tilec/tune.py:29-32.

    Shape and config sizes enter as log2, plus the derived quantities that
    decide occupancy: workgroups launched per CU and the K rows per split,
    the operand layout bits (x1, x2 column-major) and the variant's row
    bound (max_m; 0 = any M), which tells the FMA streaming variants apart;
    then the analytic terms of `roofline` (times as log2 seconds), and
    whether each operand's contiguous extent (K or M for x1, N or K for x2)
    is a whole number of 16-byte groups: the direct-to-LDS, row-dot and
    row-tile kernels take only such operands and run a slower fallback of
    the same tile for the others, a difference the sizes alone do not show
    the trees (on MI355X it took the held-out worst case from 2.3x to 1.5x).
    Then three variant properties the descriptor sizes do not carry: 16x16
    MFMA blocks (`*_m16`), operands transposed (`*_kc`) or padded (`*_pad`)
    into the workspace first — otherwise such a variant and its plain
    counterpart look the same to the trees.  Last, whether this config runs
    a slower fallback of its tile for these operands (`falls_back`): the
    alignment bits alone describe the shape, and the trees then have to
    learn which variants they matter for.
    """
    v = _variant_by_name()[kernel]
    tiles = cdiv(M, v["bm"]) * cdiv(N, v["bn"])
    wgs = tiles * split_k
    lg = lambda x: math.log2(max(1, x))
    t_est, t_c, t_m, t_r, pad, tail, fill, kpw, rounds = roofline(M, K, N, cus, dtype, kernel, split_k, layout)
    ls = lambda t: math.log2(max(t, 1e-12))
    return [lg(M), lg(K), lg(N), cus, 1.0 if dtype == "bf16" else 0.0,
            float(v["family"]), lg(v["bm"]), lg(v["bn"]), lg(v["bk"]), float(v["waves"]),
            float(v["unroll"]), lg(split_k), lg(tiles), math.log2(max(1, wgs) / cus),
            lg(cdiv(K, split_k)), lg(M * K * N),
            float(layout & _lib.X1_COL_MAJOR != 0), float(layout & _lib.X2_COL_MAJOR != 0),
            float(v["max_m"]),
            ls(t_est), ls(t_c), ls(t_m), ls(t_r), pad, tail, fill, lg(kpw), rounds,
            float(aligned(M if layout & _lib.X1_COL_MAJOR else K, dtype)),
            float(aligned(K if layout & _lib.X2_COL_MAJOR else N, dtype)),
            float("_m16" in kernel), float(kernel.endswith("_kc")), float(kernel.endswith("_pad")),
            float(falls_back(kernel, M, K, N, dtype, layout))]


def falls_back(kernel, M, K, N, dtype, layout=0):
    """Whether a variant runs a slower form of its kernel for these operands:
    the direct-to-LDS tiles (fp32 `*_lds`, the bf16 tiles with a ring of
    stage buffers) take only operands whose contiguous extents are whole
    16-byte groups and run a register-staged fallback otherwise.  The bf16
    transposing variants (`*_kc`) copy operands whose M, N and K are
    multiples of 8 into that form and run the plain tile on the others.  The
    row-dot kernel (`x @ W.T`, M <= 4) shifts every 16-byte piece into place
    when K is not a whole number of 16-byte groups.  The pad variants exist
    for the other shapes and never fall back."""
    v = _variant_by_name()[kernel]
    if v["family"] == _lib.FAMILY_SKINNY and re.search(r"_t\d+_r\d+_", kernel) and not kernel.endswith(
            ("_c128", "_c256")):
        return not aligned(K, dtype)
    if v["family"] != _lib.FAMILY_GEMM or kernel.endswith("_pad"):
        return False
    if kernel.endswith("_kc") and M % 8 == 0 and N % 8 == 0 and K % 8 == 0:
        return False
    lds = kernel.endswith("_lds") if dtype == "f32" else v["unroll"] >= 2
    return lds and not (aligned(M if layout & _lib.X1_COL_MAJOR else K, dtype) and
                        aligned(K if layout & _lib.X2_COL_MAJOR else N, dtype))


def aligned(extent, dtype):
    """A contiguous extent of whole 16-byte groups (4 fp32 / 8 bf16 elements)."""
    return extent % (4 if dtype == "f32" else 8) == 0


GRAPH_BELOW_MS = 0.2   # calls shorter than this are timed from a replayed HIP graph
GRAPH_FILL_MS = 2.0    # ... of this much device time per replay (at most 256 calls)
SUSTAIN_CALLS = 4      # longer calls: back-to-back launches per timed sample
SUSTAIN_WARMUP = 4     # ... after this many untimed back-to-back launches
ROTATE_BYTES = 512 << 20  # rotate x2 over copies this large in total (> 256 MB Infinity Cache)


def operands_for(M, K, N, x2):
    """The x2 operands a timing cycles through: for small-output shapes (the
    streaming regime, where x2 is read once per call) enough copies that
    they cannot all stay in the 256 MB Infinity Cache, as weights streamed
    from HBM would not; otherwise x2 alone."""
    from . import ext
    nbytes = x2.numel() * x2.element_size()
    if not ext.skinny_regime(M, N, x2.dtype) or nbytes < (1 << 20):
        return [x2]
    copies = min(16, max(1, -(-ROTATE_BYTES // nbytes)))
    return [x2] + [x2.clone() for _ in range(copies - 1)]


SETTLE_MS = 50.0  # untimed calls before a shape's first timing: MI355X clocks rise over ~30-50 ms of load


def settle(x1, x2, config, ms=SETTLE_MS):
    """Run `config` back to back for `ms` of wall time (synchronizing every
    few calls), so the first config timed on a shape does not pay for the
    clocks coming back up after the host prepared its operands."""
    import time
    import torch
    from . import ext
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(4):
            ext.matrix_mul(x1, x2, config)
        torch.cuda.synchronize()


def time_ms(x1, x2, config, best=None, reps=5, x2s=None):
    """Median of `reps` device-timed samples after warmup, with the early
    exit of tilec/tune.py:35-51 when a probe run is over twice the best.

    Device time from HIP events.  A call shorter than GRAPH_BELOW_MS is timed
    as a replay of a captured HIP graph of enough calls to fill about
    GRAPH_FILL_MS (cycling over `x2s` when given), so neither host launch
    overhead nor the replay's start-up pollutes it; the result is the median
    replay time divided by the calls per replay.  Longer calls
    are timed as SUSTAIN_CALLS back-to-back launches per sample, after
    SUSTAIN_WARMUP more, i.e. at the clock the chip holds under load."""
    import torch
    from . import ext
    x2s = x2s or [x2]
    ext.matrix_mul(x1, x2, config)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    ext.matrix_mul(x1, x2, config)
    e.record()
    e.synchronize()
    first = s.elapsed_time(e)
    # The early exit compares like with like: a single launch's time includes
    # launch overhead that a graph-timed best does not, so short calls always
    # get the graph measurement.
    if best is not None and first >= GRAPH_BELOW_MS and first > 2 * best:
        return first
    if first < GRAPH_BELOW_MS:
        # Enough calls per replay to fill about GRAPH_FILL_MS of device time
        # (a multiple of the x2 copies): a replay's start-up costs a few us,
        # which a handful of GEMV-sized calls would each carry about 1 us of.
        n = max(8, len(x2s), min(256, math.ceil(GRAPH_FILL_MS / max(first, 1e-3))))
        calls = math.ceil(n / len(x2s)) * len(x2s)
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream):
            ext.matrix_mul(x1, x2, config)  # split-K buffers of this stream exist before capture
            torch.cuda.synchronize()
            with torch.cuda.graph(graph, stream=stream):
                outs = [ext.matrix_mul(x1, x2s[i % len(x2s)], config) for i in range(calls)]
            graph.replay()
            torch.cuda.synchronize()
            times = []
            for _ in range(reps):
                s.record(stream)
                graph.replay()
                e.record(stream)
                e.synchronize()
                times.append(s.elapsed_time(e) / calls)
        del outs, graph
        return sorted(times)[reps // 2]
    # Longer calls: back-to-back launches, as a loop of products issues them.
    # MI355X holds its boost clock for a short burst but slows under sustained
    # matrix-core load, by an amount that depends on the kernel (its LDS and
    # memory traffic per flop) and the data; timing isolated launches would
    # rank kernels for a regime no training or serving loop runs in.
    for _ in range(SUSTAIN_WARMUP):
        ext.matrix_mul(x1, x2, config)
    times = []
    for _ in range(reps):
        s.record()
        for _ in range(SUSTAIN_CALLS):
            ext.matrix_mul(x1, x2, config)
        e.record()
        e.synchronize()
        times.append(s.elapsed_time(e) / SUSTAIN_CALLS)
    return sorted(times)[reps // 2]


# The BASELINE.json configurations, always part of the tuning set (row-major).
CONFIG_SHAPES = [
    (512, 4096, 64, "f32"),
    (1, 4096, 4096, "f32"), (4, 4096, 4096, "f32"), (16, 4096, 4096, "f32"),
    (1024, 1024, 1024, "f32"), (2048, 2048, 2048, "f32"), (4096, 4096, 4096, "f32"),
    (127, 1000, 513, "f32"), (513, 3001, 127, "f32"), (1000, 4097, 3001, "f32"), (3001, 513, 1000, "f32"),
    (8192, 8192, 8192, "bf16"), (4096, 4096, 4096, "bf16"),
    (1, 4096, 4096, "bf16"), (16, 4096, 4096, "bf16"),
    # large outputs with long K, past the generator's range, so the model does
    # not extrapolate small tiles there
    (4096, 8192, 4096, "f32"), (4096, 16384, 4096, "f32"), (2048, 16384, 2048, "f32"), (8192, 4096, 8192, "f32"),
    (3072, 12288, 3072, "f32"), (8192, 8192, 4096, "bf16"),
]
# The same sizes with transposed operands (x @ W.T GEMV, TN / NT / TT GEMMs).
LAYOUT_CONFIG_SHAPES = [
    (1, 4096, 4096, "f32", 2), (4, 4096, 4096, "f32", 2), (16, 4096, 4096, "f32", 2),
    (1, 4096, 4096, "bf16", 2), (16, 4096, 4096, "bf16", 2),
    (4096, 4096, 4096, "f32", 1), (4096, 4096, 4096, "f32", 2), (4096, 4096, 4096, "f32", 3),
    (8192, 8192, 8192, "bf16", 1), (8192, 8192, 8192, "bf16", 2), (8192, 8192, 8192, "bf16", 3),
]


def _draw(rng):
    """One shape of the reference's log-uniform generator with its size
    limits (tilec/tune.py:54-65; there x1 is [M1,N] and x2 is [N,M2], so its
    N is our K), widened to the regimes MI355X serves differently: skinny M
    in [1, 16] (fp32 and bf16), bf16 tile GEMMs and ragged sizes.  None when
    the draw breaks a size limit."""
    kind = rng.random()
    M = round(2 ** rng.uniform(7, 13))
    K = round(2 ** rng.uniform(8, 14))
    N = round(2 ** rng.uniform(5, 12))
    dtype = "f32"
    if rng.random() < 0.5:
        K = 1 << round(math.log2(K))
    if kind < 0.3:                      # skinny (a third of them bf16)
        M = rng.randint(1, 16)
        N = round(2 ** rng.uniform(8, 14))
        if kind < 0.1:
            dtype = "bf16"
    elif kind < 0.55:                   # bf16 tile GEMM
        dtype = "bf16"
    if M * K * N <= 1 << 33 and M * K <= 1 << 26 and K * N <= 1 << 26:
        return M, K, N, dtype
    return None


# Shapes the tuner never times, so that `bench.py` can measure its picks on
# shapes absent from the table (the model answers them): one or more per
# regime — GEMV, small output, medium, large fp32 and bf16.
UNSEEN_SHAPES = [(5, 3000, 2500, "f32"), (12, 6000, 1000, "bf16"), (48, 2900, 1800, "f32"), (96, 4000, 640, "f32"),
                 (200, 1500, 3000, "f32"), (777, 777, 777, "f32"), (1500, 3100, 900, "f32"),
                 (2000, 3000, 1000, "bf16"), (3000, 2000, 5000, "bf16")]


def _medium_stream(rng, count):
    """Medium outputs with K up to a few thousand: M in [64, 600], K in
    [500, 4000], N in [500, 6000] (either way round), fp32 and bf16 — where
    tile, direct and split choices are closest and the held-out picks of a
    model trained without them erred most."""
    got = set()
    while len(got) < count:
        M = round(2 ** rng.uniform(6, math.log2(600)))
        K = round(2 ** rng.uniform(math.log2(500), 12))
        N = round(2 ** rng.uniform(math.log2(500), math.log2(6000)))
        if rng.random() < 0.5:
            M, N = N, M
        got.add((M, K, N, rng.choice(("f32", "bf16"))))
    return got


def _narrow_stream(rng, count):
    """Few output tiles over a long K: one side of the output in [48, 400],
    the other in [500, 5000], K in [2048, 16384] — split-K territory, bf16
    twice as often as fp32."""
    got = set()
    while len(got) < count:
        a = round(2 ** rng.uniform(math.log2(48), math.log2(400)))
        b = round(2 ** rng.uniform(math.log2(500), math.log2(5000)))
        K = round(2 ** rng.uniform(11, 14))
        M, N = (a, b) if rng.random() < 0.5 else (b, a)
        if M * K <= 1 << 26 and K * N <= 1 << 26:
            got.add((M, K, N, rng.choice(("f32", "bf16", "bf16"))))
    return got


def _bf16_stream(rng, count):
    """bf16 tile GEMMs in every layout: M in [64, 8192], K in [256, 8192],
    N in [64, 8192] log-uniform — the regime with the most variants (two
    MFMA forms, prep and split choices), where held-out picks of models
    trained without this stream erred most."""
    got = set()
    while len(got) < count:
        M = round(2 ** rng.uniform(6, 13))
        K = round(2 ** rng.uniform(8, 13))
        N = round(2 ** rng.uniform(6, 13))
        if rng.random() < 0.5:
            K = 1 << round(math.log2(K))
        if M * K * N <= 1 << 33 and M * K <= 1 << 26 and K * N <= 1 << 26:
            got.add((M, K, N, "bf16", rng.choice((0, 1, 2, 3))))
    return got


def shapes(n=500, seed=0, n_layout=120, n_rows=40, n_tile=30, n_medium=80, n_narrow=60, n_bf16=80):
    """Seeded random shapes (M, K, N, dtype, layout): `n` row-major draws plus
    CONFIG_SHAPES, `n_layout` draws of a second stream (seed + 1) with a
    random non-row-major layout, plus LAYOUT_CONFIG_SHAPES, `n_rows` x @ W.T
    shapes with M <= 4 from a third stream (seed + 2), the row-dot kernel's
    domain, `n_tile` x @ W.T shapes with 5 <= M <= 16 from a fourth
    (seed + 3), the row-tile kernel's, row-major `n_medium` medium
    outputs (seed + 4) and `n_narrow` narrow outputs over a long K
    (seed + 5), and `n_bf16` bf16 tile GEMMs in random layouts (seed + 6).
    None of UNSEEN_SHAPES is ever included."""
    rng = random.Random(seed)
    out = set(CONFIG_SHAPES)
    while len(out) < n + len(CONFIG_SHAPES):
        d = _draw(rng)
        if d is not None:
            out.add(d)
    out = {s + (0,) for s in out}
    rng2 = random.Random(seed + 1)
    lay = set(LAYOUT_CONFIG_SHAPES)
    while len(lay) < n_layout + len(LAYOUT_CONFIG_SHAPES):
        d = _draw(rng2)
        if d is not None:
            lay.add(d + (rng2.choice((1, 2, 2, 3)),))  # x @ W.T (x2 column-major) twice as often
    def wt_stream(rng, count, m_lo, m_hi):
        got = set()
        while len(got) < count:
            M, K, N = rng.randint(m_lo, m_hi), round(2 ** rng.uniform(8, 14)), round(2 ** rng.uniform(8, 14))
            if rng.random() < 0.5:
                K = 1 << round(math.log2(K))
            dtype = rng.choice(("f32", "bf16"))
            if K * N <= 1 << 26:
                got.add((M, K, N, dtype, _lib.X2_COL_MAJOR))
        return got

    rows = wt_stream(random.Random(seed + 2), n_rows, 1, 4)
    tile = wt_stream(random.Random(seed + 3), n_tile, 5, 16)
    more = {t + (0,) for t in _medium_stream(random.Random(seed + 4), n_medium) |
            _narrow_stream(random.Random(seed + 5), n_narrow)}
    more |= _bf16_stream(random.Random(seed + 6), n_bf16)
    unseen = {u + (0,) for u in UNSEEN_SHAPES}
    return sorted((out | lay | rows | tile | more) - unseen, key=lambda s: (s[0] * s[1] * s[2], s))


def operands(M, K, N, dtype, layout, gen):
    """Random N(0,1) operands of a shape, laid out as asked (a column-major
    operand is the transposed view of a row-major buffer)."""
    import torch
    tdt = torch.float32 if dtype == "f32" else torch.bfloat16
    x1 = torch.randn(M, K, generator=gen, device="cuda").to(tdt)
    x2 = torch.randn(K, N, generator=gen, device="cuda").to(tdt)
    if layout & _lib.X1_COL_MAJOR:
        x1 = x1.t().contiguous().t()
    if layout & _lib.X2_COL_MAJOR:
        x2 = x2.t().contiguous().t()
    return x1, x2


def load(path=None):
    """Rows of a timing CSV; files written before the layout column count as
    row-major."""
    with open(path or DATA) as f:
        rows = [{k: (v if k in ("chip", "dtype", "kernel") else float(v)) for k, v in r.items()}
                for r in csv.DictReader(f)]
    for r in rows:
        r["layout"] = int(r.get("layout", 0) or 0)
    return rows


def bench(n=300, seed=0, path=None):
    """Benchmark every config of `n` shapes into `path` (default DATA);
    resumable per (shape, config) — a new variant is timed on the shapes
    already in the file — and flushed per shape.  Inputs are N(0,1) drawn on the GPU from a
    seeded generator (the values do not change the timings' meaning)."""
    import torch
    from . import ext
    path = path or DATA
    chip, cus = machine()
    rows = load(path) if os.path.exists(path) else []
    timed_cfgs = {}  # shape -> {(kernel, split): ms} already in the file
    for r in rows:
        timed_cfgs.setdefault(_key(r), {})[(r["kernel"], int(r["split_k"]))] = r["ms"]
    with open(path, "a", newline="") as f:
        w = csv.writer(f)
        if not rows:
            w.writerow(FIELDS)
        g = torch.Generator(device="cuda").manual_seed(seed)
        todo = shapes(n, seed)
        for i, (M, K, N, dtype, layout) in enumerate(todo):
            have = timed_cfgs.get((M, K, N, dtype, layout), {})
            missing = [c for c in ext.hip_configs(M, K, N, dtype, layout) if c not in have]
            if not missing:
                continue  # resumable: only configs not yet timed (e.g. new variants)
            x1, x2 = operands(M, K, N, dtype, layout, g)
            best = min(have.values()) if have else None
            x2s = operands_for(M, K, N, x2)
            if layout & _lib.X2_COL_MAJOR:  # keep the copies column-major
                x2s = [x2] + [x.t().contiguous().t() for x in x2s[1:]]
            settle(x1, x2, missing[0])
            for kernel, split in missing:
                v = _variant_by_name()[kernel]
                ms = time_ms(x1, x2, (kernel, split), best, x2s=x2s)
                best = ms if best is None else min(best, ms)
                w.writerow([chip, cus, M, K, N, dtype, layout, kernel, v["bm"], v["bn"], v["bk"], split,
                            f"{ms:.6g}"])
            f.flush()
            del x2s
            print(f"{i + 1}/{len(todo)}  {M}x{K} @ {K}x{N} {dtype} layout {layout}  best {best:.4f} ms", flush=True)


REFINE_WITHIN = 1.10  # refine: configs within this factor of a shape's best are re-timed


def refine(path=None, rounds=3, within=REFINE_WITHIN, seed=0, gen=None):
    """Re-time, for every shape in `path` (default DATA), the configs within
    `within` of its best, in `rounds` passes of alternating order, and
    rewrite each one's ms as the median of its first timing and the new
    ones.  One timing carries a few per cent of noise, about the gap between
    the closest configs of a shape, and the measured-best table that
    answers every timed shape would otherwise follow that noise (on MI355X,
    16 x 4096 @ 4096 x 4096 fp32: one sample put skinny_f32_w4_b1 at 15.4 us,
    where repeated timings give 14.6 us)."""
    import statistics
    import torch
    from . import ext
    path = path or DATA
    with open(path) as f:
        raw = list(csv.DictReader(f))
    by_shape = {}
    for i, r in enumerate(raw):
        key = (int(r["M"]), int(r["K"]), int(r["N"]), r["dtype"], int(r.get("layout", 0) or 0))
        by_shape.setdefault(key, []).append(i)
    names = _variant_by_name()
    g = gen if gen is not None else torch.Generator(device="cuda").manual_seed(seed)
    todo = []
    for key, idx in sorted(by_shape.items()):
        best = min(float(raw[i]["ms"]) for i in idx)
        close = [i for i in idx if float(raw[i]["ms"]) <= within * best and raw[i]["kernel"] in names]
        if len(close) >= 2:
            todo.append((key, sorted(close, key=lambda i: float(raw[i]["ms"]))))
    for n, ((M, K, N, dtype, layout), close) in enumerate(todo):
        x1, x2 = operands(M, K, N, dtype, layout, g)
        x2s = operands_for(M, K, N, x2)
        if layout & _lib.X2_COL_MAJOR:  # keep the copies column-major
            x2s = [x2] + [x.t().contiguous().t() for x in x2s[1:]]
        cfg = lambda i: (raw[i]["kernel"], int(float(raw[i]["split_k"])))
        settle(x1, x2, cfg(close[0]))
        samples = {i: [float(raw[i]["ms"])] for i in close}
        for rd in range(rounds):
            for i in (close if rd % 2 == 0 else close[::-1]):
                samples[i].append(time_ms(x1, x2, cfg(i), x2s=x2s))
        for i in close:
            raw[i]["ms"] = f"{statistics.median(samples[i]):.6g}"
        del x2s
        win = min(close, key=lambda i: float(raw[i]["ms"]))
        print(f"{n + 1}/{len(todo)}  {M}x{K} @ {K}x{N} {dtype} layout {layout}: {len(close)} configs, "
              f"best {cfg(win)} {float(raw[win]['ms']):.4f} ms", flush=True)
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=FIELDS, extrasaction="ignore")
        w.writeheader()
        w.writerows(raw)


def row_features(r):
    return features(int(r["M"]), int(r["K"]), int(r["N"]), r["cus"], r["dtype"], r["kernel"], int(r["split_k"]),
                    int(r["layout"]))


def _key(r):
    return (int(r["M"]), int(r["K"]), int(r["N"]), r["dtype"], int(r["layout"]))


def train(test_frac=0.2, seeds=(0, 1, 2), out=MODEL, path=None):
    """Fit on log(ms); report held-out quality against the best config and the
    library's built-in rule over several random 80/20 splits of the shapes
    (one per seed: the worst case of one split moves with the split); refit
    on everything and export JSON (tilec/tune.py:99-132)."""
    from . import ext
    rows = load(path)
    names = _variant_by_name()
    # only the configs hip_configs offers for the row's layout (the row-dot
    # variants only for x @ W.T)
    rows = [r for r in rows if r["kernel"] in names and
            (not ext.rows_variant(names[r["kernel"]]) or
             (r["kernel"], int(r["split_k"])) in ext.hip_configs(*_key(r)[:4], int(r["layout"])))]
    feats = {id(r): row_features(r) for r in rows}

    def data(rs):
        return [feats[id(r)] for r in rs], [math.log(max(r["ms"], 1e-6)) for r in rs]

    by_shape = {}
    for r in rows:
        by_shape.setdefault(_key(r), []).append(r)
    tests = []
    for seed in seeds:
        keys = sorted(by_shape)
        random.Random(seed).shuffle(keys)
        tests.append(set(keys[:int(len(keys) * test_frac)]))
    # one fit per held-out split and one on everything, in parallel processes
    jobs = [data([r for r in rows if _key(r) not in test]) + (seed,) for seed, test in zip(seeds, tests)]
    jobs.append(data(rows) + (seeds[0],))
    import multiprocessing
    with multiprocessing.get_context("fork").Pool(min(len(jobs), os.cpu_count() or 1)) as pool:
        models = pool.map(_fit_gbr, jobs)
    L = _lib.lib()
    gm = lambda v: math.exp(sum(math.log(a) for a in v) / len(v)) if v else float("nan")
    splits = []
    for seed, test, model in zip(seeds, tests, models):
        ratio_model, ratio_default, worst = [], [], None
        for k in sorted(test):
            rs = by_shape[k]
            best = min(r["ms"] for r in rs)
            pred = model.predict([feats[id(r)] for r in rs])
            chosen = rs[min(range(len(rs)), key=lambda i: pred[i])]
            M, K, N, dtype, layout = k
            dcode = _lib.F32 if dtype == "f32" else _lib.BF16
            auto = _lib.variants()[L.tilec_select_variant_layout(M, N, K, dcode, layout, 0, 0)]["name"]
            auto_split = L.tilec_auto_split_k(M, N, K, dcode, _lib.variant_id(auto))
            default = [r for r in rs if r["kernel"] == auto and int(r["split_k"]) == auto_split]
            ratio_model.append(chosen["ms"] / best)
            if worst is None or ratio_model[-1] > worst[0]:
                worst = (ratio_model[-1], list(k), [chosen["kernel"], int(chosen["split_k"])])
            if default:
                ratio_default.append(default[0]["ms"] / best)
        split = {"seed": seed, "held_out_shapes": len(test),
                 "model_geomean_vs_best": gm(ratio_model), "model_worst_vs_best": max(ratio_model),
                 "model_worst_case": worst[1:],
                 "builtin_geomean_vs_best": gm(ratio_default), "builtin_worst_vs_best": max(ratio_default)}
        splits.append(split)
        print(f"split {seed}: {len(test)} held-out shapes; model {split['model_geomean_vs_best']:.3f}x of best "
              f"(geo mean), worst {split['model_worst_vs_best']:.2f}x at {worst[1]} ({worst[2]}); builtin "
              f"{split['builtin_geomean_vs_best']:.3f}x, worst {split['builtin_worst_vs_best']:.2f}x", flush=True)
    report = {
        "splits": splits,
        "held_out_shapes": splits[0]["held_out_shapes"],
        "model_geomean_vs_best": gm([x["model_geomean_vs_best"] for x in splits]),
        "model_worst_vs_best": max(x["model_worst_vs_best"] for x in splits),
        "builtin_geomean_vs_best": gm([x["builtin_geomean_vs_best"] for x in splits]),
        "builtin_worst_vs_best": max(x["builtin_worst_vs_best"] for x in splits),
    }
    print(f"over {len(splits)} splits: model {report['model_geomean_vs_best']:.3f}x (geo mean of geo means), "
          f"worst {report['model_worst_vs_best']:.2f}x; builtin {report['builtin_geomean_vs_best']:.3f}x, "
          f"worst {report['builtin_worst_vs_best']:.2f}x")
    export(models[-1], out, report, best_table(rows))
    return report


def _fit_gbr(job):
    """GBR on (X, y, seed).  The reference's GBR(300, lr 0.05) with trees of
    depth 6 instead of 4: on this data set (three 80/20 shape splits) depth 6
    ran the held-out picks 1.063x of the best config (geomean) against 1.112x
    with depth 4; depth 8 overfits (worst 10x)."""
    from sklearn.ensemble import GradientBoostingRegressor
    X, y, seed = job
    return GradientBoostingRegressor(n_estimators=300, max_depth=6, learning_rate=0.05, random_state=seed).fit(X, y)


def best_table(rows):
    """Measured argmin per benchmarked shape: {"M,K,N,dtype,layout": [kernel, split_k]}."""
    best = {}
    for r in rows:
        k = _key(r)
        if k not in best or r["ms"] < best[k]["ms"]:
            best[k] = r
    return {",".join(map(str, k)): [r["kernel"], int(r["split_k"])] for k, r in sorted(best.items())}


def export(model, path, report=None, table=None):
    """Write a fitted GradientBoostingRegressor as plain JSON trees, plus the
    measured best config of every benchmarked shape (`table`)."""
    trees = []
    for est in model.estimators_[:, 0]:
        t = est.tree_
        trees.append({
            "left": t.children_left.tolist(), "right": t.children_right.tolist(),
            "feature": t.feature.tolist(), "threshold": t.threshold.tolist(),
            "value": t.value[:, 0, 0].tolist(),
        })
    init = float(model.init_.constant_[0][0]) if hasattr(model.init_, "constant_") else float(
        model._raw_predict_init([[0.0] * model.n_features_in_])[0][0])
    data = {"format": "gbr-trees-v1", "learning_rate": model.learning_rate, "init": init,
            "n_features": int(model.n_features_in_), "trees": trees, "report": report or {},
            "best": table or {}}
    with open(path, "w") as f:
        json.dump(data, f)


class TreeModel:
    """Evaluates exported trees: init + learning_rate * sum(tree(x))."""

    def __init__(self, data):
        import numpy as np
        self.lr = data["learning_rate"]
        self.init = data["init"]
        self.n_features = data["n_features"]
        self.trees = [{k: np.asarray(t[k]) for k in ("left", "right", "feature", "threshold", "value")}
                      for t in data["trees"]]
        self.report = data.get("report", {})  # held-out quality at training time
        self.best = {}
        for k, v in data.get("best", {}).items():
            f = k.split(",")
            self.best[(int(f[0]), int(f[1]), int(f[2]), f[3], int(f[4]) if len(f) > 4 else 0)] = tuple(v)

    def predict(self, X):
        import numpy as np
        X = np.asarray(X, dtype=np.float64)
        out = np.full(len(X), self.init)
        rows = np.arange(len(X))
        for t in self.trees:
            node = np.zeros(len(X), dtype=np.int64)
            while True:
                leaf = t["left"][node] < 0
                if leaf.all():
                    break
                f = t["feature"][node]
                go_left = X[rows, np.where(leaf, 0, f)] <= t["threshold"][node]
                nxt = np.where(go_left, t["left"][node], t["right"][node])
                node = np.where(leaf, node, nxt)
            out += self.lr * t["value"][node]
        return out


@lru_cache(None)
def _model(path=MODEL):
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return TreeModel(json.load(f))


@lru_cache(4096)
def pick(M, K, N, dtype="f32", layout=0):
    """(variant name, split_k) with the least predicted time, or None to use
    the library's built-in rule (tilec/tune.py:143-151).  A shape that was
    benchmarked exactly (in this layout) takes its measured best config
    (when still offered)."""
    model = _model()
    if model is None or 0 in (M, K, N):
        return None
    from . import ext
    cands = ext.hip_configs(M, K, N, dtype, layout)
    if not cands:
        return None
    measured = model.best.get((M, K, N, dtype, layout))
    if measured is not None and measured in cands:
        return measured
    cus = _cus()
    if model.n_features < len(features(M, K, N, cus, dtype, cands[0][0], cands[0][1], layout)):
        return None  # a model trained on fewer features than these: use the built-in rule
    pred = model.predict([features(M, K, N, cus, dtype, k, s, layout) for k, s in cands])
    return cands[int(pred.argmin())]


@lru_cache(None)
def _cus():
    try:
        return machine()[1]
    except Exception:
        return 256


if __name__ == "__main__":
    cmd = sys.argv[1]
    if cmd == "bench":
        bench(int(sys.argv[2]) if len(sys.argv) > 2 else 300, path=sys.argv[3] if len(sys.argv) > 3 else None)
    elif cmd == "refine":
        refine(path=sys.argv[2] if len(sys.argv) > 2 else None)
    elif cmd == "train":
        train()
    else:
        raise SystemExit("usage: python -m tilec.tune bench [n] [csv] | refine [csv] | train")
