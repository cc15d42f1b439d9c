"""Benchmark of tilec.ext.matrix_mul on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--settle-ms S] [--no-cpu] [--no-extra]
                    [--only SECTION [--case TEXT]]

Prints ONE JSON line.  The headline workload is BASELINE config 2 at its
largest size, fp32 4096^3 (the metric's "TFLOP/s + %MFMA peak at 4096^3"):
a step is one `matrix_mul` call on resident, seeded U(-1,1) inputs; K steps
are timed between HIP events on the stream the kernel runs on, after S ms of
untimed calls (default 200: the GPU's clocks settle under sustained load)
and W warmup steps.  Extra objects in the same line:
  roofline     — the 4096^3 kernel against the fp32 MFMA peak (157.3 TFLOP/s)
  skinny       — the metric's "GB/s + %HBM roofline at M<=16" (config 1):
                 M in {1,4,16} fp32 and {1,16} bf16, K=N=4096, x2 rotated
                 over 512 MiB of copies (beyond the 256 MB Infinity Cache),
                 launches replayed from a HIP graph so the host does not
                 bound an 8 us kernel; with `floor`, one bare pass over the
                 same x2 (tilec_read_floor), the fastest any GEMV can read it
  bf16_8192    — config 4, bf16 8192^3 with fp32 accumulate, vs 2.5 PFLOP/s
  configs      — every fp32 config (0, 2 at 1024/2048/4096, the 4 ragged
                 shapes of 3): device time per call from graph replay
  layouts      — transposed operands read in place: x @ W.T GEMV (weight
                 W [N, K] row-major) as in `skinny`, and the 4096^3 fp32 /
                 8192^3 bf16 GEMMs with x1, x2 or both column-major
  ragged_bf16  — bf16 products whose operand rows are not whole 16-byte
                 groups: the library's pick (a pad variant) beside the plain
                 variant of the same tile and torch.mm, graph-replayed
  reduce       — row and column sums (ext.sum, the reference's tl.sum) in
                 HBM GB/s, graph-replayed over rotating inputs, beside
                 torch.sum of the same inputs timed the same way
  vendor_torch_mm — the square fp32, config-4 bf16 and GEMV cases through
                 torch.mm (hipBLASLt / rocBLAS, fp32 result) on the same
                 box, data and timing protocol, for reference
  tuner_unseen — the tuner's model on shapes absent from its timing table:
                 its pick against the best of every offered config, timed
                 with the tuner's own protocol, beside its held-out report
  host_overhead — eager wall time per ext.matrix_mul call (Python, ctypes,
                 launch) for a 1x1x1 product, a ragged small-output shape and
                 the M=1 GEMV, next to their device time per call
  cpu_baseline — torch.matmul on this box's host cores (every CPU the
                 process may use), the reference's own CPU oracle: the full
                 4096^3 product and the M=1/16 GEMVs, median of >= 5 runs
                 after a warmup; plus (oracle_port) the oracle's tiled C
                 restatement of the reference kernel on a row sample
Only one GPU: --gpus above 1 exits with a message.
"""

import argparse
import json
import math
import os
import platform
import sys
import time

PEAK_FP32_MFMA = 157.3   # TFLOP/s, MI355X dense fp32 matrix
PEAK_BF16_MFMA = 2516.6  # TFLOP/s, MI355X dense bf16 matrix
PEAK_HBM = 8000.0        # GB/s
METRIC = "matrix_mul TFLOP/s + %MFMA peak at 4096³; GB/s + %HBM roofline at M≤16"


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--settle-ms", type=float, default=SETTLE_MS,
                   help="untimed calls before each GEMM timing, in ms of wall time (clock settling)")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--no-extra", action="store_true", help="skip the skinny and bf16 sections")
    p.add_argument("--cpu-seconds", type=float, default=10.0, help="target CPU baseline sample time")
    p.add_argument("--case", default=None,
                   help="with --only skinny, configs or reduce: run only the cases whose key contains this "
                        "text (one kernel per profile run)")
    p.add_argument("--only", choices=["square", "skinny", "bf16", "configs", "layouts", "reduce", "vendor", "copy",
                                      "host", "tuner", "cpu", "ksweep", "floor", "ragged_bf16"],
                   help="run one section and print its own JSON (for profiling); 'copy' is a plain "
                        "device copy of 256 MiB, the calibration run for the FETCH_SIZE/WRITE_SIZE counters")
    return p.parse_args()


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# Untimed load before each GEMM timing.  After the GPU idles (process start,
# data upload, a host pause), MI355X raises its clocks over the first 30-50 ms
# of sustained matrix-core load: an 8192^3 bf16 product goes from 1.18 ms to
# 0.87 ms over its first ~40 calls, a 4096^3 fp32 one from 1.16 to 0.98 ms.
# Timing starts from the steady state a loop of products runs at.
SETTLE_MS = 200.0


def settle(fn, ms=SETTLE_MS, batch=4):
    """Call fn() for `ms` of wall time, synchronizing every `batch` calls so
    the queue never runs far ahead of the clock."""
    import torch
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(batch):
            fn()
        torch.cuda.synchronize()


def timed(fn, steps, warmup, stream=None, settle_ms=0.0):
    """Average ms per call of fn() over `steps` calls, between events recorded
    on the stream the work is issued to, after `settle_ms` of untimed calls
    (clock settling, see SETTLE_MS) and `warmup` more."""
    import torch
    if settle_ms > 0:
        settle(fn, settle_ms)
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    stream = stream or torch.cuda.current_stream()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record(stream)
    for _ in range(steps):
        fn()
    e.record(stream)
    torch.cuda.synchronize()
    return s.elapsed_time(e) / steps


def kernel_name_for(M, K, N, dtype, layout=0):
    from tilec import _lib, tune
    p = tune.pick(M, K, N, dtype, layout)
    if p is not None:
        return p
    L = _lib.lib()
    code = _lib.F32 if dtype == "f32" else _lib.BF16
    v = L.tilec_select_variant_layout(M, N, K, code, layout, 0, 0)
    return _lib.variants()[v]["name"], L.tilec_auto_split_k(M, N, K, code, v)


def bench_square(args):
    import torch
    from oracle import oracle as O  # seeded generators only
    from tilec import ext
    n = 4096
    a = torch.from_numpy(O.uniform((n, n), 4)).cuda()
    b = torch.from_numpy(O.uniform((n, n), 5)).cuda()
    cfg = kernel_name_for(n, n, n, "f32")
    log(f"square fp32 {n}^3 with {cfg}")
    ms = timed(lambda: ext.matrix_mul(a, b), args.steps, args.warmup, settle_ms=args.settle_ms)
    tflops = 2 * n ** 3 / (ms * 1e-3) / 1e12
    return dict(ms=ms, tflops=tflops, config=cfg)


def _gemv(x1, x2s, steps, mm=None, settle_ms=0.0):
    """us per launch of mm(x1, x2s[i]) (default ext.matrix_mul) over rotating
    x2 buffers, launches replayed from a HIP graph (an ~8 us kernel is not
    host-bound), after `settle_ms` of untimed replays."""
    import torch
    from tilec import ext
    mm = mm or ext.matrix_mul
    nbuf = len(x2s)
    for i in range(nbuf):  # warm up: workspace exists before capture
        mm(x1, x2s[i])
    torch.cuda.synchronize()
    reps = 4 * nbuf
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        mm(x1, x2s[0])
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            outs = [mm(x1, x2s[i % nbuf]) for i in range(reps)]
    torch.cuda.synchronize()
    replays = max(1, steps // reps)
    with torch.cuda.stream(s):
        ms = timed(g.replay, replays, 2, stream=s, settle_ms=settle_ms) / reps
    del outs
    return ms * 1e3


CASE = None  # --case filter (profiling runs)


def _gemv_cases(ms_by_dtype, transposed, steps):
    """M x 4096 @ 4096 x 4096 per (dtype, M): x2 row-major, or (transposed)
    the column-major view W.T of a row-major weight W [N, K].  Rotating x2
    copies total >= 512 MB per dtype, so neither L2 nor the 256 MB MALL
    serves a repeat."""
    import torch
    from oracle import oracle as O
    from tilec import ext
    K = N = 4096
    out = {}
    for dtype, Ms in ms_by_dtype:
        tdt = torch.float32 if dtype == "f32" else torch.bfloat16
        esz = 4 if dtype == "f32" else 2
        nbuf = (512 << 20) // (esz * K * N)
        Ms = [M for M in Ms if CASE is None or CASE == (f"M{M}" if dtype == "f32" else f"bf16_M{M}")]
        if not Ms:
            continue
        x2s = [torch.from_numpy(O.normal((K, N), 3 + 1000 * i)).to(tdt).cuda() for i in range(nbuf)]
        if transposed:  # the same values, stored as W [N, K] and passed as W.T
            x2s = [x.t().contiguous().t() for x in x2s]
        for M in Ms:
            x1 = torch.from_numpy(O.normal((M, K), 2)).to(tdt).cuda()
            assert ext.layout_of(x1, x2s[0]) == (2 if transposed else 0)
            cfg = kernel_name_for(M, K, N, dtype, 2 if transposed else 0)
            us = _gemv(x1, x2s, steps, settle_ms=SETTLE_MS / 2)
            nbytes = esz * (M * K + K * N) + 4 * M * N
            gbs = nbytes / (us * 1e-6) / 1e9
            key = (f"M{M}" if dtype == "f32" else f"bf16_M{M}")
            out[key] = dict(us=us, GBps=gbs, frac=gbs / PEAK_HBM, bytes=nbytes, config=list(cfg),
                            traffic=traffic_of(cfg[0], M, N, K, "x2T" if transposed else ""))
            log(f"gemv {dtype} M={M}{' x @ W.T' if transposed else ''}: {us:.2f} us/launch, {gbs:.0f} GB/s ({cfg})")
        del x2s
    return out


def bench_skinny(steps=200):
    """M in {1,4,16} fp32 and {1,16} bf16 at K=N=4096: HBM GB/s from
    graph-replayed launches over rotating x2 copies; beside them the read
    floor of the same x2 (bench_floor)."""
    out = _gemv_cases((("f32", (1, 4, 16)), ("bf16", (1, 16))), False, steps)
    if CASE is None or CASE.startswith("floor"):
        out["floor"] = bench_floor(steps)
    return out


def bench_floor(steps=200):
    """The HBM read floor of the config-1 GEMV: one pass over a 4096 x 4096
    x2 (64 MiB fp32, 32 MiB bf16) through tilec_read_floor — the moving
    window of 16 KiB pieces the GEMV kernels' K splits imitate, two
    workgroups per CU, non-temporal 16-byte loads, no cross-workgroup
    combine — graph-replayed over rotating copies (>= 512 MiB) exactly as the
    GEMV cases are.  A GEMV cannot read x2 faster than this."""
    import ctypes
    import torch
    from tilec import _lib
    L = _lib.lib()
    out = {}
    sink = torch.empty(1 << 18, dtype=torch.float32, device="cuda")
    for dtype, esz in (("f32", 4), ("bf16", 2)):
        nbytes = esz * 4096 * 4096
        nbuf = (512 << 20) // nbytes
        xs = [torch.full((nbytes // 4,), 1.0 + i, dtype=torch.float32, device="cuda") for i in range(nbuf)]

        def read(x, _n=nbytes):
            rc = L.tilec_read_floor(ctypes.c_void_p(x.data_ptr()), _n, ctypes.c_void_p(sink.data_ptr()), 0,
                                    ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
            if rc:
                _lib.check(rc)
            return sink

        us = _gemv(None, xs, steps, mm=lambda _x1, x: read(x), settle_ms=SETTLE_MS / 2)
        gbs = nbytes / (us * 1e-6) / 1e9
        out[f"x2_{dtype}"] = dict(us=us, GBps=gbs, frac=gbs / PEAK_HBM, bytes=nbytes, workgroups=min(
            2 * torch.cuda.get_device_properties(0).multi_processor_count, nbytes // 16384),
            traffic=traffic_of("read_floor", nbytes, 1, 1))
        log(f"read floor {dtype} x2 ({nbytes >> 20} MiB): {us:.2f} us/launch, {gbs:.0f} GB/s")
        del xs
    torch.cuda.synchronize()
    return out


def bench_layouts(steps=200, gemm_steps=20):
    """Transposed operands read in place (no .contiguous() copy): x @ W.T
    GEMV (x2 column-major) as in the skinny section, and the fp32 4096^3 and
    bf16 8192^3 GEMMs with x1, x2 or both column-major."""
    import torch
    from oracle import oracle as O
    from tilec import ext
    out = {"gemv_x_WT": _gemv_cases((("f32", (1, 16)), ("bf16", (1, 16))), True, steps)}
    for dtype, n, peak in (("f32", 4096, PEAK_FP32_MFMA), ("bf16", 8192, PEAK_BF16_MFMA)):
        if CASE is not None and not CASE.startswith(f"{dtype}_{n}"):
            continue
        tdt = torch.float32 if dtype == "f32" else torch.bfloat16
        a = torch.from_numpy(O.uniform((n, n), 4)).to(tdt).cuda()
        b = torch.from_numpy(O.uniform((n, n), 5)).to(tdt).cuda()
        at, bt = a.t().contiguous().t(), b.t().contiguous().t()  # same values, column-major
        for name, x1, x2 in (("x1T", at, b), ("x2T", a, bt), ("x1T_x2T", at, bt)):
            if CASE is not None and CASE not in f"{dtype}_{n}_{name}":
                continue
            cfg = kernel_name_for(n, n, n, dtype, ext.layout_of(x1, x2))
            ms = timed(lambda: ext.matrix_mul(x1, x2), gemm_steps, 3, settle_ms=SETTLE_MS)
            tflops = 2 * n ** 3 / (ms * 1e-3) / 1e12
            out[f"{dtype}_{n}_{name}"] = dict(ms=ms, TFLOPs=tflops, frac=tflops / peak, layout=ext.layout_of(x1, x2),
                                              config=list(cfg))
            log(f"{dtype} {n}^3 {name}: {ms:.3f} ms, {tflops:.1f} TFLOP/s ({cfg})")
        del a, b, at, bt
    return out


def bench_bf16(steps=20, warmup=2, rounds=3):
    """BASELINE config 4 (bf16 8192^3, fp32 accumulate and out), timed in
    `rounds` interleaved rounds of this library and of torch.mm (hipBLASLt,
    fp32 result) on the same inputs, each after its own clock settling; the
    medians are reported, so the spread of one box does not decide the
    comparison (the part is power-bound here and its clock moves with it)."""
    import torch
    from oracle import oracle as O
    from tilec import ext
    n = 8192
    sigma = n ** -0.25
    a = torch.from_numpy(O.normal((n, n), 8, std=sigma)).to(torch.bfloat16).cuda()
    b = torch.from_numpy(O.normal((n, n), 9, std=sigma)).to(torch.bfloat16).cuda()
    cfg = kernel_name_for(n, n, n, "bf16")
    mine, vend = [], []
    for _ in range(rounds):
        mine.append(timed(lambda: ext.matrix_mul(a, b), steps, warmup, settle_ms=SETTLE_MS))
        vend.append(timed(lambda: _vendor_mm(a, b), steps, warmup, settle_ms=SETTLE_MS))
    ms, vms = sorted(mine)[rounds // 2], sorted(vend)[rounds // 2]
    tflops, vtflops = 2 * n ** 3 / (ms * 1e-3) / 1e12, 2 * n ** 3 / (vms * 1e-3) / 1e12
    log(f"bf16 8192^3: {ms:.3f} ms, {tflops:.1f} TFLOP/s ({cfg}); torch.mm {vms:.3f} ms, {vtflops:.1f} TFLOP/s "
        f"(medians of {rounds} interleaved rounds: {[round(x, 3) for x in mine]} / {[round(x, 3) for x in vend]})")
    return dict(ms=ms, TFLOPs=tflops, frac=tflops / PEAK_BF16_MFMA, config=list(cfg), rounds=rounds,
                ms_rounds=mine, torch_mm_ms=vms, torch_mm_TFLOPs=vtflops, torch_mm_ms_rounds=vend,
                speedup_vs_torch_mm=vms / ms)


def _vendor_mm(a, b):
    """torch's library product (hipBLASLt / rocBLAS) with an fp32 result, as
    ext.matrix_mul returns: bf16 inputs use the out_dtype form of torch.mm."""
    import torch
    if a.dtype == torch.bfloat16:
        return torch.mm(a, b, out_dtype=torch.float32)
    return torch.mm(a, b)


def bench_vendor(steps=200):
    """The same cases through torch.mm (ROCm's hipBLASLt / rocBLAS) on the
    same box, data and timing protocol: the square fp32 GEMM, config 4 bf16
    and the GEMVs.  A reference point for what the vendor library reaches
    here, not part of the product."""
    import torch
    from oracle import oracle as O
    out = {}
    n = 4096
    a = torch.from_numpy(O.uniform((n, n), 4)).cuda()
    b = torch.from_numpy(O.uniform((n, n), 5)).cuda()
    ms = timed(lambda: _vendor_mm(a, b), 20, 3, settle_ms=SETTLE_MS)
    out["f32_4096"] = dict(ms=ms, TFLOPs=2 * n ** 3 / (ms * 1e-3) / 1e12)
    del a, b
    n = 8192
    sigma = n ** -0.25
    a = torch.from_numpy(O.normal((n, n), 8, std=sigma)).to(torch.bfloat16).cuda()
    b = torch.from_numpy(O.normal((n, n), 9, std=sigma)).to(torch.bfloat16).cuda()
    ms = timed(lambda: _vendor_mm(a, b), 20, 2, settle_ms=SETTLE_MS)
    out["bf16_8192"] = dict(ms=ms, TFLOPs=2 * n ** 3 / (ms * 1e-3) / 1e12)
    # x2 column-major (both operands k-contiguous), beside the library's
    # layouts section figure for the same layout
    bt = b.t().contiguous().t()
    ms = timed(lambda: _vendor_mm(a, bt), 20, 2, settle_ms=SETTLE_MS)
    out["bf16_8192_x2T"] = dict(ms=ms, TFLOPs=2 * n ** 3 / (ms * 1e-3) / 1e12)
    del a, b, bt
    K = N = 4096
    for dtype, Ms in (("f32", (1, 16)), ("bf16", (1, 16))):
        tdt = torch.float32 if dtype == "f32" else torch.bfloat16
        esz = 4 if dtype == "f32" else 2
        nbuf = (512 << 20) // (esz * K * N)
        x2s = [torch.from_numpy(O.normal((K, N), 3 + 1000 * i)).to(tdt).cuda() for i in range(nbuf)]
        for M in Ms:
            x1 = torch.from_numpy(O.normal((M, K), 2)).to(tdt).cuda()
            us = _gemv(x1, x2s, steps, mm=_vendor_mm)
            nbytes = esz * (M * K + K * N) + 4 * M * N
            gbs = nbytes / (us * 1e-6) / 1e9
            out[f"gemv_{dtype}_M{M}"] = dict(us=us, GBps=gbs, frac=gbs / PEAK_HBM)
        del x2s
    for k, v in out.items():
        log(f"torch.mm {k}: " + ", ".join(f"{f}={x:.3f}" for f, x in v.items()))
    return out


CONFIG_CASES = (
    # (name, M, K, N, generator): BASELINE configs 0, 2 and 3 (fp32)
    ("readme_512x4096x64", 512, 4096, 64, "normal"),
    ("square_1024", 1024, 1024, 1024, "uniform"),
    ("square_2048", 2048, 2048, 2048, "uniform"),
    ("square_4096", 4096, 4096, 4096, "uniform"),
    ("ragged_127x1000x513", 127, 1000, 513, "normal"),
    ("ragged_513x3001x127", 513, 3001, 127, "normal"),
    ("ragged_1000x4097x3001", 1000, 4097, 3001, "normal"),
    ("ragged_3001x513x1000", 3001, 513, 1000, "normal"),
)


def _graph_ms(fn, reps):
    """ms per call of fn() from replays of a HIP graph of `reps` calls, after
    SETTLE_MS / 2 of untimed replays."""
    import torch
    fn()  # workspace exists before capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            outs = [fn() for _ in range(reps)]
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        ms = timed(g.replay, 3, 1, stream=s, settle_ms=SETTLE_MS / 2) / reps
    del outs
    return ms


def bench_configs(reps=20):
    """Every fp32 BASELINE config: device time per call from a HIP graph of
    `reps` calls (so small, latency-bound shapes are not timed as host
    overhead), TFLOP/s and the fraction of the fp32 matrix peak; beside it
    the vendor's torch.mm (hipBLASLt / rocBLAS) on the same inputs, timed the
    same way."""
    import torch
    from oracle import oracle as O
    from tilec import ext
    out = {}
    for i, (name, M, K, N, gen) in enumerate(CONFIG_CASES):
        if CASE is not None and CASE not in name:
            continue
        draw = O.uniform if gen == "uniform" else O.normal
        x1 = torch.from_numpy(draw((M, K), 100 + 2 * i)).cuda()
        x2 = torch.from_numpy(draw((K, N), 101 + 2 * i)).cuda()
        cfg = kernel_name_for(M, K, N, "f32")
        ms = _graph_ms(lambda: ext.matrix_mul(x1, x2), reps)
        tflops = 2 * M * N * K / (ms * 1e-3) / 1e12
        vendor_ms = _graph_ms(lambda: torch.mm(x1, x2), reps) if CASE is None else None
        out[name] = dict(us=ms * 1e3, TFLOPs=tflops, frac=tflops / PEAK_FP32_MFMA, config=list(cfg),
                         traffic=traffic_of(cfg[0], M, N, K),
                         torch_mm_us=vendor_ms and vendor_ms * 1e3,
                         speedup_vs_torch_mm=vendor_ms and vendor_ms / ms)
        log(f"{name}: {ms * 1e3:.1f} us, {tflops:.1f} TFLOP/s ({cfg})"
            + (f"; torch.mm {vendor_ms * 1e3:.1f} us" if vendor_ms else ""))
    return out


RAGGED_BF16_CASES = (
    # (name, M, K, N, layout): bf16 products whose operand rows are not whole
    # 16-byte groups (the pad variants' domain), from the tuner's data, and a
    # square one just short of 8192^3
    ("bf16_1359x4447x1009", 1359, 4447, 1009, 0),
    ("bf16_4354x4096x330_x1T", 4354, 4096, 330, 1),
    ("bf16_560x4565x3046_x1T_x2T", 560, 4565, 3046, 3),
    ("bf16_8191", 8191, 8191, 8191, 0),
)


def bench_ragged_bf16(reps=10):
    """bf16 products with unaligned operand rows: device time per call of the
    library's pick (a pad variant: both operands copied into the workspace
    with 16-byte rows, then the LDS-DMA tile) from a HIP graph of `reps`
    calls, beside the plain variant of the same tile on the operands as they
    are (its register-staged fallback) and torch.mm (hipBLASLt), timed the
    same way."""
    import torch
    from tilec import ext, tune
    out = {}
    g = torch.Generator(device="cuda").manual_seed(0)
    for name, M, K, N, layout in RAGGED_BF16_CASES:
        if CASE is not None and CASE not in name:
            continue
        x1, x2 = tune.operands(M, K, N, "bf16", layout, g)
        cfg = tuple(tune.pick(M, K, N, "bf16", layout) or ("auto", 0))
        n = max(2, min(reps, int(reps * 2e9 / (M * K * N))))
        ms = _graph_ms(lambda: ext.matrix_mul(x1, x2), n)
        rec = dict(us=ms * 1e3, TFLOPs=2 * M * N * K / (ms * 1e-3) / 1e12, layout=layout, config=list(cfg))
        if cfg[0].endswith("_pad"):
            plain = (cfg[0][:-4], cfg[1])
            plain_ms = _graph_ms(lambda: ext.matrix_mul(x1, x2, plain), n)
            rec.update(plain=list(plain), plain_us=plain_ms * 1e3)
        vendor_ms = _graph_ms(lambda: torch.mm(x1, x2).float(), n)
        rec.update(torch_mm_us=vendor_ms * 1e3, speedup_vs_torch_mm=vendor_ms / ms)
        rec["frac"] = rec["TFLOPs"] / PEAK_BF16_MFMA
        out[name] = rec
        log(f"{name}: {ms * 1e3:.1f} us ({cfg})" + (f", plain {rec['plain_us']:.1f} us" if "plain_us" in rec else "")
            + f"; torch.mm {vendor_ms * 1e3:.1f} us")
        del x1, x2
    return out


REDUCE_CASES = (
    # (name, R, C, dtype, axis): the config-1 x2 summed both ways, a few long
    # rows (split columns) and a tall, narrow bf16 matrix (split rows)
    ("rows_4096x4096_f32", 4096, 4096, "f32", 1),
    ("cols_4096x4096_f32", 4096, 4096, "f32", 0),
    ("rows_8x4194304_f32", 8, 1 << 22, "f32", 1),
    ("rows_4096x8192_bf16", 4096, 8192, "bf16", 1),
    ("cols_1048576x64_bf16", 1 << 20, 64, "bf16", 0),
)


def bench_reduce(reps=8):
    """Row and column sums (ext.sum): HBM GB/s from graph-replayed calls over
    rotating inputs (>= 512 MB in total, beyond the Infinity Cache), and the
    vendor's own sum of the same inputs (torch.sum over the same axis, fp32
    accumulate and out) timed the same way."""
    import torch
    from oracle import oracle as O
    from tilec import ext
    out = {}
    for i, (name, R, C, dtype, axis) in enumerate(REDUCE_CASES):
        if CASE is not None and CASE not in name:
            continue
        tdt = torch.float32 if dtype == "f32" else torch.bfloat16
        esz = 4 if dtype == "f32" else 2
        nbuf = max(2, (512 << 20) // (esz * R * C))
        xs = [torch.from_numpy(O.normal((R, C), 2000 + 10 * i + j)).to(tdt).cuda() for j in range(nbuf)]
        calls = 4 * nbuf

        def per_call_ms(fn):
            for x in xs:  # workspace exists before capture
                fn(x)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                fn(xs[0])
                torch.cuda.synchronize()
                with torch.cuda.graph(g, stream=s):
                    outs = [fn(xs[j % nbuf]) for j in range(calls)]
            torch.cuda.synchronize()
            with torch.cuda.stream(s):
                ms = timed(g.replay, reps, 2, stream=s) / calls
            del outs, g
            return ms

        ms = per_call_ms(lambda x: ext.sum(x, axis))
        vms = per_call_ms(lambda x: torch.sum(x, dim=axis, dtype=torch.float32))
        del xs
        nbytes = esz * R * C + 4 * (R if axis == 1 else C)
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[name] = dict(us=ms * 1e3, GBps=gbs, frac=gbs / PEAK_HBM, bytes=nbytes, traffic=traffic_of("sum", R, C, axis),
                         torch_sum_us=vms * 1e3, torch_sum_frac=nbytes / (vms * 1e-3) / 1e9 / PEAK_HBM)
        log(f"sum {name}: {ms * 1e3:.2f} us, {gbs:.0f} GB/s ({100 * gbs / PEAK_HBM:.1f}% of HBM); "
            f"torch.sum {vms * 1e3:.2f} us")
    return out




def bench_tuner():
    """The tuner on shapes it has never timed, where `tune.pick` answers from
    its model rather than its measured-best table: the pick against the best
    of every config `hip_configs` offers, all timed with the tuner's own
    protocol (`tune.time_ms`, x2 rotated as in its table), beside the
    held-out report stored with the model."""
    import torch
    from tilec import tune, ext
    model = tune._model()
    g = torch.Generator(device="cuda").manual_seed(0)
    cases = []
    for M, K, N, dtype in tune.UNSEEN_SHAPES:
        if CASE is not None and CASE not in f"{M}x{K}x{N}_{dtype}":
            continue
        assert (M, K, N, dtype, 0) not in model.best, "an unseen shape is in the tuner's table"
        pick = tuple(tune.pick(M, K, N, dtype, 0))
        x1, x2 = tune.operands(M, K, N, dtype, 0, g)
        x2s = tune.operands_for(M, K, N, x2)
        tune.settle(x1, x2, pick)
        t_pick = tune.time_ms(x1, x2, pick, None, x2s=x2s)
        best_t, best_c = t_pick, pick
        for c in ext.hip_configs(M, K, N, dtype, 0):
            if tuple(c) == pick:
                continue
            t = tune.time_ms(x1, x2, c, best_t, x2s=x2s)
            if t < best_t:
                best_t, best_c = t, tuple(c)
        del x1, x2, x2s
        cases.append(dict(shape=[M, K, N], dtype=dtype, pick=list(pick), pick_us=t_pick * 1e3, best=list(best_c),
                          best_us=best_t * 1e3, ratio=t_pick / best_t))
        log(f"tuner {M}x{K}x{N} {dtype}: pick {pick} {t_pick * 1e3:.1f} us, best {best_c} {best_t * 1e3:.1f} us "
            f"({t_pick / best_t:.2f}x)")
    ratios = [c["ratio"] for c in cases]
    geo = math.exp(sum(math.log(r) for r in ratios) / len(ratios)) if ratios else None
    return dict(unseen_shapes=len(cases), geomean_vs_best=geo, worst_vs_best=max(ratios) if ratios else None,
                cases=cases, held_out_report=getattr(model, "report", None))


def bench_ksweep(ks=(4096, 8192, 16384), rounds=3):
    """fp32 4096 x K x 4096 for growing K, through the kernel the library
    picks at 4096^3 and through torch.mm, medians of `rounds` timings in one process: the change in time
    per added 4096 of K is the K loop's steady state, the rest the fixed cost
    of a launch (prologue, epilogue, imbalance across CUs)."""
    import torch
    from oracle import oracle as O
    from tilec import ext
    n, out = 4096, {}
    cfg = kernel_name_for(n, n, n, "f32")  # one kernel for every K: the 4096^3 pick
    for K in ks:
        a = torch.from_numpy(O.uniform((n, K), 4)).cuda()
        b = torch.from_numpy(O.uniform((K, n), 5)).cuda()
        mine = sorted(timed(lambda: ext.matrix_mul(a, b, cfg), 10, 2, settle_ms=SETTLE_MS) for _ in range(rounds))
        vend = sorted(timed(lambda: _vendor_mm(a, b), 10, 2, settle_ms=SETTLE_MS) for _ in range(rounds))
        flops = 2 * n * n * K
        out[f"K{K}"] = dict(ms=mine[rounds // 2], frac=flops / (mine[rounds // 2] * 1e-3) / 1e12 / PEAK_FP32_MFMA,
                            config=list(cfg), torch_mm_ms=vend[rounds // 2])
        log(f"4096x{K}x4096: {mine[rounds // 2]:.4f} ms ({cfg[0]}), torch.mm {vend[rounds // 2]:.4f} ms")
        del a, b
    k0, k1 = ks[0], ks[-1]
    per = (out[f"K{k1}"]["ms"] - out[f"K{k0}"]["ms"]) / ((k1 - k0) / 4096)
    per_v = (out[f"K{k1}"]["torch_mm_ms"] - out[f"K{k0}"]["torch_mm_ms"]) / ((k1 - k0) / 4096)
    t4096 = 2 * n ** 3 / (PEAK_FP32_MFMA * 1e12) * 1e3
    out["steady_state"] = dict(ms_per_4096_k=per, frac=t4096 / per, fixed_ms=out[f"K{k0}"]["ms"] - per * k0 / 4096,
                               torch_mm_ms_per_4096_k=per_v, torch_mm_frac=t4096 / per_v,
                               torch_mm_fixed_ms=out[f"K{k0}"]["torch_mm_ms"] - per_v * k0 / 4096)
    return out


def bench_copy(nbytes=256 << 20, reps=10):
    """A plain device-to-device copy of known size: what FETCH_SIZE and
    WRITE_SIZE read for it calibrates those counters."""
    import torch
    x = torch.ones(nbytes // 4, device="cuda")
    y = torch.empty_like(x)
    ms = timed(lambda: y.copy_(x), reps, 2)
    return dict(bytes_each_way=nbytes, reps=reps, us=ms * 1e3, GBps=2 * nbytes / (ms * 1e-3) / 1e9)


def traffic_of(kernel, M, N, K, tag=""):
    """HBM bytes per launch measured with rocprofv3 (FETCH_SIZE + WRITE_SIZE,
    scaled by the copy calibration), as recorded in profiles/traffic.json for
    this kernel and shape (key kernel@MxNxK, plus /tag for a layout other
    than row-major); None when it has not been measured.  Sums: kernel
    "sum", M x N = R x C, K = axis."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f).get(f"{kernel}@{M}x{N}x{K}" + (f"/{tag}" if tag else ""))
    except (OSError, ValueError):
        return None
    return None if rec is None else rec.get("bytes")


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor()


def host_threads():
    """CPU threads this process may run on (the box's share of the host)."""
    try:
        return len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        return os.cpu_count() or 1


def _median_runs(fn, min_runs=5, target_s=3.0, max_runs=50):
    """Median wall time of fn() after one untimed warmup run: at least
    `min_runs` runs, more while the total stays under `target_s`."""
    fn()
    runs = []
    while len(runs) < min_runs or (sum(runs) < target_s and len(runs) < max_runs):
        t = time.perf_counter()
        fn()
        runs.append(time.perf_counter() - t)
    return sorted(runs)[len(runs) // 2], runs


def bench_cpu(target_s):
    """CPU baseline: torch.matmul on this box's host cores (the reference's
    own CPU oracle, tests/test_matmul.py:39) on the same seeded inputs, all
    threads this process may use; the full 4096^3 product and the config-1
    GEMVs (M = 1, 16).  Also, as an extra key, the oracle's tiled C
    restatement of `_matmul_tiled` (oracle/matmul_oracle.c, OpenMP) on a row
    sample of the 4096^3 product."""
    import torch
    from oracle import oracle as O
    n = 4096
    threads = host_threads()
    torch.set_num_threads(threads)
    a_np, b_np = O.uniform((n, n), 4), O.uniform((n, n), 5)
    a, b = torch.from_numpy(a_np), torch.from_numpy(b_np)
    dt, runs = _median_runs(lambda: torch.matmul(a, b), target_s=min(target_s, 5.0))
    tflops = 2 * n ** 3 / dt / 1e12
    log(f"cpu torch.matmul 4096^3: {dt * 1e3:.1f} ms (median of {len(runs)}) -> {tflops:.3f} TFLOP/s "
        f"on {threads} threads")
    gemv = {}
    x2 = torch.from_numpy(O.normal((n, n), 3))
    for M in (1, 16):
        x1 = torch.from_numpy(O.normal((M, n), 2))
        t, r = _median_runs(lambda: torch.matmul(x1, x2), min_runs=20, target_s=1.0, max_runs=200)
        nbytes = 4 * (M * n + n * n) + 4 * M * n
        gemv[f"M{M}"] = dict(us=t * 1e6, GBps=nbytes / t / 1e9, runs=len(r))
        log(f"cpu torch.matmul {M}x4096 @ 4096x4096: {t * 1e6:.0f} us, {nbytes / t / 1e9:.1f} GB/s")
    # The oracle port, on a row sample sized to about target_s / 2 of work.
    O.set_num_threads(threads)
    rows = 64
    t0 = time.perf_counter()
    O.matmul_tiled_f32(a_np[:rows], b_np)
    t0 = time.perf_counter() - t0
    rows = int(min(n, max(64, 64 * round(0.5 * target_s / max(t0, 1e-3))))) // 64 * 64
    pdt, pruns = _median_runs(lambda: O.matmul_tiled_f32(a_np[:rows], b_np), target_s=0.5 * target_s, max_runs=25)
    port = dict(value=2 * rows * n * n / pdt / 1e12, unit="TFLOP/s", cores=threads,
                sample=f"rows 0..{rows - 1} of the fp32 4096^3 product, tiled BM=BN=64 BK=16 restatement of "
                       f"_matmul_tiled (oracle/matmul_oracle.c): median of {len(pruns)} runs after 1 warmup")
    log(f"cpu oracle port: {rows} rows in {pdt:.2f} s -> {port['value'] * 1e3:.1f} GFLOP/s on {threads} threads")
    return dict(value=tflops, unit="TFLOP/s", cores=threads, kind="reference",
                sample=f"the full fp32 4096^3 product (same seeded U(-1,1) inputs) through torch.matmul on the "
                       f"CPU, torch.set_num_threads({threads}) = every CPU this process may run on: median of "
                       f"{len(runs)} runs after 1 warmup, {dt * 1e3:.1f} ms per run",
                cpu=cpu_model(), gemv_torch_matmul=gemv, oracle_port=port)


HOST_CASES = (
    # (name, M, K, N): the smallest product, a ragged small-output shape and
    # the config-1 GEMV, fp32 row-major
    ("1x1x1", 1, 1, 1),
    ("127x1000x513", 127, 1000, 513),
    ("gemv_1x4096x4096", 1, 4096, 4096),
)


def bench_host(calls=2000):
    """Per-call cost of the eager path, ext.matrix_mul as a caller runs it:
    `calls` back-to-back calls from Python then one synchronize, in wall
    time per call, against the device time per call of the same product
    replayed from a HIP graph (what the GPU needs).  Also the host time of
    the Python side alone (shape checks, operand analysis, config lookup and
    output allocation, no launch)."""
    import torch
    from oracle import oracle as O
    from tilec import ext
    out = {}
    for i, (name, M, K, N) in enumerate(HOST_CASES):
        x1 = torch.from_numpy(O.normal((M, K), 300 + i)).cuda()
        x2 = torch.from_numpy(O.normal((K, N), 400 + i)).cuda()
        for _ in range(50):
            ext.matrix_mul(x1, x2)
        torch.cuda.synchronize()
        t = time.perf_counter()
        for _ in range(calls):
            ext.matrix_mul(x1, x2)
        torch.cuda.synchronize()
        eager_us = (time.perf_counter() - t) / calls * 1e6
        # Python side only: everything matrix_mul does before the library call.
        t = time.perf_counter()
        for _ in range(calls):
            M_, K_, N_ = ext._prepare(x1, x2)
            ops = (ext._operand(x1, M_, K_), ext._operand(x2, K_, N_))
            ext._resolve_config(None, M_, K_, N_, x1.dtype, 0)
            torch.empty((M_, N_), dtype=torch.float32, device=x1.device)
            torch.cuda.current_stream(x1.device).cuda_stream
        py_us = (time.perf_counter() - t) / calls * 1e6
        reps = 20
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            ext.matrix_mul(x1, x2)
            torch.cuda.synchronize()
            with torch.cuda.graph(g, stream=s):
                outs = [ext.matrix_mul(x1, x2) for _ in range(reps)]
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            dev_us = timed(g.replay, 20, 2, stream=s) / reps * 1e3
        del outs
        out[name] = dict(eager_us_per_call=eager_us, python_us_per_call=py_us, device_us_per_call=dev_us,
                         calls=calls, config=list(kernel_name_for(M, K, N, "f32")))
        log(f"host {name}: eager {eager_us:.2f} us/call (python side {py_us:.2f}), device {dev_us:.2f} us/call")
    return out


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "bench.py runs on one GPU only: this build has no multi-GPU path "
                                   "(see the sharding design notes); run with --gpus 1"}), flush=True)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no ROCm GPU visible"}), flush=True)
        sys.exit(1)
    from tilec import _lib
    _lib.lib()  # fail loudly if the HIP library is missing
    props = torch.cuda.get_device_properties(0)

    global CASE
    CASE = args.case
    if args.only:
        out = {"square": lambda: bench_square(args), "skinny": bench_skinny, "bf16": bench_bf16,
               "configs": bench_configs, "layouts": bench_layouts, "reduce": bench_reduce,
               "vendor": bench_vendor, "copy": bench_copy, "host": bench_host, "tuner": bench_tuner,
               "ksweep": bench_ksweep, "floor": bench_floor, "ragged_bf16": bench_ragged_bf16,
               "cpu": lambda: bench_cpu(args.cpu_seconds)}[args.only]()
        print(json.dumps({"section": args.only, **out}), flush=True)
        return

    sq = bench_square(args)
    extra = {}
    if not args.no_extra:
        extra["skinny"] = bench_skinny()
        extra["bf16_8192"] = bench_bf16()
        extra["configs"] = bench_configs()
        extra["layouts"] = bench_layouts()
        extra["ragged_bf16"] = bench_ragged_bf16()
        extra["reduce"] = bench_reduce()
        extra["host_overhead"] = bench_host()
        extra["tuner_unseen"] = bench_tuner()
        extra["vendor_torch_mm"] = bench_vendor()
    cpu = None if args.no_cpu else bench_cpu(args.cpu_seconds)

    rec = {
        "metric": METRIC,
        "value": round(sq["tflops"], 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_ms": args.settle_ms,
        "ms_per_step": round(sq["ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded U(-1,1), generated on the CPU, resident in HBM)",
        "config": {"workload": "BASELINE config 2 at 4096^3: fp32 square GEMM, M=N=K=4096, row-major",
                   "M": 4096, "N": 4096, "K": 4096, "kernel": list(sq["config"])},
        "roofline": {"bound": "mfma", "achieved": round(sq["tflops"], 3), "peak": PEAK_FP32_MFMA,
                     "unit": "TFLOP/s", "frac": round(sq["tflops"] / PEAK_FP32_MFMA, 4),
                     "traffic": traffic_of(sq["config"][0], 4096, 4096, 4096)},
        "cpu_baseline": cpu,
        "device": {"name": props.name, "cus": props.multi_processor_count,
                   "arch": getattr(props, "gcnArchName", "")},
    }
    rec.update(extra)
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
