"""tilec_matmul_noalloc (the entry point for callers that cannot allocate)
against tilec_matmul with caller-owned scratch, through the C ABI.

Both run the same kernels on the same inputs, so the outputs must agree bit
for bit: on two calls in a row that split K (the second one smaller, so the
static scratch holds the first call's partials when it starts), for the
streaming, panel, direct and tile-GEMM kernels, fp32 and bf16.
"""

import ctypes
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402
from tilec import _lib  # noqa: E402

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)


def _dev(a, dtype):
    """fp32 array, or (bf16) the uint16 bit patterns oracle.bf16_round returns."""
    if dtype == torch.bfloat16:
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to("cuda").view(torch.bfloat16)
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def _operands(x1, x2):
    """(M, K, N, dtype code, layout, ldx1, ldx2) of a row-major x1 and an x2
    that is row-major or the transposed view W.t() of a row-major W."""
    M, K = x1.shape
    N = x2.shape[1]
    code = _lib.F32 if x1.dtype == torch.float32 else _lib.BF16
    if x2.stride(0) == 1 and N > 1:
        return M, K, N, code, _lib.X2_COL_MAJOR, K, x2.stride(1)
    return M, K, N, code, 0, K, x2.stride(0)


def _with_buffers(x1, x2, variant, split):
    """tilec_matmul with freshly allocated workspace and zeroed counters."""
    L = _lib.lib()
    M, K, N, code, layout, ld1, ld2 = _operands(x1, x2)
    out = torch.empty((M, N), dtype=torch.float32, device="cuda")
    ws_n, cnt_n = ctypes.c_size_t(0), ctypes.c_size_t(0)
    _lib.check(L.tilec_matmul_scratch_bytes(M, N, K, ld1, ld2, layout, code, variant, split,
                                            ctypes.byref(ws_n), ctypes.byref(cnt_n)))
    ws_n, cnt_n = ws_n.value, cnt_n.value
    ws = torch.empty(max(ws_n, 1), dtype=torch.uint8, device="cuda")
    cnt = torch.zeros(max(cnt_n, 1), dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    _lib.check(L.tilec_matmul(x1.data_ptr(), x2.data_ptr(), out.data_ptr(), M, N, K, ld1, ld2, N, layout, code,
                              variant, split, ws.data_ptr(), ws.numel(), cnt.data_ptr(), cnt.numel(), stream))
    torch.cuda.synchronize()
    return out, ws_n, cnt_n


def _noalloc_into(out, x1, x2, variant, split):
    """Enqueue tilec_matmul_noalloc on the current stream (no synchronize)."""
    M, K, N, code, layout, ld1, ld2 = _operands(x1, x2)
    stream = torch.cuda.current_stream().cuda_stream
    _lib.check(_lib.lib().tilec_matmul_noalloc(x1.data_ptr(), x2.data_ptr(), out.data_ptr(), M, N, K, ld1, ld2,
                                               N, layout, code, variant, split, stream))


def _noalloc(x1, x2, variant, split):
    out = torch.empty((x1.shape[0], x2.shape[1]), dtype=torch.float32, device="cuda")
    _noalloc_into(out, x1, x2, variant, split)
    torch.cuda.synchronize()
    return out


# (name or AUTO, dtype, large shape, smaller shape, split): every case splits K
CASES = [
    (None, torch.float32, (16, 4096, 4096), (3, 1000, 300), 0),        # streaming kernel, auto split
    ("skinny_f32_p_v1_w8", torch.float32, (1, 4096, 4096), (1, 1500, 520), 0),  # panel kernel
    ("skinny_f32_w4_b2", torch.float32, (7, 8192, 1000), (2, 3000, 130), 16),   # streaming, 16 splits
    ("gemm_f32_64x64x16_w2x2", torch.float32, (100, 4096, 200), (65, 2000, 70), 8),  # tile GEMM split K
    ("direct_f32_32x64_w4_db", torch.float32, (513, 3001, 127), (127, 1000, 513), 7),  # direct kernel, 7 splits
    ("skinny_bf16_p_v1_w8", torch.bfloat16, (1, 4096, 4096), (1, 2048, 264), 0),
    (None, torch.bfloat16, (16, 4096, 4096), (5, 999, 136), 0),
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_noalloc_matches_caller_buffers(case):
    name, dt, big, small, split = CASES[case]
    variant = _lib.VARIANT_AUTO if name is None else _lib.variant_id(name)
    for i, (m, k, n) in enumerate((big, small)):
        a, b = O.normal((m, k), 70 + 10 * case + 2 * i), O.normal((k, n), 71 + 10 * case + 2 * i)
        if dt == torch.bfloat16:
            a, b = O.bf16_round(a), O.bf16_round(b)
        x1, x2 = _dev(a, dt), _dev(b, dt)
        say(f"noalloc case {case} ({name}, {dt}) call {i}: {(m, k, n)} split {split}")
        want, ws_n, cnt_n = _with_buffers(x1, x2, variant, split)
        assert ws_n > 0 and cnt_n > 0, "the case must use scratch"
        got = _noalloc(x1, x2, variant, split)
        assert torch.equal(got, want), (case, i)
        ref = O.matmul_bf16_f64(a, b) if dt == torch.bfloat16 else O.matmul_f64(a, b)
        assert O.rel_l2(got.cpu().numpy(), ref) <= (1e-5 if dt == torch.bfloat16 else O.TOL_F32)


# x @ W.T through the allocation-free entry point: W [N, K] row-major, read in
# place as a column-major x2 (layout bit TILEC_X2_COL_MAJOR).
WT_CASES = [
    (None, (4, 4096, 1000), 0),                    # built-in rule: the streaming kernel, auto split
    ("skinny_f32_w8_b1", (16, 3000, 520), 6),      # streaming kernel, column-major block, 6 splits
    ("direct_f32_32x64_w4", (40, 2000, 300), 5),   # direct kernel, column-major x2, 5 splits
]


@pytest.mark.parametrize("case", range(len(WT_CASES)))
def test_noalloc_x_at_w_t(case):
    name, (m, k, n), split = WT_CASES[case]
    variant = _lib.VARIANT_AUTO if name is None else _lib.variant_id(name)
    for i, (mm, kk, nn) in enumerate(((m, k, n), (max(m // 2, 1), k - 512, n // 2))):
        a, w = O.normal((mm, kk), 300 + 10 * case + 2 * i), O.normal((nn, kk), 301 + 10 * case + 2 * i)
        x1, wd = _dev(a, torch.float32), _dev(w, torch.float32)
        say(f"noalloc x @ W.T case {case} ({name}) call {i}: {(mm, kk, nn)} split {split}")
        want, ws_n, _ = _with_buffers(x1, wd.t(), variant, split)
        assert ws_n > 0, "the case must use scratch"
        got = _noalloc(x1, wd.t(), variant, split)
        assert torch.equal(got, want), (case, i)
        assert O.rel_l2(got.cpu().numpy(), O.matmul_f64(a, np.ascontiguousarray(w.T))) <= O.TOL_F32


# Captured in a graph: split-K calls of the streaming, panel and direct
# kernels and an x @ W.T call, in a fresh process so that the first captured
# call is the process's first tilec_matmul_noalloc call (it looks up the
# static array and clears its counters with a kernel, inside the capture).
GRAPH_CASES = [
    ("skinny_f32_p_v1_w8", (1, 4096, 4096), 0, False),
    ("skinny_f32_w8_b1", (16, 4096, 2048), 8, False),
    ("direct_f32_32x64_w4_db", (127, 1000, 513), 8, False),
    ("skinny_f32_w8_b1", (8, 2048, 700), 4, True),
]


def _graph_child():
    torch.cuda.init()
    tensors = []
    for j, (name, (m, k, n), split, wt) in enumerate(GRAPH_CASES):
        x1 = torch.empty((m, k), dtype=torch.float32, device="cuda")
        x2 = torch.empty((n, k) if wt else (k, n), dtype=torch.float32, device="cuda")
        out = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
        tensors.append((x1, x2, out))
    # caller-buffer results first, outside the capture (loads the library's code object)
    x1, x2, _ = tensors[0]
    x1.copy_(torch.from_numpy(O.normal(tuple(x1.shape), 400)))
    x2.copy_(torch.from_numpy(O.normal(tuple(x2.shape), 401)))
    _with_buffers(x1, x2, _lib.variant_id(GRAPH_CASES[0][0]), GRAPH_CASES[0][2])
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for (name, _, split, wt), (x1, x2, out) in zip(GRAPH_CASES, tensors):
                _noalloc_into(out, x1, x2.t() if wt else x2, _lib.variant_id(name), split)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    print("captured", flush=True)
    for rep in range(3):
        wants = []
        for j, ((name, _, split, wt), (x1, x2, out)) in enumerate(zip(GRAPH_CASES, tensors)):
            a = O.normal(tuple(x1.shape), 500 + 20 * rep + 2 * j)
            b = O.normal(tuple(x2.shape), 501 + 20 * rep + 2 * j)
            x1.copy_(torch.from_numpy(a))
            x2.copy_(torch.from_numpy(b))
            want, ws_n, cnt_n = _with_buffers(x1, x2.t() if wt else x2, _lib.variant_id(name), split)
            assert ws_n > 0 and cnt_n > 0, (name, "must use scratch")
            ref = O.matmul_f64(a, np.ascontiguousarray(b.T) if wt else b)
            assert O.rel_l2(want.cpu().numpy(), ref) <= O.TOL_F32, (name, rep)
            wants.append(want)
            out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for j, (want, (_, _, out)) in enumerate(zip(wants, tensors)):
            assert torch.equal(out, want), (GRAPH_CASES[j][0], rep)
        print(f"replay {rep} matches", flush=True)
    print("CHILD OK", flush=True)


def test_noalloc_under_graph_capture_first_call():
    say("noalloc graph capture: child process")
    env = dict(os.environ)
    env["PYTHONPATH"] = ROOT + os.pathsep + env.get("PYTHONPATH", "")
    r = subprocess.run([sys.executable, "-u", os.path.abspath(__file__), "graph-child"], cwd=ROOT, env=env,
                       capture_output=True, text=True, timeout=300)
    say(r.stdout[-2000:])
    assert r.returncode == 0 and "CHILD OK" in r.stdout, r.stdout[-2000:] + r.stderr[-4000:]


if __name__ == "__main__" and sys.argv[1:] == ["graph-child"]:
    _graph_child()
