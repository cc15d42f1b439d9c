"""tilec_matmul_noalloc (the entry point for callers that cannot allocate)
against tilec_matmul with caller-owned scratch, through the C ABI.

Both run the same kernels on the same inputs, so the outputs must agree bit
for bit: on two calls in a row that split K (the second one smaller, so the
static scratch holds the first call's partials when it starts), for the
streaming, panel, direct and tile-GEMM kernels, fp32 and bf16.
"""

import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tilec import _lib

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)


def _dev(a, dtype):
    """fp32 array, or (bf16) the uint16 bit patterns oracle.bf16_round returns."""
    if dtype == torch.bfloat16:
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to("cuda").view(torch.bfloat16)
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def _with_buffers(x1, x2, variant, split):
    """tilec_matmul with freshly allocated workspace and zeroed counters."""
    L = _lib.lib()
    M, K = x1.shape
    N = x2.shape[1]
    code = _lib.F32 if x1.dtype == torch.float32 else _lib.BF16
    out = torch.empty((M, N), dtype=torch.float32, device="cuda")
    ws_n = L.tilec_matmul_workspace_bytes(M, N, K, code, variant, split)
    cnt_n = L.tilec_matmul_counter_bytes(M, N, K, code, variant, split)
    ws = torch.empty(max(ws_n, 1), dtype=torch.uint8, device="cuda")
    cnt = torch.zeros(max(cnt_n, 1), dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    _lib.check(L.tilec_matmul(x1.data_ptr(), x2.data_ptr(), out.data_ptr(), M, N, K, K, N, N, 0, code, variant,
                              split, ws.data_ptr(), ws.numel(), cnt.data_ptr(), cnt.numel(), stream))
    torch.cuda.synchronize()
    return out, ws_n, cnt_n


def _noalloc(x1, x2, variant, split):
    L = _lib.lib()
    M, K = x1.shape
    N = x2.shape[1]
    code = _lib.F32 if x1.dtype == torch.float32 else _lib.BF16
    out = torch.empty((M, N), dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    _lib.check(L.tilec_matmul_noalloc(x1.data_ptr(), x2.data_ptr(), out.data_ptr(), M, N, K, K, N, N, 0, code,
                                      variant, split, stream))
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
