"""CPU oracle for tilec's matmul path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, and only as the checker (or the timed CPU baseline).  The product
(tilec) never imports it.

Contents
  * numpy wrappers of liboracle.so (matmul_oracle.c): the literal tiled
    restatement of `_matmul_tiled` (tilec/ext.py:13-24) in fp32, and fp64
    references, for fp32 and bf16 inputs;
  * bf16 rounding (round-to-nearest-even);
  * pure-Python restatements of the host integer helpers `cdiv`
    (tilec/language.py:16-18), `plan`, `_blocks`, `mm_configs`
    (tilec/ext.py:10,29-51) and the tuner's shape generator
    (tilec/tune.py:54-65);
  * the seeded input generators and error metrics every parity check uses;
  * numpy restatements of the reduction `tl.sum` (row and column sums).

Pinning (tests/test_oracle.py): see the header of matmul_oracle.c.  The
integer helpers are pinned by the reference's one known answer
(cdiv(5000, 4096) == 2, tilec/language.py:17), by hand-derived values
(plan(300) == (1024, 1), plan(5000) == (4096, 2), ...) and by brute-force
characterisations (smallest power of 4, the two filter rules of mm_configs).
The sums are pinned by the known answer of the reference's own example
(kernel1.py:18-27: the row sums of arange(32).reshape(4, 8), which it checks
against numpy's x.sum(axis=1)), by brute-force loops on small inputs and by
the invariant that row and column sums share one total.
"""

import ctypes
import math
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_fp = ctypes.POINTER(ctypes.c_float)
_dp = ctypes.POINTER(ctypes.c_double)
_up = ctypes.POINTER(ctypes.c_uint16)
_i64 = ctypes.c_int64


def build():
    """Compile liboracle.so with its Makefile (gcc)."""
    subprocess.run(["make", "-s", "-B", "-C", HERE, "liboracle.so"], check=True)
    _lib_cache.clear()


_lib_cache = {}


def lib():
    if "L" not in _lib_cache:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        L.oracle_matmul_tiled_f32.argtypes = [_fp, _fp, _fp] + [_i64] * 9
        L.oracle_matmul_tiled_bf16.argtypes = [_up, _up, _fp] + [_i64] * 9
        L.oracle_matmul_f64.argtypes = [_fp, _fp, _dp] + [_i64] * 6
        L.oracle_matmul_bf16_f64.argtypes = [_up, _up, _dp] + [_i64] * 6
        L.oracle_bf16_from_f32.argtypes = [_fp, _up, _i64]
        L.oracle_num_threads.restype = ctypes.c_int
        L.oracle_set_num_threads.argtypes = [ctypes.c_int]
        for f in ("oracle_matmul_tiled_f32", "oracle_matmul_tiled_bf16", "oracle_matmul_f64",
                  "oracle_matmul_bf16_f64", "oracle_bf16_from_f32", "oracle_set_num_threads"):
            getattr(L, f).restype = None
        _lib_cache["L"] = L
    return _lib_cache["L"]


def _ptr(a, t):
    return a.ctypes.data_as(t)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def _shapes(a, b):
    M, K = a.shape
    K2, N = b.shape
    if K != K2:
        raise ValueError(f"shapes {a.shape} and {b.shape} don't match")
    return M, K, N


# ---------------------------------------------------------------------------
# Matmul restatements
# ---------------------------------------------------------------------------

def matmul_tiled_f32(a, b, BM=64, BN=64, BK=16):
    """`_matmul_tiled` restated (fp32 accumulate, K steps of BK)."""
    a, b = _c(a, np.float32), _c(b, np.float32)
    M, K, N = _shapes(a, b)
    c = np.zeros((M, N), np.float32)
    if M and N:
        lib().oracle_matmul_tiled_f32(_ptr(a, _fp), _ptr(b, _fp), _ptr(c, _fp), M, N, K,
                                      max(K, 1), max(N, 1), max(N, 1), BM, BN, BK)
    return c


def matmul_f64(a, b):
    """fp64-accumulated product of fp32 inputs."""
    a, b = _c(a, np.float32), _c(b, np.float32)
    M, K, N = _shapes(a, b)
    c = np.zeros((M, N), np.float64)
    if M and N:
        lib().oracle_matmul_f64(_ptr(a, _fp), _ptr(b, _fp), _ptr(c, _dp), M, N, K,
                                max(K, 1), max(N, 1), max(N, 1))
    return c


def matmul_tiled_bf16(a16, b16, BM=64, BN=64, BK=16):
    """Tiled restatement on bf16 bit patterns (uint16 arrays), fp32 accumulate."""
    a16, b16 = _c(a16, np.uint16), _c(b16, np.uint16)
    M, K, N = _shapes(a16, b16)
    c = np.zeros((M, N), np.float32)
    if M and N:
        lib().oracle_matmul_tiled_bf16(_ptr(a16, _up), _ptr(b16, _up), _ptr(c, _fp), M, N, K,
                                       max(K, 1), max(N, 1), max(N, 1), BM, BN, BK)
    return c


def matmul_bf16_f64(a16, b16):
    """fp64-accumulated product of bf16 inputs (uint16 bit patterns)."""
    a16, b16 = _c(a16, np.uint16), _c(b16, np.uint16)
    M, K, N = _shapes(a16, b16)
    c = np.zeros((M, N), np.float64)
    if M and N:
        lib().oracle_matmul_bf16_f64(_ptr(a16, _up), _ptr(b16, _up), _ptr(c, _dp), M, N, K,
                                     max(K, 1), max(N, 1), max(N, 1))
    return c


def bf16_round(x):
    """fp32 array -> bf16 bit patterns (uint16), round to nearest even."""
    x = _c(x, np.float32)
    y = np.empty(x.shape, np.uint16)
    if x.size:
        lib().oracle_bf16_from_f32(_ptr(x, _fp), _ptr(y, _up), x.size)
    return y


def bf16_to_f32(h):
    """bf16 bit patterns -> exact fp32 values."""
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


def num_threads():
    return lib().oracle_num_threads()


def set_num_threads(n):
    lib().oracle_set_num_threads(int(n))


# ---------------------------------------------------------------------------
# Metrics
# ---------------------------------------------------------------------------

def rel_l2(got, ref):
    """||got - ref||_2 / ||ref||_2 in float64 (0 when both are zero)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    num = np.linalg.norm((got - ref).ravel())
    den = np.linalg.norm(ref.ravel())
    if den == 0.0:
        return 0.0 if num == 0.0 else math.inf
    return float(num / den)


# Tolerances stated by the north star: rel-L2 against the fp32/fp64 reference.
TOL_F32 = 1e-5
TOL_BF16 = 1e-2


# ---------------------------------------------------------------------------
# Seeded inputs (generated on the CPU so GPU and CPU see identical values).
# Seeds follow the plan: 2*i for x1 and 2*i+1 for x2, i = config index.
# ---------------------------------------------------------------------------

def normal(shape, seed, std=1.0):
    rng = np.random.Generator(np.random.PCG64(seed))
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float32)


def uniform(shape, seed, lo=-1.0, hi=1.0):
    rng = np.random.Generator(np.random.PCG64(seed))
    return rng.uniform(lo, hi, size=shape).astype(np.float32)


def small_ints(shape, seed, lo=-8, hi=8):
    rng = np.random.Generator(np.random.PCG64(seed))
    return rng.integers(lo, hi + 1, size=shape).astype(np.float32)


# ---------------------------------------------------------------------------
# Host integer helpers (pure Python)
# ---------------------------------------------------------------------------

MAX_BLOCK = 4096
SPLITS = (1, 2, 4, 8, 16, 32, 64)
JOINS = (1, 2, 4, 8)
BLOCKS = (256, 1024, 4096)


def cdiv(a, b):
    """tilec/language.py:16-18."""
    return (a + b - 1) // b


def plan(N, block=None):
    """tilec/ext.py:29-34."""
    if block is None:
        block = 1
        while block < N and block < MAX_BLOCK:
            block *= 4
    return block, cdiv(N, block)


def blocks(n):
    """tilec/ext.py:43-45."""
    top = plan(n)[0]
    return [b for b in BLOCKS if b < top and cdiv(n, b) <= 16] + [top]


def mm_configs(M1, N, M2):
    """tilec/ext.py:48-51."""
    return [(p, r, b) for p in SPLITS for r in JOINS
            if (p == 1 or N // p >= 32) and (r == 1 or M1 >= r)
            for b in blocks(cdiv(N, p))]


# ---------------------------------------------------------------------------
# Reductions.  The reference plans `tl.sum` (README.md:88) and shows it as
# the `row_sum` kernel (kernel1.py:8-15): out[r] = tl.sum(x[r, :]) over a
# row-major [R, C] fp32 matrix.  Restated in float64 (the parity reference)
# and as the literal fp32 left-to-right sum of one thread (the CPU baseline).
# ---------------------------------------------------------------------------

def sum_f64(x, axis=1):
    """Row (axis=1) or column (axis=0) sums of a 2-D array, in float64."""
    x = np.asarray(x)
    assert x.ndim == 2 and axis in (0, 1)
    return x.astype(np.float64).sum(axis=axis)


def sum_abs_f64(x, axis=1):
    """sum |x| along the same axis: the scale of a sum's rounding error."""
    return np.abs(np.asarray(x).astype(np.float64)).sum(axis=axis)


def row_sum_f32_seq(x):
    """kernel1.py:14 as one thread runs it: for each row, acc = 0.0f, then
    acc += x[r][c] for c = 0 .. C-1 in fp32 (vectorised over rows)."""
    x = np.asarray(x, dtype=np.float32)
    acc = np.zeros(x.shape[0], dtype=np.float32)
    for c in range(x.shape[1]):
        acc += x[:, c]
    return acc


def sum_error_ok(got, x, axis=1, rel=2e-6):
    """Per output: |got - sum| <= rel * sum |x| (fp32 accumulation in any
    order; rel covers chains of a few hundred fp32 additions)."""
    ref = sum_f64(x, axis)
    bound = rel * sum_abs_f64(x, axis) + 1e-30
    return bool(np.all(np.abs(np.asarray(got, np.float64) - ref) <= bound))
