"""tilec ops on PyTorch-ROCm tensors: `matrix_mul(x1, x2)` and `sum(x, axis)`.

Host code mirroring the reference's op module (tilec/ext.py): the same public
call, the same shape error, the same `.contiguous()` semantics and a freshly
allocated output, launching hand-written gfx950 kernels through the C ABI in
libtilec_hip.so instead of a JIT-compiled Metal tile kernel.

    import torch, tilec
    x1 = torch.randn(512, 4096, device="cuda")
    x2 = torch.randn(4096, 64, device="cuda")
    out = tilec.ext.matrix_mul(x1, x2)
    rows = tilec.ext.sum(x1, axis=1)       # [512] fp32 row sums

Kernel choice per shape comes from `tune.pick` (the shape→config model trained
on MI355X), falling back to the library's built-in rule when no model is
present.  The legacy config-space helpers of the reference (`plan`,
`mm_configs`, ...) are kept with their original meaning.
"""

import ctypes
import re
from functools import lru_cache

import torch

from . import _lib
from .language import cdiv

__all__ = [
    "matrix_mul", "_matrix_mul_tiled", "sum", "cdiv", "plan", "mm_configs", "_blocks",
    "MAX_BLOCK", "SPLITS", "JOINS", "BLOCKS", "hip_configs", "workspace_for", "counters_for",
]

# ---------------------------------------------------------------------------
# Legacy config space of the reference's split/join/block kernel
# (tilec/ext.py:10,29-51).  Pure integer helpers, restated with the same
# meaning; the MI355X config space is `hip_configs` below.
# ---------------------------------------------------------------------------

MAX_BLOCK = 4096


def plan(N, block=None):
    """(block, chunks): the smallest power of 4 >= N capped at MAX_BLOCK, and
    cdiv(N, block).  Restates tilec/ext.py:29-34."""
    if block is None:
        block = 1
        while block < N and block < MAX_BLOCK:
            block *= 4
    return block, cdiv(N, block)


SPLITS = (1, 2, 4, 8, 16, 32, 64)
JOINS = (1, 2, 4, 8)
BLOCKS = (256, 1024, 4096)


def _blocks(n):
    """Restates tilec/ext.py:43-45."""
    top = plan(n)[0]
    return [b for b in BLOCKS if b < top and cdiv(n, b) <= 16] + [top]


def mm_configs(M1, N, M2):
    """(split, join, block) triples of the legacy kernel; N is the reduction
    dimension.  Restates tilec/ext.py:48-51."""
    return [(p, r, b) for p in SPLITS for r in JOINS
            if (p == 1 or N // p >= 32) and (r == 1 or M1 >= r)
            for b in _blocks(cdiv(N, p))]


# ---------------------------------------------------------------------------
# MI355X config space: (variant name, split_k) pairs valid for a shape.
# ---------------------------------------------------------------------------

_SKINNY_SPLITS = (1, 2, 4, 8, 16, 32, 64)


def hip_configs(M, K, N, dtype="f32", layout=None):
    """Every (variant, split_k) the library can run for out[M,N] = x1[M,K]·x2[K,N].

    The row-dot and row-tile variants are offered only where their kernel
    runs: with `layout` given, x @ W.T (x2 column-major, x1 row-major), and
    for the row-tile kernel K a multiple of the 16-byte element count (the
    row-dot kernel takes any K).  Elsewhere they run the streaming kernel
    unsplit, which is never the config to pick.

    The skinny family (a K split, 16-row blocks) and the direct family (fp32
    MFMAs on operands loaded straight into registers, a K split) are offered
    for M <= 16 and, for fp32, outputs too small to fill the chip with 64x64
    tiles; the direct family also for fp32 outputs of up to four such tiles
    per CU (direct_regime), with K splits that keep its grid within 8
    workgroups per CU; the tile GEMMs
    take any M, and K splits too when their own tiles cannot fill the CUs
    (for tiles small enough to split, at least 4 K steps per split).  This
    is the search space of tune.bench / tune.pick, as `mm_configs` is for
    the reference's tuner (tilec/tune.py:82,148).
    """
    code = _dtype_code_name(dtype)
    out = []
    for v in _lib.variants():
        if v["dtype"] != code or (v["max_m"] and M > v["max_m"]):
            continue
        if v["family"] == _lib.FAMILY_SKINNY and not skinny_regime(M, N, code):
            continue
        if panel_variant(v) and layout is not None and layout & _lib.X2_COL_MAJOR:
            continue  # the panel kernel reads a row-major x2 (it runs the streaming kernel otherwise)
        if pad_variant(v) and not needs_pad(M, K, N, layout, code):
            continue  # aligned operands: the direct-to-LDS variants read them in place
        if v["family"] == _lib.FAMILY_SKINNY and rows_variant(v):
            epl = 4 if code == _lib.F32 else 8  # elements per 16-byte load
            row_tile = v["name"].endswith(("_c128", "_c256"))  # the row-dot kernel takes any K
            if (K % epl == 0 or not row_tile) and (layout is None or layout == _lib.X2_COL_MAJOR):
                out.append((v["name"], 1))  # neither kernel splits K
        elif v["family"] == _lib.FAMILY_DIRECT:
            # Any split that leaves every wave at least one 16-row step;
            # no tile more than twice as tall as M needs.
            if not (skinny_regime(M, N, code) or direct_regime(M, N, code)) or v["bm"] >= 2 * max(M, 16):
                continue
            # Splits that fill the CUs exactly once or twice over are
            # offered beside the powers of two; none that takes the grid
            # past 8 workgroups per CU (a K split is there to fill the chip:
            # on MI355X the cap moved the measured best of 5 of 842 timed
            # shapes, by at most 3.5 %, and keeps the tuner off splits that
            # launch 100 000 workgroups) and none whose partials would reach
            # the library's 2 GiB limit.
            tiles = cdiv(M, v["bm"]) * cdiv(N, v["bn"])
            if tiles == 0:
                continue  # an empty output: nothing for a K split to fill
            fills = [f for f in (device_cus() // tiles, 2 * device_cus() // tiles) if f > 1]
            seen = set()
            for s in sorted(set(_SKINNY_SPLITS) | set(fills)):
                eff = _direct_splits(K, s)
                if eff in seen or (eff > 1 and cdiv(K, eff) < 16 * v["waves"]):
                    continue
                if eff > 1 and tiles * eff > 8 * device_cus():
                    continue
                if eff > 1 and direct_workspace_bytes(v, M, N, eff) >= 1 << 31:
                    continue
                seen.add(eff)
                out.append((v["name"], s))
        elif v["family"] == _lib.FAMILY_SKINNY:
            # A workgroup takes at most BK (the variant's K-slice cap) rows
            # of K, so small splits are raised; keep one entry per distinct
            # effective split, each giving every wave at least one 16-row block.
            seen = set()
            for s in _SKINNY_SPLITS:
                eff = _skinny_splits(K, s, v["bk"])
                if eff in seen or (eff > 1 and K // eff < 16 * v["waves"]):
                    continue
                seen.add(eff)
                out.append((v["name"], s))
        else:
            out.append((v["name"], 1))
            tiles = cdiv(M, v["bm"]) * cdiv(N, v["bn"])
            if tiles < device_cus() and tile_can_split(v):
                seen = {1}
                for s in _GEMM_SPLITS:
                    eff = _gemm_splits(K, s, v["bk"])
                    if eff in seen or cdiv(K, v["bk"]) < 4 * eff:
                        continue
                    seen.add(eff)
                    out.append((v["name"], s))
    return out


_GEMM_SPLITS = (2, 4, 8, 16)
SPLIT_MAX_ACC_PER_THREAD = 64  # tilec/csrc/common.h, kSplitMaxAccPerThread


def rows_variant(v):
    """Variants named *_t<MR>_r<R>_* run a kernel for x @ W.T over all of K,
    with no K split (csrc/skinny.hip): the row-dot kernel (gemv_rows_kernel,
    one wave per 1-2 rows of W, M <= 4) or the row-tile kernel (*_c128 /
    *_c256: gemv_wt_kernel, 16 rows of W per workgroup, M <= 16); other
    layouts run the streaming kernel."""
    return re.search(r"_t\d+_r\d+_", v["name"]) is not None


def panel_variant(v):
    """Variants named *_p_v<M>_* run the panel kernel (csrc/panel.hip) for a
    row-major x2 and M up to <M>."""
    return "_p_v" in v["name"]


def pad_variant(v):
    """Variants named *_pad copy both operands into the workspace with rows
    padded to 16 bytes and K to the K step (zeros), then run the
    direct-to-LDS tile kernel (csrc/gemm_f32.hip, launch_gemm_f32_pad;
    csrc/gemm_bf16.hip, launch_gemm_bf16_pad)."""
    return v["name"].endswith("_pad")


def needs_pad(M, K, N, layout=None, dtype="f32"):
    """Whether an operand's rows are not whole 16-byte groups (4 fp32 or 8
    bf16 elements) along its contiguous extent (K of a row-major x1 or of a
    column-major x2, M of a column-major x1, N of a row-major x2), so the
    direct-to-LDS tile variants would run their slower fallback kernel."""
    layout = layout or 0
    epl = 4 if _dtype_code_name(dtype) == _lib.F32 else 8
    run1 = M if layout & _lib.X1_COL_MAJOR else K
    run2 = K if layout & _lib.X2_COL_MAJOR else N
    return run1 % epl != 0 or run2 % epl != 0


def prep_variant(v):
    """Variants named *_kc transpose each operand that is not k-contiguous
    into the workspace before the GEMM (csrc/common.h, VariantDesc::prep);
    they never split K."""
    return v["name"].endswith("_kc")


def tile_can_split(v):
    """Whether a tile-GEMM variant splits K (its threads hold at most 64
    accumulators; csrc/common.h, tile_can_split; prep variants never do)."""
    return not prep_variant(v) and v["bm"] * v["bn"] <= SPLIT_MAX_ACC_PER_THREAD * 64 * v["waves"]


def _gemm_splits(K, split_k, bk):
    """Splits a tile GEMM actually runs (csrc/common.h, gemm_split_geom)."""
    total = cdiv(K, bk)
    if total <= 0:
        return 1
    s = min(max(split_k, 1), total)
    steps = cdiv(total, s)
    return cdiv(total, steps)


_CUS = None


def device_cus():
    """CUs of the current GPU, read once (the library's own rule reads the
    same count); 64x64 output tiles below this count leave CUs idle.  256, an
    MI355X's count, where no GPU is visible (host-side tests)."""
    global _CUS
    if _CUS is None:
        _CUS = (torch.cuda.get_device_properties(torch.cuda.current_device()).multi_processor_count
                if torch.cuda.is_available() else 256)
    return _CUS


def skinny_regime(M, N, dtype="f32"):
    """Whether the streaming (skinny) kernels are candidates: M <= 16, or for
    fp32 also fewer 64x64 output tiles than CUs (the rule of
    tilec_select_variant).  bf16 inputs stream through fp32 MFMAs, so past
    16 rows the bf16 tile GEMMs (with a K split) serve them better."""
    if M <= 16:
        return True
    return _dtype_code_name(dtype) == _lib.F32 and cdiv(M, 64) * cdiv(N, 64) < device_cus()


def direct_regime(M, N, dtype="f32"):
    """Whether the direct-operand kernel is also a candidate past the
    small-output rule: fp32 outputs of up to four 64x64 tiles per CU
    (1024^2 .. 2048^2-sized), where the tile GEMMs' large tiles leave CUs
    idle or need a K split and the direct kernel's 32x64 tiles (two register
    sets of operands in flight) fill the chip unsplit."""
    return _dtype_code_name(dtype) == _lib.F32 and cdiv(M, 64) * cdiv(N, 64) <= 4 * device_cus()


def _skinny_splits(K, split_k, kc_max):
    """Splits the skinny kernel actually runs (tilec/csrc/skinny.hip, skinny_geom)."""
    if K <= 0:
        return 1
    s = max(split_k, 1, cdiv(K, kc_max))
    kc = cdiv(cdiv(K, s), 16) * 16
    return cdiv(K, kc)


def direct_workspace_bytes(v, M, N, splits):
    """Split-K partials of a direct variant (tilec/csrc/direct.hip,
    direct_workspace_bytes): splits x tiles x (16-byte results per thread
    after the waves meet) x threads."""
    items = 4 * (v["bm"] // 16) * (v["bn"] // 64)
    return splits * cdiv(M, v["bm"]) * cdiv(N, v["bn"]) * cdiv(items, v["waves"]) * v["waves"] * 64 * 16


def _direct_splits(K, split_k):
    """Splits the direct kernel actually runs (tilec/csrc/direct.hip, direct_geom)."""
    if K <= 0:
        return 1
    kc = cdiv(cdiv(K, max(split_k, 1)), 16) * 16
    return cdiv(K, kc)


def _dtype_code_name(dtype):
    if dtype in ("f32", "float32", torch.float32, _lib.F32):
        return _lib.F32
    if dtype in ("bf16", "bfloat16", torch.bfloat16, _lib.BF16):
        return _lib.BF16
    raise TypeError(f"unsupported dtype {dtype!r} (use float32 or bfloat16)")


# ---------------------------------------------------------------------------
# Split-K buffers, one pair per (device, stream): scratch for the partial sums
# (any contents) and completion counters, zeroed once at allocation; every
# completed call leaves the counters zero, so both are reused across calls of
# any shape.  A buffer is only replaced (by a larger one) when a call needs
# more; code that captures calls into a HIP graph runs them once before
# capture so the buffers the graph records stay in place.
# ---------------------------------------------------------------------------

_SCRATCH = {}
_COUNTERS = {}


def _buffer(table, device, stream, nbytes, zero, quantum):
    key = (device.index, stream)
    buf = table.get(key)
    if buf is None or buf.numel() < nbytes:
        size = max(nbytes, quantum)
        size = (size + quantum - 1) // quantum * quantum
        buf = (torch.zeros if zero else torch.empty)(size, dtype=torch.uint8, device=device)
        table[key] = buf
    return buf


def workspace_for(device, stream, nbytes):
    """Scratch (uint8 device tensor, >= nbytes) for split-K partial sums."""
    return _buffer(_SCRATCH, device, stream, nbytes, False, 1 << 20)


def counters_for(device, stream, nbytes):
    """Zero-initialised completion counters (uint8 device tensor, >= nbytes)."""
    return _buffer(_COUNTERS, device, stream, nbytes, True, 1 << 16)


# ---------------------------------------------------------------------------
# The op
# ---------------------------------------------------------------------------

def _operand(x, rows, cols):
    """(tensor, leading dimension, column-major?) the kernels read in place:
    row-major with unit column stride and a row stride >= cols, or
    column-major (the transposed view x.T of a row-major matrix) with unit
    row stride and a column stride >= rows; anything else (broadcast,
    negative or doubly strided views) gets the reference's `.contiguous()`
    copy (tilec/ext.py:59-60).  Size-1 dimensions impose no stride."""
    if rows == 0 or cols == 0:
        return x, max(cols, 1), False
    s0, s1 = x.stride()
    if (cols == 1 or s1 == 1) and (rows == 1 or s0 >= cols):
        return x, (s0 if rows > 1 else cols), False
    if (rows == 1 or s0 == 1) and (cols == 1 or s1 >= rows):
        return x, (s1 if cols > 1 else rows), True
    return x.contiguous(), cols, False


def layout_of(x1, x2):
    """The layout bits tilec_matmul gets for these operands (0 = both
    row-major; after a `.contiguous()` copy an operand is row-major)."""
    M, K = x1.shape
    N = x2.shape[1]
    return ((_lib.X1_COL_MAJOR if _operand(x1, M, K)[2] else 0) |
            (_lib.X2_COL_MAJOR if _operand(x2, K, N)[2] else 0))


def _prepare(x1, x2):
    if x1.dim() != 2 or x2.dim() != 2:
        raise ValueError(f"matrix_mul: expected 2-D tensors, got shapes {tuple(x1.shape)} "
                         f"and {tuple(x2.shape)}")
    M, K = x1.shape
    K2, N = x2.shape
    if K != K2:
        raise ValueError(f"matrix_mul: shapes {tuple(x1.shape)} and {tuple(x2.shape)} don't match")
    if x1.dtype != x2.dtype or x1.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"unsupported kernel arguments of dtype {x1.dtype} and {x2.dtype} "
                        "(use float32 tensors, or bfloat16 tensors)")
    if x1.device.type != "cuda" or x2.device != x1.device:
        raise TypeError(f"matrix_mul needs both tensors on one ROCm GPU "
                        f"(got {x1.device} and {x2.device})")
    return M, K, N


@lru_cache(4096)
def _scratch_sizes(M, N, K, lda, ldb, layout, dtype, variant, split_k):
    """(workspace, counter) bytes a call needs, for exactly the arguments
    tilec_matmul gets (layout and strides decide what TILEC_VARIANT_AUTO
    runs); the C ABI's answer depends only on these arguments, so repeat
    calls skip the library crossing."""
    ws, cnt = ctypes.c_size_t(0), ctypes.c_size_t(0)
    rc = _lib.lib().tilec_matmul_scratch_bytes(M, N, K, lda, ldb, layout, dtype, variant, split_k,
                                               ctypes.byref(ws), ctypes.byref(cnt))
    if rc:
        _lib.check(rc)
    return ws.value, cnt.value


def _launch(x1, x2, M, K, N, variant, split_k, ops=None):
    """Enqueue one tilec_matmul on the current stream.  `ops`: the two
    (tensor, leading dimension, column-major?) triples of `_operand`, when
    the caller has them already."""
    dtype = _lib.F32 if x1.dtype == torch.float32 else _lib.BF16
    (a, lda, ca), (b, ldb, cb) = ops or (_operand(x1, M, K), _operand(x2, K, N))
    layout = (_lib.X1_COL_MAJOR if ca else 0) | (_lib.X2_COL_MAJOR if cb else 0)
    out = torch.empty((M, N), dtype=torch.float32, device=x1.device)
    if M == 0 or N == 0:
        return out
    stream = torch.cuda.current_stream(x1.device).cuda_stream
    ws_ptr, ws_bytes, cnt_ptr, cnt_bytes = None, 0, None, 0
    need, need_cnt = _scratch_sizes(M, N, K, lda, ldb, layout, dtype, variant, split_k)
    if need:
        ws = workspace_for(x1.device, stream, need)
        ws_ptr, ws_bytes = ws.data_ptr(), ws.numel()
        cnt = counters_for(x1.device, stream, need_cnt)
        cnt_ptr, cnt_bytes = cnt.data_ptr(), cnt.numel()
    rc = _lib.lib().tilec_matmul(a.data_ptr(), b.data_ptr(), out.data_ptr(), M, N, K, lda, ldb, N, layout,
                                 dtype, variant, split_k, ws_ptr, ws_bytes, cnt_ptr, cnt_bytes, stream)
    if rc:
        _lib.check(rc)
    return out


@lru_cache(4096)
def _tuned(M, K, N, dtype, layout):
    """(variant id, split_k) for the tuned pick of a shape, resolved once."""
    from . import tune
    config = tune.pick(M, K, N, dtype, layout)
    if config is None:
        return _lib.VARIANT_AUTO, 0
    return _lib.variant_id(config[0]), int(config[1])


def _resolve_config(config, M, K, N, dtype, layout=0):
    """config: None (tuned pick for this shape and layout), a variant name /
    id, or (variant, split_k)."""
    if config is None:
        return _tuned(M, K, N, "bf16" if dtype == torch.bfloat16 else "f32", layout)
    if isinstance(config, (str, int)):
        config = (config, 0)
    variant, split_k = config
    if isinstance(variant, str):
        variant = _lib.variant_id(variant)
    return int(variant), int(split_k)


def matrix_mul(x1, x2, config=None):
    """out[M,N] (float32) = x1[M,K] · x2[K,N] on the GPU.

    Same contract as the reference (tilec/ext.py:54-67): ValueError when K does
    not match, the output is new.  Inputs are float32, or bfloat16 (fp32
    accumulate, fp32 output).  Row-strided and transposed views (x.T) are
    read in place; only other strided views get the reference's
    `.contiguous()` copy.  `config`
    (optional, as the reference's tuner passes it, tilec/tune.py:37) forces a
    (variant, split_k) from `hip_configs`.
    """
    M, K, N = _prepare(x1, x2)
    ops = (_operand(x1, M, K), _operand(x2, K, N))
    layout = (_lib.X1_COL_MAJOR if ops[0][2] else 0) | (_lib.X2_COL_MAJOR if ops[1][2] else 0)
    variant, split_k = _resolve_config(config, M, K, N, x1.dtype, layout)
    return _launch(x1, x2, M, K, N, variant, split_k, ops)


def _matrix_mul_tiled(x1, x2, BM=64, BN=64, BK=16):
    """Run the tile GEMM with a given output tile, as the reference's
    `_matrix_mul_tiled(x1, x2, BM, BN, BK)` does (tilec/ext.py:54-63).

    Tiles are compiled ahead of time; (BM, BN) must name one of them.  BK must
    match too for float32; bfloat16 kernels step K by their own BK.
    """
    M, K, N = _prepare(x1, x2)
    code = _lib.F32 if x1.dtype == torch.float32 else _lib.BF16
    tiles = [v for v in _lib.variants()
             if v["family"] == _lib.FAMILY_GEMM and v["dtype"] == code and (v["bm"], v["bn"]) == (BM, BN)]
    exact = [v for v in tiles if v["bk"] == BK]
    chosen = exact or (tiles if code == _lib.BF16 else [])
    if not chosen:
        have = sorted({(v["bm"], v["bn"], v["bk"]) for v in _lib.variants()
                       if v["family"] == _lib.FAMILY_GEMM and v["dtype"] == code})
        raise ValueError(f"_matrix_mul_tiled: no compiled tile BM={BM} BN={BN} BK={BK} "
                         f"for {x1.dtype}; available (BM, BN, BK): {have}")
    return _launch(x1, x2, M, K, N, chosen[0]["id"], 1)


def sum(x, axis=1):
    """Row sums (axis=1: out[r] = sum_c x[r, c], shape [R]) or column sums
    (axis=0: out[c] = sum_r x[r, c], shape [C]) of a 2-D float32 or bfloat16
    tensor on the GPU, accumulated and returned in float32.  A 1-D x is one
    row.

    The reduction the reference plans as `tl.sum` (README.md:88) and shows
    as the `row_sum` kernel, `out[r] = tl.sum(x[r, :])`, with the op-level
    spelling `tl.ext.sum(x, axis=1)` (kernel1.py:8-15).  Row- and
    column-major views are read in place; other strided views are copied
    first.  Long reductions with few outputs split across workgroups and
    combine in a fixed order: results are deterministic.
    """
    if x.dim() == 1:
        x = x.unsqueeze(0)
    if x.dim() != 2:
        raise ValueError(f"sum: expected a 1-D or 2-D tensor, got shape {tuple(x.shape)}")
    if axis not in (0, 1, -1, -2):
        raise ValueError(f"sum: axis must be 0 or 1 (got {axis})")
    axis = axis % 2
    if x.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"unsupported tensor of dtype {x.dtype} (use float32 or bfloat16)")
    if x.device.type != "cuda":
        raise TypeError(f"sum needs a tensor on a ROCm GPU (got {x.device})")
    R, C = x.shape
    out = torch.empty((R if axis == 1 else C,), dtype=torch.float32, device=x.device)
    if out.numel() == 0:
        return out
    t, ld, col = _operand(x, R, C)
    layout = _lib.X1_COL_MAJOR if col else 0
    dtype = _lib.F32 if x.dtype == torch.float32 else _lib.BF16
    L = _lib.lib()
    stream = torch.cuda.current_stream(x.device).cuda_stream
    ws_ptr, ws_bytes, cnt_ptr, cnt_bytes = None, 0, None, 0
    need = L.tilec_sum_workspace_bytes(R, C, layout, dtype, axis)
    if need:
        ws = workspace_for(x.device, stream, need)
        ws_ptr, ws_bytes = ws.data_ptr(), ws.numel()
        cnt = counters_for(x.device, stream, L.tilec_sum_counter_bytes(R, C, layout, dtype, axis))
        cnt_ptr, cnt_bytes = cnt.data_ptr(), cnt.numel()
    _lib.check(L.tilec_sum(t.data_ptr(), out.data_ptr(), R, C, ld, layout, dtype, axis,
                           ws_ptr, ws_bytes, cnt_ptr, cnt_bytes, stream))
    return out
