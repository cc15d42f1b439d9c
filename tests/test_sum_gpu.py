"""GPU parity of tilec.ext.sum (row / column sums) on an MI355X.

The reference plans the reduction as `tl.sum` (README.md:88) and shows it as
the `row_sum` kernel of kernel1.py:8-15, checked there against numpy's
x.sum(axis=1) on arange(32).reshape(4, 8).  Here: that example exactly,
ragged shapes in both axes, dtypes and layouts against the fp64 oracle (per
output |err| <= 2e-6 * sum |x|, the bound of fp32 accumulation in any order),
small-integer data bit-exact, split and unsplit geometries, determinism,
empty inputs, and size-independent properties at full size.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tilec import _lib, ext
import tilec

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)


def dev(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda").to(dtype)


def col_major(x, pad=0):
    """The [R, C] device matrix x as a column-major view (column stride R + pad)."""
    R, C = x.shape
    buf = torch.zeros((C, R + pad), dtype=x.dtype, device=x.device)
    buf[:, :R] = x.t()
    return buf[:, :R].t()


def check(got, x64, axis, what):
    got = got.cpu().numpy()
    assert got.dtype == np.float32 and got.shape == (x64.shape[0] if axis == 1 else x64.shape[1],), what
    assert O.sum_error_ok(got, x64, axis), what


def test_reference_example_exact():
    """kernel1.py:18-27: row sums of arange(32).reshape(4, 8)."""
    x = dev(np.arange(32, dtype=np.float32).reshape(4, 8))
    rows = tilec.ext.sum(x, axis=1)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(rows.cpu().numpy(), [28, 92, 156, 220])
    np.testing.assert_array_equal(tilec.ext.sum(x, axis=0).cpu().numpy(), [48 + 4 * c for c in range(8)])
    say("kernel1 example ok")


SHAPES = [(1, 1), (3, 5), (4, 8), (17, 65), (64, 1), (1, 4096), (127, 1000), (1000, 127), (256, 16), (300, 257),
          (5, 100003), (3, 1 << 18), (200001, 3), (65536, 17), (2, 8), (4096, 4096)]


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("axis", [1, 0])
def test_sum_shapes_layouts(dtype, axis):
    for i, (R, C) in enumerate(SHAPES):
        x = O.normal((R, C), 1000 + i)
        if dtype == "bf16":
            x = O.bf16_round(x)
            x = O.bf16_to_f32(x)
        t = dev(x, torch.float32 if dtype == "f32" else torch.bfloat16)
        for name, view in (("row-major", t), ("column-major", col_major(t)), ("padded column-major", col_major(t, 5))):
            if name != "row-major" and R * C > (1 << 22):
                continue
            say(f"sum {dtype} axis {axis} {(R, C)} {name}")
            check(ext.sum(view, axis), x, axis, (dtype, axis, (R, C), name))


def test_sum_row_strided_and_misaligned():
    x = O.normal((300, 1000), 1100)
    big = torch.zeros(300, 1003, device="cuda")
    big[:, :1000] = dev(x)
    for axis in (0, 1):
        check(ext.sum(big[:, :1000], axis), x, axis, ("strided", axis))       # row stride 1003
    # every other column: neither row- nor column-major, copied first
    check(ext.sum(big[:, :1000][:, ::2], 1), np.ascontiguousarray(x[:, ::2]), 1, "every other column")
    # an offset view: 4-byte aligned, not 16 (element path)
    flat = torch.zeros(1 + 300 * 1000, device="cuda")
    flat[1:] = dev(x).reshape(-1)
    v = flat[1:].view(300, 1000)
    for axis in (0, 1):
        check(ext.sum(v, axis), x, axis, ("misaligned", axis))
    say("strided ok")


def test_sum_integers_exact_and_deterministic():
    for i, (R, C) in enumerate([(7, 9), (3, 1 << 18), (100000, 33), (1000, 1000)]):
        x = O.small_ints((R, C), 1200 + i).astype(np.float32)
        t = dev(x)
        for axis in (0, 1):
            want = O.sum_f64(x, axis).astype(np.float32)
            got = ext.sum(t, axis)
            again = ext.sum(t, axis)
            torch.cuda.synchronize()
            np.testing.assert_array_equal(got.cpu().numpy(), want)
            assert torch.equal(got, again)
        xb = dev(x, torch.bfloat16)  # |x| <= 8: exact in bf16
        np.testing.assert_array_equal(ext.sum(xb, 1).cpu().numpy(), O.sum_f64(x, 1).astype(np.float32))
    say("integer sums exact")


def test_sum_split_determinism():
    """Split reductions add partials in a fixed order: bit-identical repeats."""
    x = dev(O.normal((3, 1 << 20), 1300))
    y = dev(O.normal((1 << 20, 5), 1301))
    a = [ext.sum(x, 1) for _ in range(5)]
    b = [ext.sum(y, 0) for _ in range(5)]
    torch.cuda.synchronize()
    assert all(torch.equal(a[0], t) for t in a[1:]) and all(torch.equal(b[0], t) for t in b[1:])
    assert _lib.lib().tilec_sum_workspace_bytes(3, 1 << 20, 0, _lib.F32, 1) > 0
    assert _lib.lib().tilec_sum_workspace_bytes(1 << 20, 5, 0, _lib.F32, 0) > 0


def test_sum_empty_and_vectors():
    z = torch.zeros(0, 5, device="cuda")
    assert ext.sum(z, 1).shape == (0,)
    np.testing.assert_array_equal(ext.sum(z, 0).cpu().numpy(), np.zeros(5, np.float32))
    e = torch.zeros(4, 0, device="cuda")
    np.testing.assert_array_equal(ext.sum(e, 1).cpu().numpy(), np.zeros(4, np.float32))
    v = dev(O.normal((1000,), 1400))
    got = ext.sum(v, 1).cpu().numpy()
    assert got.shape == (1,) and O.sum_error_ok(got, v.cpu().numpy()[None, :], 1)
    with pytest.raises(ValueError):
        ext.sum(torch.zeros(2, 2, 2, device="cuda"))
    with pytest.raises(ValueError):
        ext.sum(z, axis=3)
    with pytest.raises(TypeError):
        ext.sum(torch.zeros(2, 2, dtype=torch.float64, device="cuda"))


def test_sum_full_size_properties():
    """4096 x 4096 (the config-1 x2) and a tall bf16 case: totals agree
    between axes and sums are linear, within fp32 accumulation error."""
    a, b = O.normal((4096, 4096), 1500), O.normal((4096, 4096), 1501)
    da, db = dev(a), dev(b)
    rows, cols = ext.sum(da, 1).double(), ext.sum(da, 0).double()
    tot = float(np.abs(a).sum())
    assert abs(float(rows.sum() - cols.sum())) <= 1e-6 * tot
    lin = ext.sum(da + db, 1).double() - ext.sum(da, 1).double() - ext.sum(db, 1).double()
    assert float(lin.abs().max()) <= 1e-5 * float(np.abs(a).sum(1).max() + np.abs(b).sum(1).max())
    t = dev(O.bf16_to_f32(O.bf16_round(O.normal((1 << 20, 64), 1502))), torch.bfloat16)
    r, c = ext.sum(t, 1).double().sum(), ext.sum(t, 0).double().sum()
    assert abs(float(r - c)) <= 1e-5 * float(t.float().abs().sum())
    say("full-size properties ok")


@pytest.mark.parametrize("pieces,workgroups", [(1, 0), (7, 3), (64, 0), (4096, 0), (4096, 1000)])
def test_read_floor_sums(pieces, workgroups):
    """tilec_read_floor (the HBM read floor the GEMV kernels are measured
    against) reads every byte once: the four per-wave sums of workgroup g
    over small-integer data add up to the exact sum of its own pieces
    g, g + G, ..., and wave w's sum to that of 16-byte groups w, w + 4 of
    each 1 KiB row of those pieces."""
    import ctypes
    n = pieces * 4096
    x = O.small_ints((n,), 77 + pieces, -8, 8)
    xd = dev(x)
    L = _lib.lib()
    G = min(workgroups or 2 * torch.cuda.get_device_properties(0).multi_processor_count, pieces)
    sink = torch.full((4 * G + 1,), float("nan"), dtype=torch.float32, device="cuda")
    say(f"read floor: {pieces} pieces, {G} workgroups")
    _lib.check(L.tilec_read_floor(ctypes.c_void_p(xd.data_ptr()), 4 * n, ctypes.c_void_p(sink.data_ptr()),
                                  workgroups, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
    torch.cuda.synchronize()
    got = sink.cpu().numpy()
    assert np.isnan(got[4 * G]), "wrote past its workgroups"
    # a piece is 4 loads x 256 threads x 4 floats; thread t (wave t // 64)
    # reads floats 4 (t + 256 u) .. + 3, u < 4
    per = x.reshape(pieces, 4, 4, 64, 4).astype(np.int64).sum(axis=(1, 3, 4))  # [piece, wave]
    want = np.array([[per[g::G, w].sum() for w in range(4)] for g in range(G)], dtype=np.float32).ravel()
    np.testing.assert_array_equal(got[:4 * G], want)
