"""CPU check of the index arithmetic of the row-dot kernel's unaligned form
(tilec/csrc/skinny.hip: gemv_rows_kernel with AL = false), restated step for
step in Python on byte arrays: each row's resource starts at the 16-byte
boundary below the row and ends at the one above its last element; chunk c's
lane l loads the aligned 16 bytes at c * 1008 + 16 l, takes lane l + 1's load
by a shuffle and shifts the pair by the row's misalignment; lane 63 and
elements past K are cleared.  Asserted: the lanes' elements cover 0 .. K - 1
exactly once, in order, with the row's values; loads past the resource read
zeros (as buffer loads past num_records do) and never supply a used byte.
The GPU tests compare the kernel's results with the oracle."""

import random

import numpy as np

from tests.test_pad_copy_index_math import _funnel16, _keep_bytes


def _row(esz, K, b, rng):
    epl = 16 // esz
    ch_elems = 63 * epl
    row = rng.integers(1, 256, size=K * esz, dtype=np.uint8)
    num_records = (b + K * esz + 15) & ~15
    mem = np.zeros(num_records + 64, dtype=np.uint8)
    mem[:num_records] = 0xEE  # bytes of neighbouring rows or padding
    mem[b:b + K * esz] = row

    def load(off):  # a 16-byte buffer load; past num_records it returns zeros
        return mem[off:off + 16].view(np.uint32).tolist() if off + 16 <= num_records else [0, 0, 0, 0]

    covered = []
    nch = -(-K // ch_elems)
    for c in range(nch):
        a0 = [load(c * 1008 + 16 * lane) for lane in range(64)]
        for lane in range(64):
            hi = a0[lane + 1] if lane < 63 else a0[lane]  # shuffle down by one
            x = _funnel16(a0[lane], hi, b)
            kvalid = 0 if lane == 63 else K - c * ch_elems - epl * lane
            if kvalid < epl:
                x = _keep_bytes(x, kvalid * esz)
            got = np.array(x, dtype=np.uint32).view(np.uint8)
            for e in range(epl):
                k = c * ch_elems + epl * lane + e
                val = got[e * esz:(e + 1) * esz]
                if lane < 63 and k < K:
                    np.testing.assert_array_equal(val, row[k * esz:(k + 1) * esz])
                    covered.append(k)
                else:
                    assert not val.any()
    assert covered == list(range(K))


def test_windows_cover_k_once_with_the_row_values():
    rng = np.random.default_rng(3)
    pick = random.Random(4)
    for esz in (2, 4):
        for _ in range(60):
            K = pick.randint(1, 3000)
            b = esz * pick.randint(0, 16 // esz - 1)
            _row(esz, K, b, rng)
