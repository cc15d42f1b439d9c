"""CPU checks of the index arithmetic of the pad variants' operand copy
(tilec/csrc/common.h: pad_copy_kernel, funnel16, keep_bytes, and the launch
geometry of pad_copy), restated step for step in Python on byte arrays:

* every 16-byte output chunk equals the zero-padded input row, for either
  element size, any base misalignment, row stride, and padded extents;
* every load a lane issues lies inside the 16-byte aligned chunks that the
  row it serves touches (no access past the matrix, no page it does not
  touch);
* the 1-D grid (first operand's workgroups, then the second's, each over its
  own gx x gy grid with a grid-stride row loop) writes every (row, chunk) of
  both operands exactly once.

These pin the device code's arithmetic, not the product: the GPU tests
compare the pad variants' results with the oracle."""

import random

import numpy as np


def _alignbyte(hi, lo, s):
    return (((hi << 32) | lo) >> (8 * (s & 3))) & 0xFFFFFFFF


def _funnel16(lo, hi, b):
    d = list(lo) + list(hi)
    w, rb = b >> 2, b & 3
    e = [d[j + w] for j in range(5)]
    return [_alignbyte(e[j + 1], e[j], rb) for j in range(4)]


def _keep_bytes(v, keep):
    out = []
    for j in range(4):
        kb = keep - 4 * j
        out.append(v[j] if kb >= 4 else 0 if kb <= 0 else v[j] & ((1 << (8 * kb)) - 1))
    return out


def _copy(esz, R, C, ld, Rp, Cp, base_off, rng):
    epc = 16 // esz
    start_addr = 4096 + base_off * esz
    nbytes = ((R - 1) * ld + C) * esz
    mem = np.zeros(start_addr + nbytes + 64, dtype=np.uint8)
    mem[start_addr:start_addr + nbytes] = rng.integers(1, 256, size=nbytes, dtype=np.uint8)
    want = np.zeros((Rp, Cp * esz), dtype=np.uint8)
    for r in range(R):
        want[r, :C * esz] = mem[start_addr + r * ld * esz:start_addr + (r * ld + C) * esz]
    got = np.zeros_like(want)
    for r in range(Rp):
        for ch in range(Cp // epc):
            c0 = ch * epc
            v = [0, 0, 0, 0]
            if r < R and c0 < C:
                start = start_addr + r * ld * esz
                lo_row, hi_row = start & ~15, (start + C * esz + 15) & ~15
                b = start & 15
                lo = start - b + c0 * esz
                assert lo_row <= lo and lo + 16 <= hi_row
                a0 = mem[lo:lo + 16].view(np.uint32).tolist()
                a1 = [0, 0, 0, 0]
                if b != 0 and c0 * esz + 16 < b + C * esz:
                    assert lo + 32 <= hi_row
                    a1 = mem[lo + 16:lo + 32].view(np.uint32).tolist()
                v = _funnel16(a0, a1, b)
                if c0 + epc > C:
                    v = _keep_bytes(v, (C - c0) * esz)
            got[r, c0 * esz:(c0 + epc) * esz] = np.array(v, dtype=np.uint32).view(np.uint8)
    np.testing.assert_array_equal(got, want)


def test_copy_bytes_and_load_bounds():
    rng = np.random.default_rng(0)
    pick = random.Random(1)
    for esz in (2, 4):
        epc = 16 // esz
        for _ in range(150):
            R, C = pick.randint(1, 7), pick.randint(1, 40)
            ld = C + pick.randint(0, 9)
            Rp = R + pick.randint(0, 3)
            Cp = -(-C // epc) * epc + epc * pick.randint(0, 2)
            _copy(esz, R, C, ld, Rp, Cp, pick.randint(0, epc - 1), rng)


def _op(Rp, Cp, epc):
    nch = Cp // epc
    lg = 0
    while lg < 8 and (1 << lg) < nch:
        lg += 1
    rpb = 256 >> lg
    gx = (nch + (1 << lg) - 1) >> lg
    gy = -(-Rp // rpb) if Rp > 0 and gx > 0 else 0
    while gy > 1 and gx * gy > (1 << 29):
        gy = (gy + 1) // 2
    return dict(Rp=Rp, nch=nch, lg=lg, rpb=rpb, gx=gx, gy=gy)


def test_grid_writes_every_chunk_once():
    pick = random.Random(2)
    for _ in range(120):
        epc = pick.choice((4, 8))
        ops = [_op(pick.randint(0, 200), epc * pick.randint(0, 400), epc) for _ in range(2)]
        n0 = ops[0]["gx"] * ops[0]["gy"]
        blocks = n0 + ops[1]["gx"] * ops[1]["gy"]
        seen = [set(), set()]
        for blk in range(blocks):
            second = blk >= n0
            o = ops[second]
            b = blk - (n0 if second else 0)
            bx, by = b % o["gx"], b // o["gx"]
            for tid in range(256):
                ch = bx * (1 << o["lg"]) + (tid & ((1 << o["lg"]) - 1))
                if ch >= o["nch"]:
                    continue
                r = by * o["rpb"] + (tid >> o["lg"])
                while r < o["Rp"]:
                    assert (r, ch) not in seen[second]
                    seen[second].add((r, ch))
                    r += o["gy"] * o["rpb"]
        for i in range(2):
            assert len(seen[i]) == ops[i]["Rp"] * ops[i]["nch"]
