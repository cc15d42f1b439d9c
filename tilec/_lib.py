"""ctypes binding of libtilec_hip.so (the C ABI declared in include/tilec.h).

This module replaces the reference's compile-and-launch layer
(`JITFunction.run` / `_launch`, tilec/jit.py:81-105): instead of compiling
Metal per specialization and launching it through `torch.mps`, the host calls
precompiled gfx950 kernels through a plain C ABI.  There is no fallback: if
the library is missing, every call raises.
"""

import ctypes
import os
from functools import lru_cache

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtilec_hip.so")

# Status codes and enums (include/tilec.h).
OK, ERR_VALUE, ERR_TYPE, ERR_UNSUPPORTED, ERR_WORKSPACE, ERR_HIP = 0, 1, 2, 3, 4, 5
F32, BF16 = 0, 1
FAMILY_SKINNY, FAMILY_GEMM, FAMILY_DIRECT = 0, 1, 2
X1_COL_MAJOR, X2_COL_MAJOR = 1, 2  # layout bits
VARIANT_AUTO = -1

# Every function include/tilec.h declares: name -> (restype, argtypes).
_i64, _i32, _vp, _sz = ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p, ctypes.c_size_t
SIGNATURES = {
    "tilec_matmul": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i32,
                                    _i32, _i32, _i32, _vp, _sz, _vp, _sz, _vp]),
    "tilec_matmul_noalloc": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i32,
                                            _i32, _i32, _i32, _vp]),
    "tilec_matmul_workspace_bytes": (_sz, [_i64, _i64, _i64, _i32, _i32, _i32]),
    "tilec_matmul_counter_bytes": (_sz, [_i64, _i64, _i64, _i32, _i32, _i32]),
    "tilec_matmul_scratch_bytes": (ctypes.c_int, [_i64, _i64, _i64, _i64, _i64, _i32, _i32, _i32, _i32,
                                                  ctypes.POINTER(_sz), ctypes.POINTER(_sz)]),
    "tilec_sum": (ctypes.c_int, [_vp, _vp, _i64, _i64, _i64, _i32, _i32, _i32, _vp, _sz, _vp, _sz, _vp]),
    "tilec_sum_workspace_bytes": (_sz, [_i64, _i64, _i32, _i32, _i32]),
    "tilec_read_floor": (ctypes.c_int, [_vp, _sz, _vp, _i32, _vp]),
    "tilec_sum_counter_bytes": (_sz, [_i64, _i64, _i32, _i32, _i32]),
    "tilec_select_variant": (_i32, [_i64, _i64, _i64, _i32]),
    "tilec_select_variant_layout": (_i32, [_i64, _i64, _i64, _i32, _i32, _i64, _i64]),
    "tilec_auto_split_k": (_i32, [_i64, _i64, _i64, _i32, _i32]),
    "tilec_num_variants": (_i32, []),
    "tilec_variant_info": (ctypes.c_int, [_i32, ctypes.POINTER(_i32), ctypes.POINTER(ctypes.c_char_p)]),
    "tilec_last_error": (ctypes.c_char_p, []),
    "tilec_version": (_i32, []),
}


class LibraryMissing(RuntimeError):
    pass


@lru_cache(None)
def lib():
    """Load libtilec_hip.so once; raise if it has not been built."""
    if not os.path.exists(LIB_PATH):
        raise LibraryMissing(
            f"{LIB_PATH} is not built; run `python -m tilec.build` "
            "(or __graft_entry__.build()) first")
    L = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    return L


def last_error():
    return lib().tilec_last_error().decode(errors="replace")


def check(rc):
    """Map a C-ABI status to the reference's exception types (tilec/ext.py:57-58,
    tilec/jit.py:34-39)."""
    if rc == OK:
        return
    msg = last_error() or f"tilec status {rc}"
    if rc == ERR_VALUE:
        raise ValueError(msg)
    if rc == ERR_TYPE:
        raise TypeError(msg)
    raise RuntimeError(msg)


@lru_cache(None)
def variants():
    """All compiled variants: list of dicts, index == variant id."""
    L = lib()
    out = []
    for v in range(L.tilec_num_variants()):
        info = (_i32 * 8)()
        name = ctypes.c_char_p()
        check(L.tilec_variant_info(v, info, ctypes.byref(name)))
        out.append(dict(id=v, name=name.value.decode(), family=info[0], dtype=info[1],
                        bm=info[2], bn=info[3], bk=info[4], waves=info[5],
                        max_m=info[6], unroll=info[7]))
    return out


@lru_cache(None)
def variant_id(name):
    for v in variants():
        if v["name"] == name:
            return v["id"]
    raise ValueError(f"no compiled variant named {name!r}")
