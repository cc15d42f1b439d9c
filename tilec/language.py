"""Host-side helpers of the reference's tile language that the matmul path uses.

Only `cdiv` is on the hot path (grid math); the DSL builtins
(`tl.load`, `tl.dot`, ...; tilec/language.py:1-14) belong to the tile compiler,
which this implementation replaces with hand-written gfx950 kernels.
"""


def cdiv(a, b):
    """Ceiling division, for host code: cdiv(5000, 4096) == 2.

    Restates tilec/language.py:16-18.
    """
    return (a + b - 1) // b
