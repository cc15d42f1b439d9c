"""tilec — the reference's package name (tilec/__init__.py), backed by the
MI355X implementation in tilec_amd.

    import torch, tilec
    out = tilec.ext.matrix_mul(x1, x2)   # x1, x2 on a ROCm GPU

Only the op API is provided; the tile DSL compiler (`tilec.jit`,
`tilec.CompileError`) is not part of this implementation.
"""

from . import ext, language, tune

__all__ = ["ext", "language", "tune"]
__version__ = "1.0.0"
