"""tilec: tilec's matmul op on MI355X (gfx950), with the reference's package name
(tilec/__init__.py).

    import torch, tilec
    out = tilec.ext.matrix_mul(x1, x2)   # x1, x2 on a ROCm GPU

`ext.matrix_mul(x1, x2)` runs hand-written HIP kernels (libtilec_hip.so,
built by `python -m tilec.build`) on PyTorch-ROCm tensors; `ext.sum` is the
row/column reduction; `tune` holds the MI355X shape->config model.  Only the
op API is provided: the tile DSL compiler (`tilec.jit`, `tilec.CompileError`)
is not part of this implementation.
"""

from . import ext, language, tune

__all__ = ["ext", "language", "tune"]
__version__ = "1.0.0"
