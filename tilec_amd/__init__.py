"""tilec_amd: MI355X (gfx950) implementation of tilec's matmul op.

`ext.matrix_mul(x1, x2)` runs hand-written HIP kernels (libtilec_hip.so,
built by `python -m tilec_amd.build`) on PyTorch-ROCm tensors; `tune` holds
the shape→config model.  The `tilec` package re-exports these names so code
written against the reference (`import tilec; tilec.ext.matrix_mul`) runs
unchanged.
"""

from . import ext, language, tune

__all__ = ["ext", "language", "tune"]
__version__ = "1.0.0"
