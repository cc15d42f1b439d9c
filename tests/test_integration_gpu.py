"""The reference-side binding of the repository's integration guide, run as
written.

The guide shows the ctypes stub a maintainer of the reference would put in
tilec/ext.py in place of the Metal launch.  This test takes that code block
verbatim (only the library path is made absolute), executes it, and checks
its matrix_mul and sum against the oracle, so the documented binding cannot
drift from include/tilec.h.
"""

import os
import re

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tilec import _lib

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GUIDE = "INTEGRATION.md"


def _stub_namespace():
    text = open(os.path.join(ROOT, GUIDE)).read()
    blocks = re.findall(r"```python\n(.*?)```", text, flags=re.S)
    assert blocks, "the integration guide has no python block"
    code = blocks[0]
    assert 'ctypes.CDLL("libtilec_hip.so")' in code
    code = code.replace('ctypes.CDLL("libtilec_hip.so")', f"ctypes.CDLL({_lib.LIB_PATH!r})")
    ns = {}
    exec(compile(code, GUIDE, "exec"), ns)
    return ns


def test_documented_binding_runs():
    ns = _stub_namespace()
    for i, (m, k, n) in enumerate([(65, 17, 63), (4, 4096, 4096), (300, 1000, 257)]):
        a, b = O.normal((m, k), 3000 + i), O.normal((k, n), 3001 + i)
        out = ns["matrix_mul"](torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda())
        torch.cuda.synchronize()
        assert O.rel_l2(out.cpu().numpy(), O.matmul_f64(a, b)) <= O.TOL_F32, (m, k, n)
    with pytest.raises(ValueError):
        ns["matrix_mul"](torch.zeros(3, 4, device="cuda"), torch.zeros(5, 6, device="cuda"))
    x = np.arange(32, dtype=np.float32).reshape(4, 8)
    np.testing.assert_array_equal(ns["sum"](torch.from_numpy(x).cuda(), 1).cpu().numpy(), [28, 92, 156, 220])
    y = O.normal((3, 1 << 18), 3010)  # a split sum (workspace and counters)
    got = ns["sum"](torch.from_numpy(y).cuda(), 1).cpu().numpy()
    assert O.sum_error_ok(got, y, 1)
