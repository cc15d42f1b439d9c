"""`tilec.ext` (the reference's op module, tilec/ext.py), served by tilec_amd.ext."""

from tilec_amd.ext import *  # noqa: F401,F403
from tilec_amd.ext import __all__  # noqa: F401
