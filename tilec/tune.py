"""`tilec.tune` (tilec/tune.py), served by tilec_amd.tune — the MI355X tuner."""

from tilec_amd.tune import *  # noqa: F401,F403
from tilec_amd.tune import bench, features, load, machine, pick, shapes, time_ms, train  # noqa: F401
