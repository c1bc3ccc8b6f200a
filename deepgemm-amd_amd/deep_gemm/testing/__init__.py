"""Metric and timing helpers of the reference's `deep_gemm.testing`."""
from . import bench, numeric  # noqa: F401
from .bench import *  # noqa: F401,F403
from .numeric import *  # noqa: F401,F403
