"""Caller-side helpers of the reference's `deep_gemm.utils` (quantizers and layout aliases)."""
from . import math, layout  # noqa: F401
from .layout import *  # noqa: F401,F403
from .math import *  # noqa: F401,F403
