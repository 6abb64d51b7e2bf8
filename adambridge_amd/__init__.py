"""adambridge_amd: adambridge's fused AdamW / Lion update, MI355X-native.

The optimizer state (FP32 or FP24 master weights, FP32 / BF16 / FP8 moments)
lives in HBM and one hand-written HIP kernel for gfx950 updates a whole batch
of parameters per launch.  The public API mirrors the reference package
``adambridge`` (adambridge/__init__.py:4-25).
"""

from . import native, precision
from .engine import StepStats
from .losses import causal_lm_loss
from .optimizer import AdamBridge, AutoTuneConfig, LionBridge, OptiComputeAdamW
from .precision import bytes_per_param

__version__ = "0.1.0"

__all__ = [
    "AdamBridge",
    "LionBridge",
    "OptiComputeAdamW",
    "AutoTuneConfig",
    "StepStats",
    "bytes_per_param",
    "causal_lm_loss",
    "native",
    "precision",
    "__version__",
]
