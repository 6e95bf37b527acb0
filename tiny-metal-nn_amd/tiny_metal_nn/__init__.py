"""tiny_metal_nn -- MI355X (gfx950) implementation of tiny-metal-nn's
neural-field hot path: hash-grid encoding, fused MLP and Adam as
hand-written HIP kernels behind a C-ABI (include/tmnn_hip.h).

Same module name and Trainer surface as the reference's Python package
(tiny_metal_nn/__init__.py, src/python/tmnn_pybind.cpp).
"""
from __future__ import annotations

from .config import ConfigError, canonicalize_model_config
from .trainer import (ClosedError, ConcurrentTrainingStepError, DTypeError,
                      OptimizerStateBlob, Trainer, philox_uniform, plan_network)

__version__ = "0.1.0"

__all__ = [
    "ClosedError",
    "ConcurrentTrainingStepError",
    "ConfigError",
    "DTypeError",
    "OptimizerStateBlob",
    "Trainer",
    "canonicalize_model_config",
    "philox_uniform",
    "plan_network",
    "__version__",
]
