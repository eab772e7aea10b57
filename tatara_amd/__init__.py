"""tatara_amd: MI355X (gfx950) training backend for tatara's GPU hot path.

The compute path is libtatara_hip.so (hand-written HIP kernels behind the C
ABI of include/tatara_hip.h); this package is its host-side mirror of the
reference's step API (trait TrainerBackend).  There is no CPU fallback.
"""
from .trainer import (Batch, DeviceArray, DeviceBatch, LayerStackConfig, LayerStackTrainer,  # noqa: F401
                      Sigmoid, Wrm)

__all__ = ["Batch", "DeviceArray", "DeviceBatch", "LayerStackConfig", "LayerStackTrainer",
           "Sigmoid", "Wrm"]
