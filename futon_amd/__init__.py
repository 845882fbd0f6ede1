"""futon encoder forward pass on AMD MI355X (gfx950).

The compute path is libfuton_hip.so (hand-written HIP kernels behind the C ABI
in include/futon_hip.h); this package is its host side, mirroring the
reference's ``native`` API (LoadModel / Model.EncodeTokens / PackConfig).
"""
from .native import (LoadModel, LoadPackConfig, LoadSafetensors, LoadSafetensorsRaw, Model, PackConfig,
                     PackError, ParseSafetensors)
from ._lib import FutonError

__all__ = ["LoadModel", "LoadPackConfig", "LoadSafetensors", "LoadSafetensorsRaw", "Model", "PackConfig",
           "PackError", "ParseSafetensors", "FutonError"]
