"""stacr_amd: MI355X-native STAC-R activation save / weight-gradient path.

Drop-in for the reference package's public API (Manar-Hamed/STAC-R, stacr/__init__.py):
``import stacr_amd as stacr``.  The arithmetic runs in HIP kernels (libstacr_amd.so, C ABI in
include/stacr_amd.h); this package is the host side.
"""
from .adaptive import AdaptiveSTACRConfig, AdaptiveSTACRLinear, apply_adaptive_stacr, set_stacr_runtime_state
from .compressor import STACRCompressor, STACRConfig, stacr_saved_tensors
from .layers import STACRFunction, STACRLinear
from .memory import saved_surface_predictor, stacr_stored_bytes
from .quant import QuantizedValues, quantize_values
from .surgery import apply_stacr, classify, select_target_names, set_step

__all__ = [
    "STACRConfig",
    "STACRCompressor",
    "stacr_saved_tensors",
    "STACRFunction",
    "STACRLinear",
    "apply_stacr",
    "classify",
    "select_target_names",
    "set_step",
    "quantize_values",
    "QuantizedValues",
    "stacr_stored_bytes",
    "saved_surface_predictor",
    "AdaptiveSTACRConfig",
    "AdaptiveSTACRLinear",
    "apply_adaptive_stacr",
    "set_stacr_runtime_state",
]
