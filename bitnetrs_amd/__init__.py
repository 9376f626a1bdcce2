"""bitnetrs_amd -- MI355X (gfx950) GQA attention hot path of bitnetrs.

RoPE (half-split) on Q/K, KV-cache append into an HBM-resident head-major
cache, split-K decode attention and causal prefill, and the W2A8 ternary
GEMV of the layer projections, as hand-written HIP kernels behind the C ABI
in ``include/bitnet_hip.h``.  ``HipBackend`` mirrors the reference's
``Backend::rope_embed`` / ``Backend::masked_attention`` /
``Backend::ternary_gemv_preq``.
"""
from ._lib import LIB_PATH, build, load
from .stack import AttentionStack
from .backend import (BNR_MIRROR_FULL, BNR_MIRROR_INCREMENTAL, BackendError, BitNetError,
                      DeviceKVCache, HipBackend, InvalidConfig, InvalidShape, NativeKVCache,
                      QuantizationError, UnsupportedDevice)

__all__ = ["HipBackend", "DeviceKVCache", "NativeKVCache", "AttentionStack", "BitNetError", "InvalidShape",
           "InvalidConfig", "BackendError", "UnsupportedDevice", "QuantizationError",
           "BNR_MIRROR_FULL", "BNR_MIRROR_INCREMENTAL", "build", "load", "LIB_PATH"]
