"""raya_amd: MI355X (gfx950) backend for raya's block-local attention hot path.

The compute lives in libraya_hip.so (hand-written HIP kernels behind the C ABI
of include/raya_hip.h); this package is the host-side mirror of the
reference's `raya-kernels` interface (see ``raya_amd.kernels``).
"""
from .kernels import (AttentionKernel, AttnParams, AttnShape, BLOCK, DeviceError, GemmBackend,
                      HipAttention, HipGemm, KernelError, LengthError, Mask, ShapeError,
                      StageTimes, UnsupportedError, WINDOW)

__all__ = ["AttentionKernel", "AttnParams", "AttnShape", "BLOCK", "DeviceError", "GemmBackend",
           "HipAttention", "HipGemm", "KernelError", "LengthError", "Mask", "ShapeError",
           "StageTimes", "UnsupportedError", "WINDOW"]
