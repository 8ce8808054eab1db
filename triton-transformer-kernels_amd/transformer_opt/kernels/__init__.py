"""gfx950 HIP kernels behind the reference's kernel-module surface."""

from .attention import hip_attention, hip_available, triton_attention, triton_available
from .gelu import gelu, gelu_
from .linear import linear, linear_gelu, linear_supported
from .linear_ln import linear_ln_supported, linear_residual_layer_norm, pack_weight
from .residual_layer_norm import fused_residual_layer_norm, layer_norm, short_layer_norm

__all__ = [
    "fused_residual_layer_norm",
    "gelu",
    "gelu_",
    "hip_attention",
    "hip_available",
    "layer_norm",
    "linear",
    "linear_gelu",
    "linear_ln_supported",
    "linear_residual_layer_norm",
    "linear_supported",
    "pack_weight",
    "short_layer_norm",
    "triton_attention",
    "triton_available",
]
