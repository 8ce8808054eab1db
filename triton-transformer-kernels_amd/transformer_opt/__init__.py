"""MI355X (gfx950) HIP kernels behind the reference's ``transformer_opt`` surface.

Drop-in for the hot path of jared-makes-stuff/Triton-Transformer-Kernels:
fused flash-style attention and fused residual-add + LayerNorm, hand-written
for CDNA4 and reached through a C ABI (include/ttk_hip.h).
"""

from .config import ATTENTION_BACKENDS, hip_attention_support, triton_attention_support
from .dispatch import AttentionDispatch, attention_forward

__all__ = [
    "ATTENTION_BACKENDS",
    "AttentionDispatch",
    "attention_forward",
    "hip_attention_support",
    "triton_attention_support",
]
