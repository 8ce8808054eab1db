"""Residual + LayerNorm oracle (test infrastructure only; see oracle/__init__.py)."""

from __future__ import annotations

from typing import Optional, Tuple

import numpy as np
import torch
import torch.nn.functional as F


def explicit_residual_layer_norm(
    x: torch.Tensor,
    update: Optional[torch.Tensor],
    weight: torch.Tensor,
    bias: Optional[torch.Tensor],
    eps: float,
    valid_token_mask: Optional[torch.Tensor] = None,
    *,
    zero_invalid_residual: bool = False,
    zero_invalid_normalized: bool = False,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Explicit torch ops for the fused kernel's contract.

    Restates ``_residual_layer_norm_fwd`` (reference transformer_opt/kernels/
    residual_layer_norm.py:95-126) exactly as the reference test checks it
    (tests/test_gpu_residual_layer_norm.py:38-63): r = x + update (eager add
    in the tensor dtype), invalid rows of r zeroed when requested, then
    ``F.layer_norm`` over the last dimension, invalid rows of the result
    zeroed when requested.  ``update=None`` means r = x.
    """
    residual = x + update if update is not None else x.clone()
    if zero_invalid_residual:
        residual = residual.masked_fill(~valid_token_mask[..., None], 0)
    normalized = F.layer_norm(residual, (x.shape[-1],), weight, bias, eps)
    if zero_invalid_normalized:
        normalized = normalized.masked_fill(~valid_token_mask[..., None], 0)
    return residual, normalized


def brute_force_layer_norm_f64(r, weight, bias, eps) -> np.ndarray:
    """Independent float64 LayerNorm from the definition (biased variance).

    y = (r - mean) / sqrt(mean((r - mean)^2) + eps) * weight + bias, per row
    of the last dimension.
    """
    r = np.asarray(r, dtype=np.float64)
    w = np.asarray(weight, dtype=np.float64)
    b = np.zeros_like(w) if bias is None else np.asarray(bias, dtype=np.float64)
    mean = r.mean(axis=-1, keepdims=True)
    var = ((r - mean) ** 2).mean(axis=-1, keepdims=True)
    return (r - mean) / np.sqrt(var + eps) * w + b
