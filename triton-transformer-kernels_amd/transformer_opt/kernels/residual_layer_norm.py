"""Strict wrappers of the gfx950 fused residual-add + LayerNorm kernel.

``fused_residual_layer_norm`` mirrors the reference wrapper of the same name
(transformer_opt/kernels/residual_layer_norm.py:159-237): same arguments, same
``(residual, normalized)`` result, same fail-closed ``ValueError`` contract,
``RuntimeError`` when the kernel library is missing.  The HIP kernel also
accepts bf16 and fp16 rows (fp32 statistics), which the reference kernel did
not.  ``layer_norm`` is the same kernel without an update or residual output,
used for the first norm of the fused model route; ``short_layer_norm`` keeps
the reference's entry point for rows of exactly 32 values (eight rows per
wavefront here too) on the same kernel.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from .. import _native
from ..config import LAYER_NORM_MAX_WIDTH, SUPPORTED_DTYPES
from .attention import _DTYPE_CODE


def _check_rows(x: torch.Tensor, what: str) -> None:
    if x.ndim < 2:
        raise ValueError(f"{what} must have rank two or higher")
    if x.device.type != "cuda":
        raise ValueError("fused residual LayerNorm requires co-located ROCm device tensors")
    if x.dtype not in SUPPORTED_DTYPES:
        raise ValueError("fused residual LayerNorm supports float32, bfloat16 and float16")
    if not x.is_contiguous():
        raise ValueError("fused residual LayerNorm requires contiguous inputs")


def _check_affine(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor]) -> None:
    width = x.shape[-1]
    if weight is None:
        raise ValueError("fused residual LayerNorm requires an affine weight")
    if weight.shape != (width,) or weight.device != x.device or weight.dtype != x.dtype:
        raise ValueError("weight must match the normalized feature dimension")
    if not weight.is_contiguous():
        raise ValueError("weight must be contiguous")
    if bias is not None:
        if bias.shape != (width,) or bias.device != x.device or bias.dtype != x.dtype:
            raise ValueError("bias must match the normalized feature dimension")
        if not bias.is_contiguous():
            raise ValueError("bias must be contiguous")
    if width > LAYER_NORM_MAX_WIDTH:
        raise ValueError("normalized feature dimension exceeds the fused kernel limit")


def _check_mask(x: torch.Tensor, valid_token_mask: Optional[torch.Tensor]) -> None:
    if valid_token_mask is None:
        return
    if valid_token_mask.shape != x.shape[:-1]:
        raise ValueError("valid_token_mask must match every non-feature dimension")
    if valid_token_mask.dtype is not torch.bool or valid_token_mask.device != x.device:
        raise ValueError("valid_token_mask must be a co-located bool tensor")
    if not valid_token_mask.is_contiguous():
        raise ValueError("valid_token_mask must be contiguous")


def _launch(x, update, weight, bias, eps, mask, residual_out, normalized_out,
            zero_invalid_residual, zero_invalid_normalized) -> None:
    lib = _native.load()
    width = x.shape[-1]
    rows = x.numel() // width
    with torch.cuda.device(x.device):
        stream = torch.cuda.current_stream(x.device).cuda_stream
        status = lib.ttk_residual_layernorm_fwd(
            x.data_ptr(),
            update.data_ptr() if update is not None else None,
            weight.data_ptr(),
            bias.data_ptr() if bias is not None else None,
            mask.data_ptr() if mask is not None else None,
            residual_out.data_ptr() if residual_out is not None else None,
            normalized_out.data_ptr(),
            _DTYPE_CODE[x.dtype], rows, width, float(eps),
            1 if zero_invalid_residual else 0,
            1 if zero_invalid_normalized else 0,
            stream,
        )
    _native.check(status, "HIP residual LayerNorm")


def fused_residual_layer_norm(
    x: torch.Tensor,
    update: torch.Tensor,
    weight: torch.Tensor,
    bias: Optional[torch.Tensor],
    eps: float,
    valid_token_mask: Optional[torch.Tensor] = None,
    *,
    zero_invalid_residual: bool = False,
    zero_invalid_normalized: bool = False,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Return ``(x + update, layer_norm(x + update))`` from one HIP kernel."""
    _native.load()
    if x.shape != update.shape or x.ndim < 2:
        raise ValueError("x and update must have the same rank-two-or-higher shape")
    _check_rows(x, "x")
    if update.device != x.device:
        raise ValueError("fused residual LayerNorm requires co-located ROCm device tensors")
    if update.dtype is not x.dtype:
        raise ValueError("x and update must share a dtype")
    if not update.is_contiguous():
        raise ValueError("fused residual LayerNorm requires contiguous inputs")
    if torch.is_grad_enabled() and (x.requires_grad or update.requires_grad):
        raise ValueError("fused residual LayerNorm is forward-inference only")
    _check_affine(x, weight, bias)
    if (zero_invalid_residual or zero_invalid_normalized) and valid_token_mask is None:
        raise ValueError("invalid-row zeroing requires valid_token_mask")
    _check_mask(x, valid_token_mask)

    residual_out = torch.empty_like(x)
    normalized_out = torch.empty_like(x)
    if x.numel() == 0:
        return residual_out, normalized_out
    _launch(x, update, weight, bias, eps, valid_token_mask, residual_out, normalized_out,
            zero_invalid_residual, zero_invalid_normalized)
    return residual_out, normalized_out


def layer_norm(
    x: torch.Tensor,
    weight: torch.Tensor,
    bias: Optional[torch.Tensor],
    eps: float,
) -> torch.Tensor:
    """``F.layer_norm(x, (N,), weight, bias, eps)`` through the HIP kernel."""
    _native.load()
    _check_rows(x, "x")
    if torch.is_grad_enabled() and x.requires_grad:
        raise ValueError("HIP LayerNorm is forward-inference only")
    _check_affine(x, weight, bias)
    out = torch.empty_like(x)
    if x.numel() == 0:
        return out
    _launch(x, None, weight, bias, eps, None, None, out, False, False)
    return out


def short_layer_norm(
    x: torch.Tensor,
    weight: torch.Tensor,
    bias: Optional[torch.Tensor],
    eps: float,
) -> torch.Tensor:
    """Inference LayerNorm of contiguous float32 rows of exactly 32 values.

    The reference entry point of the same name
    (transformer_opt/kernels/residual_layer_norm.py:129-156) and its
    contract: ``ValueError`` unless ``x`` is a contiguous device float32
    tensor of rank >= 2 with last dimension 32, gradients are disabled and
    ``weight`` (required) and ``bias`` are contiguous ``[32]`` tensors of the
    same device and dtype.  It runs the general HIP LayerNorm kernel, whose
    narrow-row form already gives eight such rows to one wavefront; results
    are within float32 rounding of ``F.layer_norm``, not bit-identical to a
    particular vendor reduction order.
    """
    _native.load()
    if (x.ndim < 2 or x.shape[-1] != 32 or x.dtype != torch.float32 or x.device.type != "cuda"
            or not x.is_contiguous()):
        raise ValueError("short LayerNorm requires contiguous device float32 rows of width 32")
    if torch.is_grad_enabled():
        raise ValueError("short LayerNorm requires disabled gradients")
    for name, tensor in (("weight", weight), ("bias", bias)):
        if tensor is not None and (tensor.shape != (32,) or tensor.device != x.device
                                   or tensor.dtype != x.dtype or not tensor.is_contiguous()):
            raise ValueError(f"{name} must match the normalized feature dimension")
    if weight is None:
        raise ValueError("short LayerNorm requires affine weight")
    return layer_norm(x, weight, bias, eps)
