"""Fused Linear + exact GELU on the gfx950 HIP kernel.

``linear_gelu(x, weight, bias)`` returns ``F.gelu(F.linear(x, weight, bias),
approximate="none")`` for bf16 / fp16 inputs in one kernel: the product
accumulates in fp32, bias and GELU act on the fp32 value, and the result is
rounded once (the unfused route rounds the GEMM output first).  It stands in
for the model's ``F.gelu(layer.ffn_in(...), approximate="none")`` (reference
transformer_opt/submission.py:507).  Unsupported inputs raise ``ValueError``;
a missing library raises ``RuntimeError``.  ``linear_gelu_supported`` says
whether the kernel takes a given call, so a caller can keep the library GEMM
for the rest (fp32 above all, whose library GEMM already runs near the fp32
MFMA peak).
"""

from __future__ import annotations

from typing import Optional

import torch

from .. import _native
from .attention import _DTYPE_CODE


def linear_gelu_supported(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor]) -> bool:
    if x.dtype not in (torch.bfloat16, torch.float16) or x.device.type != "cuda":
        return False
    if weight.ndim != 2 or x.ndim < 1 or x.shape[-1] != weight.shape[1]:
        return False
    if weight.dtype != x.dtype or weight.device != x.device or not weight.is_contiguous():
        return False
    if bias is not None and (bias.shape != (weight.shape[0],) or bias.dtype != x.dtype
                             or bias.device != x.device or not bias.is_contiguous()):
        return False
    out_features, in_features = weight.shape
    return in_features % 64 == 0 and out_features % 4 == 0


def linear_gelu(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """gelu(x @ weight.T + bias) with the exact (erf) GELU, for bf16 / fp16."""
    lib = _native.load()
    if not linear_gelu_supported(x, weight, bias):
        raise ValueError("linear_gelu needs bf16/fp16 co-located contiguous tensors, "
                         "in_features a multiple of 64 and out_features a multiple of 4")
    rows = x.reshape(-1, x.shape[-1])
    if not rows.is_contiguous() or rows.data_ptr() % 16:
        rows = rows.contiguous()
    out_features, in_features = weight.shape
    y = torch.empty((rows.shape[0], out_features), device=x.device, dtype=x.dtype)
    status = lib.ttk_linear_gelu_fwd(
        rows.data_ptr(), weight.data_ptr(), None if bias is None else bias.data_ptr(), y.data_ptr(),
        _DTYPE_CODE[x.dtype], rows.shape[0], out_features, in_features,
        rows.stride(0), weight.stride(0), y.stride(0),
        torch.cuda.current_stream(x.device).cuda_stream,
    )
    _native.check(status, "linear_gelu")
    return y.view(*x.shape[:-1], out_features)
