"""Linear layer with the exact GELU in its epilogue, on the gfx950 HIP kernel.

``linear_gelu(x, weight, bias)`` returns what the reference's FFN input
computes in 16-bit torch, ``F.gelu(F.linear(x, weight, bias))``
(transformer_opt/submission.py:507; benchmarks/torch_transformer_benchmark.py:
95-97): the linear output rounded to x's dtype, then the exact (erf) GELU of
that value rounded again - as one kernel, the GELU applied in the GEMM's
epilogue (``ttk_linear_fwd``).  ``linear(x, weight, bias)`` is the same kernel
without the activation.

bf16 and fp16 only (fp32 keeps the library GEMM and the elementwise GELU
kernel).  ``linear_supported`` reports whether a call fits the kernel's
envelope; unsupported inputs raise ``ValueError`` and a missing library
``RuntimeError``.
"""

from __future__ import annotations

from typing import Optional

import torch

from .. import _native

_CODES = {torch.bfloat16: _native.TTK_BF16, torch.float16: _native.TTK_F16}


def linear_supported(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor]) -> Optional[str]:
    """None when the kernel takes this call, else the reason it does not."""
    if x.device.type != "cuda" or weight.device != x.device:
        return "inputs must be on one ROCm device"
    if x.dtype not in _CODES or weight.dtype != x.dtype:
        return "x and weight must both be bfloat16 or both float16"
    if weight.ndim != 2 or x.ndim < 1 or x.shape[-1] != weight.shape[1]:
        return "weight must be [out_features, in_features] with in_features == x.shape[-1]"
    out_features, in_features = weight.shape
    if in_features % 128 != 0 or in_features < 256:
        return "in_features must be a multiple of 128 and at least 256"
    if out_features % 32 != 0:
        return "out_features must be a multiple of 32"
    if bias is not None and (bias.shape != (out_features,) or bias.dtype != x.dtype
                             or bias.device != x.device):
        return "bias must be [out_features] of x's dtype on x's device"
    rows = x.numel() // max(1, in_features)
    if (rows * in_features * 2 >= 1 << 32 or out_features * in_features * 2 >= 1 << 32
            or rows * out_features * 2 >= 1 << 31):
        return "operands too large for 32-bit offsets"
    return None


def _run(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor], activation: int) -> torch.Tensor:
    reason = linear_supported(x, weight, bias)
    if reason is not None:
        raise ValueError(f"unsupported HIP linear input: {reason}")
    lib = _native.load()
    # 16-byte aligned rows for the copies (4 bytes for the bias): contiguous
    # views at an odd storage offset are copied.
    xs, w = x.contiguous(), weight.contiguous()
    if xs.data_ptr() % 16:
        xs = xs.clone()
    if w.data_ptr() % 16:
        w = w.clone()
    b = None if bias is None else bias.contiguous()
    if b is not None and b.data_ptr() % 4:
        b = b.clone()
    out_features, in_features = w.shape
    rows = xs.numel() // in_features
    y = torch.empty(*x.shape[:-1], out_features, dtype=x.dtype, device=x.device)
    # The launcher sizes its grid from the current device's CU count.
    with torch.cuda.device(x.device):
        status = lib.ttk_linear_fwd(xs.data_ptr(), w.data_ptr(), None if b is None else b.data_ptr(),
                                    y.data_ptr(), _CODES[x.dtype], rows, out_features, in_features,
                                    in_features, in_features, out_features, activation,
                                    torch.cuda.current_stream(x.device).cuda_stream)
    _native.check(status, "linear")
    return y


def linear_gelu(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``F.gelu(F.linear(x, weight, bias), approximate="none")`` in one kernel."""
    return _run(x, weight, bias, _native.TTK_ACT_GELU)


def linear(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``F.linear(x, weight, bias)`` on the same kernel (no activation)."""
    return _run(x, weight, bias, _native.TTK_ACT_NONE)
