"""Exact (erf) GELU on the gfx950 HIP kernel.

``gelu(x)`` returns ``F.gelu(x, approximate="none")`` for fp32 / bf16 / fp16
CUDA tensors, computed in fp32 and rounded once to the tensor's dtype;
``gelu_(x)`` overwrites ``x``.  It is the encoder FFN's GELU pass
(reference transformer_opt/submission.py:507) as one bandwidth-bound kernel.
Unsupported inputs raise ``ValueError``; a missing library raises
``RuntimeError``.
"""

from __future__ import annotations

import torch

from .. import _native
from .attention import _DTYPE_CODE


def _check(x: torch.Tensor) -> None:
    if x.device.type != "cuda" or x.dtype not in _DTYPE_CODE:
        raise ValueError("gelu needs a CUDA tensor of float32, bfloat16 or float16")


def _launch(src: torch.Tensor, dst: torch.Tensor) -> None:
    lib = _native.load()
    with torch.cuda.device(src.device):
        status = lib.ttk_gelu_fwd(src.data_ptr(), dst.data_ptr(), _DTYPE_CODE[src.dtype], src.numel(),
                                  torch.cuda.current_stream(src.device).cuda_stream)
    _native.check(status, "gelu")


def gelu(x: torch.Tensor) -> torch.Tensor:
    """gelu(x) with the exact (erf) form, as a new tensor."""
    _check(x)
    src = x.contiguous()
    out = torch.empty_like(src)
    _launch(src, out)
    return out.view(x.shape)


def gelu_(x: torch.Tensor) -> torch.Tensor:
    """In-place exact GELU of a contiguous tensor; returns x."""
    _check(x)
    if not x.is_contiguous():
        raise ValueError("gelu_ needs a contiguous tensor")
    _launch(x, x)
    return x
