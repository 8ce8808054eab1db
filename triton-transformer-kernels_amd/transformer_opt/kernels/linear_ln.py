"""Output projection + residual add + LayerNorm on one gfx950 HIP kernel.

``linear_residual_layer_norm(a, packed_weight, bias, x, ln_weight, ln_bias,
eps)`` returns ``(r, y)`` with

    r = x + F.linear(a, W, bias)        (the projection rounded to x's dtype,
                                          the sum rounded again)
    y = F.layer_norm(r, (1024,), ln_weight, ln_bias, eps)

- the attention output projection of an encoder block followed by the
reference's fused residual + LayerNorm (transformer_opt/submission.py:
497-505 with fused_residual_layer_norm, residual_layer_norm.py:159-237), as
one kernel (``ttk_linear_residual_ln_fwd``): the projection never goes
through HBM and the LayerNorm launch is gone.  bf16 and fp16, rows of 1024
features, the weight packed once by ``pack_weight``.

``linear_ln_supported`` reports whether a call fits the kernel's envelope;
unsupported inputs raise ``ValueError`` and a missing library
``RuntimeError``.
"""

from __future__ import annotations

import threading
from collections import OrderedDict
from typing import Optional, Tuple

import torch

from .. import _native

_CODES = {torch.bfloat16: _native.TTK_BF16, torch.float16: _native.TTK_F16}
WIDTH = 1024

# One workspace per (device, stream), most recently used last, zero-filled
# when made; every launch leaves its counters zero, so a buffer serves every
# later launch on its stream.  During graph capture the buffer comes from the
# graph's pool and is cleared inside the graph (a fill kernel).
_WORKSPACES: "OrderedDict[tuple, torch.Tensor]" = OrderedDict()
_MAX_WORKSPACES = 8
_WS_LOCK = threading.Lock()


def _workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    if torch.cuda.is_current_stream_capturing():
        return torch.zeros(nbytes, dtype=torch.uint8, device=device)
    key = (device.index, torch.cuda.current_stream(device).cuda_stream)
    with _WS_LOCK:
        ws = _WORKSPACES.pop(key, None)
        if ws is None or ws.numel() < nbytes:
            ws = torch.zeros(nbytes, dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
        while len(_WORKSPACES) > _MAX_WORKSPACES:
            _WORKSPACES.popitem(last=False)
    return ws


def pack_weight(weight: torch.Tensor) -> torch.Tensor:
    """``weight`` [N, K] (bf16/fp16 on a ROCm device) in the MFMA fragment
    order the kernel reads, as a new contiguous tensor of N * K elements."""
    if weight.device.type != "cuda" or weight.dtype not in _CODES or weight.ndim != 2:
        raise ValueError("pack_weight needs a 2-D bfloat16 or float16 tensor on a ROCm device")
    n, k = weight.shape
    w = weight.contiguous()
    if w.data_ptr() % 16:
        w = w.clone()
    packed = torch.empty(n * k, dtype=w.dtype, device=w.device)
    lib = _native.load()
    with torch.cuda.device(w.device):
        status = lib.ttk_linear_pack_weight(w.data_ptr(), packed.data_ptr(), _CODES[w.dtype], n, k, k,
                                            torch.cuda.current_stream(w.device).cuda_stream)
    _native.check(status, "pack weight")
    return packed


def linear_ln_supported(a: torch.Tensor, packed_weight: torch.Tensor, bias: Optional[torch.Tensor],
                        x: torch.Tensor, ln_weight: torch.Tensor,
                        ln_bias: Optional[torch.Tensor]) -> Optional[str]:
    """None when the kernel takes this call, else the reason it does not."""
    tensors = [a, packed_weight, x, ln_weight] + [t for t in (bias, ln_bias) if t is not None]
    if a.device.type != "cuda" or any(t.device != a.device for t in tensors):
        return "inputs must be on one ROCm device"
    if a.dtype not in _CODES or any(t.dtype != a.dtype for t in tensors):
        return "all tensors must share one dtype, bfloat16 or float16"
    if x.shape[-1:] != (WIDTH,) or ln_weight.shape != (WIDTH,):
        return f"the normalised width must be {WIDTH}"
    if a.shape[:-1] != x.shape[:-1] or a.ndim < 2:
        return "a and x must have the same leading dimensions"
    in_features = a.shape[-1]
    if in_features % 128 != 0 or packed_weight.numel() != WIDTH * in_features:
        return "in_features must be a multiple of 128 and the packed weight [1024, in_features]"
    if (bias is not None and bias.shape != (WIDTH,)) or (ln_bias is not None and ln_bias.shape != (WIDTH,)):
        return "bias and ln_bias must be [1024]"
    if x.numel() * 2 >= 1 << 31:
        return "operands too large for 32-bit offsets"
    return None


def _aligned(t: torch.Tensor) -> torch.Tensor:
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def workspace_bytes(rows: int) -> int:
    """Bytes of the workspace a call over ``rows`` rows needs."""
    return int(_native.load().ttk_linear_residual_ln_workspace_size(rows))


def linear_residual_layer_norm(a: torch.Tensor, packed_weight: torch.Tensor, bias: Optional[torch.Tensor],
                               x: torch.Tensor, ln_weight: torch.Tensor, ln_bias: Optional[torch.Tensor],
                               eps: float, *, max_polls: int = -1,
                               workspace: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """``(x + F.linear(a, W, bias), layer_norm(that))`` in one kernel, W as
    packed by ``pack_weight``.  ``max_polls`` bounds how long the first
    workgroup of a row block waits for the second before handing its half
    over (negative: the library default; 0 always hands over - the same
    result by the slower route).  ``workspace``: a uint8 device tensor of at
    least ``workspace_bytes(rows)`` bytes whose first
    ``_native.LINEAR_LN_WS_COUNTER_BYTES`` are zero (every call leaves them
    zero), for callers that run several launches in order on one stream;
    by default one is kept per (device, stream)."""
    reason = linear_ln_supported(a, packed_weight, bias, x, ln_weight, ln_bias)
    if reason is not None:
        raise ValueError(f"unsupported HIP linear + LayerNorm input: {reason}")
    lib = _native.load()
    a2, wp, x2, g = (_aligned(t) for t in (a, packed_weight, x, ln_weight))
    b = None if bias is None else bias.contiguous()
    beta = None if ln_bias is None else _aligned(ln_bias)
    rows = x2.numel() // WIDTH
    r = torch.empty_like(x2)
    y = torch.empty_like(x2)
    if rows == 0:
        return r, y
    nbytes = int(lib.ttk_linear_residual_ln_workspace_size(rows))
    if workspace is not None and (workspace.dtype != torch.uint8 or workspace.device != a.device
                                  or not workspace.is_contiguous() or workspace.numel() < nbytes):
        raise ValueError(f"workspace must be a contiguous uint8 tensor of {nbytes} bytes on a's device")
    with torch.cuda.device(a.device):
        ws = _workspace(a.device, nbytes) if workspace is None else workspace
        in_features = a2.shape[-1]
        status = lib.ttk_linear_residual_ln_fwd(
            a2.data_ptr(), wp.data_ptr(), None if b is None else b.data_ptr(), x2.data_ptr(), g.data_ptr(),
            None if beta is None else beta.data_ptr(), r.data_ptr(), y.data_ptr(), ws.data_ptr(), ws.numel(),
            _CODES[a.dtype], rows, WIDTH, in_features, in_features, WIDTH, WIDTH, WIDTH, float(eps),
            int(max_polls), torch.cuda.current_stream(a.device).cuda_stream)
    _native.check(status, "linear + LayerNorm")
    return r, y
