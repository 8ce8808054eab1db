"""Strict wrapper of the gfx950 HIP fused attention kernel.

Mirrors the reference's ``triton_attention`` (transformer_opt/kernels/
attention.py:268-360): validate the support contract, allocate the output with
torch, pick the default scale ``head_dim ** -0.5``, and launch on torch's
current stream.  Unsupported inputs raise; nothing falls back.
"""

from __future__ import annotations

import threading
from collections import OrderedDict
from typing import Optional

import torch

from .. import _native
from ..config import hip_attention_support

_DTYPE_CODE = {
    torch.float32: _native.TTK_F32,
    torch.bfloat16: _native.TTK_BF16,
    torch.float16: _native.TTK_F16,
}


def hip_available() -> bool:
    """True when a ROCm device is visible and the HIP library loads."""
    return torch.cuda.is_available() and _native.available()


_WS_SIZES: dict = {}
# One workspace per (device, stream), most recently used last; at most
# _MAX_WORKSPACES are kept.  Dropping one is safe: its memory returns to the
# caching allocator of the stream it was allocated and used on, behind that
# stream's pending launches.
_WORKSPACES: "OrderedDict[tuple, torch.Tensor]" = OrderedDict()
_MAX_WORKSPACES = 8
_WS_LOCK = threading.Lock()


def _workspace_bytes(lib, dtype_code: int, batch: int, seq_len: int, heads: int, head_dim: int,
                     causal: bool, device_index: int) -> int:
    key = (dtype_code, batch, seq_len, heads, head_dim, causal, device_index)
    nbytes = _WS_SIZES.get(key)
    if nbytes is None:
        nbytes = int(lib.ttk_attention_workspace_size(dtype_code, batch, seq_len, heads, head_dim,
                                                      1 if causal else 0))
        _WS_SIZES[key] = nbytes
    return nbytes


def _workspace(device: torch.device, nbytes: int) -> Optional[torch.Tensor]:
    """Workspace of the key-split attention schedule for the current stream.

    It starts with a fixed block of arrival counters (the same bytes for
    every launch shape) that must be zero before a launch; every launch
    leaves it zero, and the partial states after it need no initialisation,
    so one buffer serves launches of any shapes in any order.  Outside graph
    capture each (device, stream) keeps one zero-filled buffer, replaced by a
    larger zero-filled one when a launch needs more; launches on one stream
    never overlap.  During a capture the buffer comes from the graph's
    memory pool and its counters are cleared inside the graph (a fill
    kernel, not a memset node), so every replay starts from zero.
    """
    if nbytes == 0:
        return None
    if torch.cuda.is_current_stream_capturing():
        ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
        ws[:_native.ATTENTION_WS_COUNTER_BYTES].zero_()
        return ws
    key = (device.index, torch.cuda.current_stream(device).cuda_stream)
    with _WS_LOCK:
        ws = _WORKSPACES.pop(key, None)
        if ws is None or ws.numel() < nbytes:
            ws = torch.zeros(nbytes, dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
        while len(_WORKSPACES) > _MAX_WORKSPACES:
            _WORKSPACES.popitem(last=False)
    return ws


def _vector_ready(t: torch.Tensor) -> bool:
    """Rows start on 16-byte boundaries (the kernel's 128-bit accesses)."""
    es = t.element_size()
    return t.data_ptr() % 16 == 0 and all((s * es) % 16 == 0 for s in t.stride()[:3])


def hip_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    valid_token_mask: Optional[torch.Tensor] = None,
    *,
    causal: bool = False,
    scale: Optional[float] = None,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Run the HIP fused attention and return the ``[B, S, H, D]`` output.

    Strict low-level wrapper: unsupported inputs raise ``ValueError``, a
    missing library raises ``RuntimeError``.  Use
    ``transformer_opt.dispatch.attention_forward`` for the audited entry point.
    """
    lib = _native.load()
    support = hip_attention_support(q, k, v, valid_token_mask)
    if not support.supported:
        raise ValueError(f"unsupported HIP attention input: {support.reason}")

    # Arbitrary B/S/H strides are part of the contract; rows that are not
    # 16-byte aligned are copied into fresh (aligned) storage so the kernel
    # keeps its vector loads - also for a contiguous view at an odd storage
    # offset, which ``contiguous()`` would return unchanged.
    if not _vector_ready(q):
        q = q.clone(memory_format=torch.contiguous_format)
    if not _vector_ready(k):
        k = k.clone(memory_format=torch.contiguous_format)
    if not _vector_ready(v):
        v = v.clone(memory_format=torch.contiguous_format)

    batch, seq_len, num_heads, head_dim = q.shape
    if out is None:
        out = torch.empty((batch, seq_len, num_heads, head_dim), dtype=q.dtype, device=q.device)
    elif out.shape != q.shape or out.dtype != q.dtype or out.device != q.device or out.stride(-1) != 1 \
            or not _vector_ready(out):
        raise ValueError("out must be a [B, S, H, D] tensor like q with 16-byte aligned rows")
    if batch == 0:
        return out

    softmax_scale = head_dim ** -0.5 if scale is None else float(scale)
    mask_ptr = None
    mask_strides = None
    if valid_token_mask is not None:
        mask_ptr = valid_token_mask.data_ptr()
        mask_strides = _native.strides2(valid_token_mask.stride())

    dtype_code = _DTYPE_CODE[q.dtype]
    with torch.cuda.device(q.device):
        nbytes = _workspace_bytes(lib, dtype_code, batch, seq_len, num_heads, head_dim, causal,
                                  q.device.index)
        ws = _workspace(q.device, nbytes)
        stream = torch.cuda.current_stream(q.device).cuda_stream
        status = lib.ttk_attention_fwd_ws(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), mask_ptr, out.data_ptr(),
            dtype_code,
            batch, seq_len, num_heads, head_dim,
            _native.strides3(q.stride()[:3]),
            _native.strides3(k.stride()[:3]),
            _native.strides3(v.stride()[:3]),
            mask_strides,
            _native.strides3(out.stride()[:3]),
            softmax_scale, 1 if causal else 0,
            None if ws is None else ws.data_ptr(), nbytes, stream,
        )
    _native.check(status, "HIP attention")
    return out


# The reference's names for the same entry points (its kernels package exports
# triton_attention and triton_available, transformer_opt/kernels/__init__.py),
# so callers written against it run unchanged; there is no Triton here.
triton_attention = hip_attention
triton_available = hip_available
