"""Support envelope and launch description of the gfx950 kernels.

Mirrors the reference's ``transformer_opt/config.py``: the same Q/K/V contract
(``_validate_qkv_contract``, reference config.py:115-140) and a support check
that explains every refusal (reference ``triton_attention_support``,
config.py:143-175).  What changes is the envelope of the hardware path:

* backends are ``auto``, ``hip``, ``triton`` and ``reference``.  The first
  three run the HIP kernel: ``triton`` is the reference's name for its
  forced fused route (config.py:11, dispatch.py:119-132), kept so callers
  that force it land on the kernel that replaces it.  ``reference`` is the
  reference's explicit-math route, run only when named, never by ``auto``.
  There is no SDPA route;
* dtypes are fp32, bf16 and fp16 (the reference stopped at fp16/fp32,
  config.py:17-18);
* sequence length is bounded by the kernel's index range, not by a measured
  8192 (config.py:20): memory is linear in S;
* the reference's per-shape RTX 5070 Ti tile table (config.py:61-112) is
  replaced by the fixed gfx950 tile below.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

ATTENTION_BACKENDS = ("auto", "hip", "triton", "reference")
# Forced backends that name the HIP kernel.
FORCED_BACKENDS = frozenset({"hip", "triton"})
SUPPORTED_HEAD_DIMS = frozenset({8, 16, 32, 64, 128})
SUPPORTED_DTYPES = frozenset({torch.float32, torch.bfloat16, torch.float16})
MAX_SEQUENCE_LENGTH = 1 << 24
LAYER_NORM_MAX_WIDTH = 65536
GFX_ARCH = "gfx950"


@dataclass(frozen=True)
class SupportResult:
    supported: bool
    reason: str


@dataclass(frozen=True)
class AttentionLaunchConfig:
    """Tile of the HIP attention kernel (fixed per head dim and dtype)."""

    block_m: int  # queries per workgroup (4 wavefronts x 32)
    block_n: int  # keys per LDS tile
    num_waves: int
    lds_stages: int


def attention_launch_config(head_dim: int, dtype: torch.dtype = torch.float32) -> AttentionLaunchConfig:
    """Return the tile the HIP kernel uses for ``head_dim`` and ``dtype``.

    fp32 stages K/V tiles of 64 keys (32 for head_dim 128, to stay inside the
    64 KB of LDS that lets two workgroups share a CU); 16-bit types always use
    64-key tiles.  Both are double-buffered.
    """
    if head_dim not in SUPPORTED_HEAD_DIMS:
        raise ValueError(f"head_dim={head_dim} is outside {sorted(SUPPORTED_HEAD_DIMS)}")
    if dtype == torch.float32:
        block_n = 32 if head_dim >= 128 else 64
    else:
        block_n = 64
    return AttentionLaunchConfig(block_m=128, block_n=block_n, num_waves=4, lds_stages=2)


def _validate_qkv_contract(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    valid_token_mask: Optional[torch.Tensor],
) -> Optional[str]:
    """Shape/dtype/device/stride contract; same messages as the reference."""
    if q.ndim != 4:
        return "q, k, and v must have shape [batch, sequence, heads, head_dim]"
    if k.shape != q.shape or v.shape != q.shape:
        return "q, k, and v must have identical shapes"
    if k.dtype != q.dtype or v.dtype != q.dtype:
        return "q, k, and v must have identical dtypes"
    if k.device != q.device or v.device != q.device:
        return "q, k, and v must be on the same device"
    if q.shape[1] <= 0 or q.shape[2] <= 0 or q.shape[3] <= 0:
        return "sequence length, head count, and head dimension must be positive"
    if q.stride(-1) != 1 or k.stride(-1) != 1 or v.stride(-1) != 1:
        return "the head-dimension stride must be 1"
    if valid_token_mask is not None:
        if valid_token_mask.shape != q.shape[:2]:
            return "valid_token_mask must have shape [batch, sequence]"
        if valid_token_mask.dtype is not torch.bool:
            return "valid_token_mask must have dtype torch.bool"
        if valid_token_mask.device != q.device:
            return "valid_token_mask must be on the q/k/v device"
    return None


def hip_attention_support(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    valid_token_mask: Optional[torch.Tensor] = None,
) -> SupportResult:
    """Explain whether the HIP forward kernel can run on these inputs."""
    contract_error = _validate_qkv_contract(q, k, v, valid_token_mask)
    if contract_error is not None:
        return SupportResult(False, contract_error)
    if q.device.type != "cuda":
        return SupportResult(False, "HIP attention requires ROCm device tensors (device type 'cuda')")
    if q.dtype not in SUPPORTED_DTYPES:
        return SupportResult(False, "HIP attention supports float32, bfloat16 and float16")
    if q.shape[-1] not in SUPPORTED_HEAD_DIMS:
        return SupportResult(
            False,
            f"head_dim={q.shape[-1]} is outside {sorted(SUPPORTED_HEAD_DIMS)}",
        )
    if q.shape[1] > MAX_SEQUENCE_LENGTH:
        return SupportResult(
            False,
            f"seq_len={q.shape[1]} exceeds the kernel maximum {MAX_SEQUENCE_LENGTH}",
        )
    if torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad):
        return SupportResult(False, "HIP attention is forward-inference only")
    arch = device_arch(q.device)
    if arch != GFX_ARCH:
        return SupportResult(False, f"device architecture {arch} is not {GFX_ARCH}")
    return SupportResult(True, f"inside the {GFX_ARCH} HIP forward envelope")


_ARCH_CACHE: dict = {}


def device_arch(device: torch.device) -> str:
    """gfx architecture name (without feature suffixes) of a ROCm device."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    arch = _ARCH_CACHE.get(index)
    if arch is None:
        name = getattr(torch.cuda.get_device_properties(index), "gcnArchName", "") or ""
        arch = name.split(":")[0]
        _ARCH_CACHE[index] = arch
    return arch


# Drop-in name of the reference's support check (config.py:143).
triton_attention_support = hip_attention_support
