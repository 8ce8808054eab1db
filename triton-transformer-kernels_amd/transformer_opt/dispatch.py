"""Auditable attention dispatch onto the gfx950 HIP kernel.

Mirrors the reference's ``transformer_opt/dispatch.py``: the same
``attention_forward(q, k, v, valid_token_mask, *, causal, scale, backend)``
signature returning ``(output, AttentionDispatch(requested, selected,
reason))`` and the same exception contract - an unknown backend is a
``ValueError`` (dispatch.py:26-30), a forced backend that cannot run is a
``RuntimeError`` when the hardware path is absent (dispatch.py:120-121) and a
``ValueError`` when the inputs are unsupported (dispatch.py:122-123).

Routes:

* ``auto`` and ``hip`` run the HIP kernel or raise with the support reason;
  ``auto`` never selects anything else (the reference's ``auto`` fell back to
  SDPA or explicit math, dispatch.py:134-161; here there is no fallback).
* ``triton`` - the reference's forced fused route (dispatch.py:119-132) -
  runs the HIP kernel that replaces it and is recorded as
  ``selected="hip"``; its errors keep the reference's "Triton attention was
  forced" wording so callers matching on it still match.
* ``reference`` - the reference's explicit-math route (dispatch.py:69-96,
  145-152), reached only when a caller names it: plain torch operations on
  the caller's device, recorded as ``selected="reference"``.  Its callers are
  the reference's own comparisons, which force it as the slow, exact side.
  There is no SDPA route (the north star forbids it).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional, Tuple

import torch

from .config import ATTENTION_BACKENDS, hip_attention_support
from .kernels.attention import hip_attention, hip_available


@dataclass(frozen=True)
class AttentionDispatch:
    requested: str
    selected: str
    reason: str


def _validate_backend(backend: str) -> None:
    if backend not in ATTENTION_BACKENDS:
        raise ValueError(
            f"attention backend must be one of {ATTENTION_BACKENDS}, got {backend!r}"
        )


def _route_phrase(backend: str) -> str:
    if backend == "triton":
        return "Triton attention was forced (it runs on the HIP kernel)"
    return f"HIP attention was {'forced' if backend == 'hip' else 'requested'}"


def explicit_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    valid_token_mask: Optional[torch.Tensor],
    causal: bool,
    scale: Optional[float],
) -> torch.Tensor:
    """The ``reference`` route: attention as explicit torch operations.

    Same dtype boundaries as the reference's explicit route
    (dispatch.py:69-96): scores ``Q.K^T`` in the input dtype, scaled, masked
    with ``-inf`` (future keys when causal, invalid keys), a float32 softmax,
    the probabilities cast back to the input dtype, then ``P.V``.  A row with
    no allowed key gives NaN there, as in the reference.  Every operand of a
    batched product is made contiguous first (the head-major copies and
    ``K^T`` itself), so no product takes a transposed view.
    """
    heads_first = (0, 2, 1, 3)
    qh = q.permute(heads_first).contiguous()
    kt = k.permute(0, 2, 3, 1).contiguous()  # [B, H, D, S]
    vh = v.permute(heads_first).contiguous()
    scores = torch.matmul(qh, kt)
    scores = scores * (q.shape[-1] ** -0.5 if scale is None else scale)
    blocked = None
    if causal:
        seq_len = q.shape[1]
        blocked = torch.ones(seq_len, seq_len, dtype=torch.bool, device=q.device).triu(1)
    if valid_token_mask is not None:
        invalid = ~valid_token_mask.to(torch.bool)[:, None, None, :]
        blocked = invalid if blocked is None else (invalid | blocked)
    if blocked is not None:
        scores = scores.masked_fill(blocked, float("-inf"))
    weights = torch.softmax(scores.float(), dim=-1).to(q.dtype)
    return torch.matmul(weights, vh).permute(heads_first).contiguous()


def attention_forward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    valid_token_mask: Optional[torch.Tensor] = None,
    *,
    causal: bool = False,
    scale: Optional[float] = None,
    backend: str = "auto",
) -> Tuple[torch.Tensor, AttentionDispatch]:
    """Execute attention on the route ``backend`` names; return the output and its record."""
    _validate_backend(backend)
    if backend == "reference":
        output = explicit_attention(q, k, v, valid_token_mask, causal, scale)
        return output, AttentionDispatch(backend, "reference", "explicit reference backend")
    route = _route_phrase(backend)
    if not hip_available():
        raise RuntimeError(f"{route} but ROCm/the HIP kernel library is unavailable")
    support = hip_attention_support(q, k, v, valid_token_mask)
    if not support.supported:
        raise ValueError(f"{route} but unsupported: {support.reason}")
    output = hip_attention(q, k, v, valid_token_mask, causal=causal, scale=scale)
    return output, AttentionDispatch(backend, "hip", support.reason)
