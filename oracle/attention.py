"""Explicit attention oracle (test infrastructure only; see oracle/__init__.py)."""

from __future__ import annotations

import math
from typing import Optional

import numpy as np
import torch


def explicit_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    valid_token_mask: Optional[torch.Tensor] = None,
    causal: bool = False,
    scale: Optional[float] = None,
) -> torch.Tensor:
    """The reference's explicit attention over BSHD inputs.

    Restates ``_reference_attention`` (reference transformer_opt/dispatch.py:
    69-96), itself the organizer's ``BaselineSelfAttention`` math
    (benchmarks/torch_transformer_benchmark.py:97-111): scores =
    (Q K^T) * scale in the input dtype, -inf on future keys (causal) and on
    invalid keys, softmax in fp32, probabilities cast back to the input dtype,
    then P V.  A query with no allowed key yields NaN here, as in the
    reference.
    """
    qh = q.transpose(1, 2).contiguous()
    kh = k.transpose(1, 2).contiguous()
    vh = v.transpose(1, 2).contiguous()
    scores = torch.matmul(qh, kh.transpose(-2, -1).contiguous())
    scores = scores * (q.shape[-1] ** -0.5 if scale is None else scale)
    if causal:
        seq_len = q.shape[1]
        future = torch.ones((seq_len, seq_len), dtype=torch.bool, device=q.device).triu(diagonal=1)
        scores = scores.masked_fill(future, float("-inf"))
    if valid_token_mask is not None:
        scores = scores.masked_fill(~valid_token_mask[:, None, None, :], float("-inf"))
    probabilities = torch.softmax(scores.float(), dim=-1).to(dtype=q.dtype)
    output = torch.matmul(probabilities, vh)
    return output.transpose(1, 2).contiguous()


def _no_allowed_key(seq_len: int, valid_token_mask: Optional[torch.Tensor], causal: bool,
                    batch: int) -> Optional[torch.Tensor]:
    """[B, S] bool: query rows whose allowed-key set is empty."""
    if valid_token_mask is None:
        return None
    if causal:
        # Query s sees keys 0..s: empty iff no valid key at or before s.
        seen = torch.cumsum(valid_token_mask.to(torch.int64), dim=1)
        return seen == 0
    any_valid = valid_token_mask.any(dim=1, keepdim=True)
    return (~any_valid).expand(batch, seq_len)


def kernel_contract_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    valid_token_mask: Optional[torch.Tensor] = None,
    causal: bool = False,
    scale: Optional[float] = None,
) -> torch.Tensor:
    """Explicit attention with the kernel's all-masked-row contract.

    Identical to :func:`explicit_attention` except that a query row with no
    allowed key is exactly zero instead of NaN (reference
    transformer_opt/kernels/attention.py:253-254; pinned by the reference
    test tests/test_gpu_attention.py:114-128).
    """
    out = explicit_attention(q, k, v, valid_token_mask, causal, scale)
    empty = _no_allowed_key(q.shape[1], valid_token_mask, causal, q.shape[0])
    if empty is not None and bool(empty.any()):
        out = out.masked_fill(empty[:, :, None, None], 0)
    return out


def chunked_kernel_contract_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    valid_token_mask: Optional[torch.Tensor] = None,
    causal: bool = False,
    scale: Optional[float] = None,
    *,
    heads: Optional[list] = None,
    query_rows: Optional[slice] = None,
) -> torch.Tensor:
    """:func:`kernel_contract_attention` evaluated one (batch, head) at a time.

    Row-for-row the same arithmetic (one query row only ever meets its own
    score row), but the [S, S] score block of one head is the largest
    temporary, so large shapes fit in host memory.  ``heads`` selects
    (b, h) pairs and ``query_rows`` a query slice; the result holds only the
    selected rows, as a [len(heads), rows, D] tensor when ``heads`` is given.
    """
    batch, seq_len, num_heads, head_dim = q.shape
    pairs = heads if heads is not None else [(b, h) for b in range(batch) for h in range(num_heads)]
    rows = query_rows if query_rows is not None else slice(0, seq_len)
    sc = head_dim ** -0.5 if scale is None else scale
    results = []
    for b, h in pairs:
        qh = q[b, rows, h, :].contiguous()
        kh = k[b, :, h, :].contiguous()
        vh = v[b, :, h, :].contiguous()
        scores = torch.matmul(qh, kh.transpose(0, 1).contiguous()) * sc
        qpos = torch.arange(seq_len)[rows]
        allowed = torch.ones((qh.shape[0], seq_len), dtype=torch.bool)
        if causal:
            allowed &= torch.arange(seq_len)[None, :] <= qpos[:, None]
        if valid_token_mask is not None:
            allowed &= valid_token_mask[b][None, :].to(torch.bool).cpu()
        scores = scores.masked_fill(~allowed, float("-inf"))
        probs = torch.softmax(scores.float(), dim=-1).to(q.dtype)
        out = torch.matmul(probs, vh)
        out = out.masked_fill(~allowed.any(dim=1)[:, None], 0)
        results.append(out)
    return torch.stack(results)


def brute_force_attention_f64(q, k, v, valid_token_mask=None, causal=False, scale=None) -> np.ndarray:
    """Independent float64 textbook attention (row by row, max-shifted softmax).

    Written from the definition, not from the reference code, to pin the
    restatement above: out[b,s,h] = sum_t softmax_t(scale * q.k_t) v_t over
    allowed t; rows without an allowed key are zero.  Inputs are array-likes
    of shape [B, S, H, D]; the result is float64.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    batch, seq_len, num_heads, head_dim = q.shape
    sc = head_dim ** -0.5 if scale is None else scale
    mask = None if valid_token_mask is None else np.asarray(valid_token_mask, dtype=bool)
    out = np.zeros_like(q)
    for b in range(batch):
        for h in range(num_heads):
            for s in range(seq_len):
                keys = [t for t in range(seq_len)
                        if (not causal or t <= s) and (mask is None or mask[b, t])]
                if not keys:
                    continue
                logits = np.array([sc * np.dot(q[b, s, h], k[b, t, h]) for t in keys])
                weights = np.exp(logits - logits.max())
                weights /= weights.sum()
                out[b, s, h] = sum(w * v[b, t, h] for w, t in zip(weights, keys))
    return out



LOG2E_F32 = np.float32(1.4426950408889634)


def _exp2_scale(head_dim: int, scale: Optional[float]) -> tuple:
    """(sign, c): the kernel works on sign * scores with c = |fl32(scale * log2 e)|.

    A negative scale is an exact sign flip of Q; scale 0 uses c = 2^-100 so
    masked scores stay -inf and every allowed score gives the same P.
    """
    sc = np.float32(head_dim ** -0.5 if scale is None else scale)
    c = float(np.float32(sc * LOG2E_F32))
    sign = -1.0 if c < 0 else 1.0
    c = abs(c)
    return sign, (c if c != 0.0 else 2.0 ** -100)


def kernel_rounding_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    valid_token_mask: Optional[torch.Tensor] = None,
    causal: bool = False,
    scale: Optional[float] = None,
    *,
    heads: Optional[list] = None,
    query_rows: Optional[slice] = None,
) -> torch.Tensor:
    """Attention with the 16-bit kernel's dtype boundaries, in float64.

    The reference's low-precision explicit attention rounds the softmax
    probabilities to the input dtype before P.V (transformer_opt/
    dispatch.py:94); a flash kernel rounds the unnormalised probabilities
    instead and divides by an fp32 row sum at the end.  This restates that
    order so a bf16/fp16 kernel can be held to a tight bound:

    * scores ``s = fl32(q . k)`` (exact products, one rounding to fp32), in
      units of ``c = |fl32(scale * log2 e)|``;
    * reference exponent ``M = ceil(fl32(max_allowed(s) * c))``, an integer;
    * ``p = fl32(exp2(fl32(s * c - M)))``, then ``P = p`` rounded to the
      input dtype (nearest even);
    * output ``sum(P v) / sum(P)`` - normalised by the sum of the rounded
      probabilities, so the weights applied to V sum to one; rows without an
      allowed key are zero.

    Any integer in place of ``M`` gives the same result up to a power of two
    that cancels in the division, so a kernel may move its reference lazily
    as long as it stays an integer.  Inputs are ``[B, S, H, D]`` fp16/bf16
    tensors; the result is float64 ``[B, S, H, D]``, or
    ``[len(heads), rows, D]`` when ``heads`` selects (b, h) pairs.
    """
    batch, seq_len, num_heads, head_dim = q.shape
    sign, c = _exp2_scale(head_dim, scale)
    pairs = heads if heads is not None else [(b, h) for b in range(batch) for h in range(num_heads)]
    rows = query_rows if query_rows is not None else slice(0, seq_len)
    qpos = torch.arange(seq_len)[rows]
    results = []
    for b, h in pairs:
        qh = q[b, rows, h, :].double() * sign
        kh = k[b, :, h, :].double()
        vh = v[b, :, h, :].double()
        s = torch.matmul(qh, kh.transpose(0, 1)).float().double()
        allowed = torch.ones((qh.shape[0], seq_len), dtype=torch.bool)
        if causal:
            allowed &= torch.arange(seq_len)[None, :] <= qpos[:, None]
        if valid_token_mask is not None:
            allowed &= valid_token_mask[b][None, :].to(torch.bool).cpu()
        s = s.masked_fill(~allowed, float("-inf"))
        any_allowed = allowed.any(dim=1)
        m = s.max(dim=1).values.masked_fill(~any_allowed, 0.0)
        ref = torch.ceil((m * c).float().double())
        p = torch.exp2((s * c - ref[:, None]).float().double()).float()
        rounded = p.to(q.dtype).double()
        total = rounded.sum(dim=1, keepdim=True)
        out = torch.matmul(rounded, vh) / total.clamp_min(torch.finfo(torch.float64).tiny)
        results.append(out.masked_fill(~any_allowed[:, None], 0.0))
    stacked = torch.stack(results)
    if heads is not None:
        return stacked
    return stacked.view(batch, num_heads, -1, head_dim).transpose(1, 2).contiguous()


def _round_bits_f32_to_bf16(x: np.float32) -> float:
    """Nearest-even bf16 of a float32, by its bit pattern."""
    bits = int(np.array(x, dtype=np.float32).view(np.uint32))
    bits = ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16) << 16
    return float(np.array(bits & 0xFFFFFFFF, dtype=np.uint32).view(np.float32))


def brute_force_kernel_rounding_f64(q, k, v, valid_token_mask=None, causal=False, scale=None,
                                    p_dtype: str = "bfloat16") -> np.ndarray:
    """Independent loop statement of :func:`kernel_rounding_attention`.

    Written from the definition, one query row at a time with numpy scalars:
    logits rounded to float32 from float64 dot products, an integer reference
    exponent ``ceil(float32(max * c))``, ``p = float32(2 ** float32(x * c -
    M))``, P rounded to bf16 by its bit pattern (nearest even) or to fp16 by
    numpy, output ``sum(P v) / sum(P)``.  ``p_dtype`` is "bfloat16",
    "float16" or "float32" (no rounding of P).
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    batch, seq_len, num_heads, head_dim = q.shape
    sc = np.float32(head_dim ** -0.5 if scale is None else scale)
    c = float(np.float32(sc * np.float32(1.4426950408889634)))
    sign = -1.0 if c < 0 else 1.0
    c = abs(c) if c != 0.0 else 2.0 ** -100
    mask = None if valid_token_mask is None else np.asarray(valid_token_mask, dtype=bool)
    rounders = {
        "bfloat16": _round_bits_f32_to_bf16,
        "float16": lambda x: float(np.float16(x)),
        "float32": float,
    }
    round_p = rounders[p_dtype]
    out = np.zeros_like(q)
    for b in range(batch):
        for h in range(num_heads):
            for s in range(seq_len):
                keys = [t for t in range(seq_len)
                        if (not causal or t <= s) and (mask is None or mask[b, t])]
                if not keys:
                    continue
                logits = [float(np.float32(sign * float(np.dot(q[b, s, h], k[b, t, h]))))
                          for t in keys]
                top = math.ceil(float(np.float32(max(logits) * c)))
                p = [np.float32(2.0 ** float(np.float32(x * c - top))) for x in logits]
                weights = [round_p(pi) for pi in p]
                total = sum(weights)
                out[b, s, h] = sum(w * v[b, t, h] for w, t in zip(weights, keys)) / total
    return out
