"""Explicit pre-LN Transformer oracle (test infrastructure only).

Restates the organizer benchmark the reference is graded against
(benchmarks/torch_transformer_benchmark.py): the config (:29-56), explicit
self-attention (:59-122), block (:125-145), stack (:148-172), strict weight
copy (:203-213), seeded random cases (:234-272) and the element-wise OR
comparator (:289-356).  Parameter names are the organizer's, so
``load_state_dict(strict=True)`` works between this model and the product's
``UserOptimizedTransformer``.
"""

from __future__ import annotations

import copy
from dataclasses import dataclass
from typing import List, Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F


@dataclass(frozen=True)
class TransformerConfig:
    """Organizer config (torch_transformer_benchmark.py:29-56)."""

    batch_size: int
    seq_len: int
    d_model: int
    num_heads: int
    ffn_dim: int
    num_layers: int
    causal: bool

    def validate(self) -> None:
        for name in ("batch_size", "seq_len", "d_model", "num_heads", "ffn_dim", "num_layers"):
            if getattr(self, name) <= 0:
                raise ValueError(f"{name} must be positive")
        if self.d_model % self.num_heads != 0:
            raise ValueError(
                f"d_model ({self.d_model}) must be divisible by num_heads ({self.num_heads})"
            )


class BaselineSelfAttention(nn.Module):
    """Explicit multi-head attention (torch_transformer_benchmark.py:59-122)."""

    def __init__(self, d_model: int, num_heads: int) -> None:
        super().__init__()
        if d_model % num_heads != 0:
            raise ValueError("d_model must be divisible by num_heads")
        self.d_model = d_model
        self.num_heads = num_heads
        self.head_dim = d_model // num_heads
        self.scale = self.head_dim ** -0.5
        self.q_proj = nn.Linear(d_model, d_model, bias=True)
        self.k_proj = nn.Linear(d_model, d_model, bias=True)
        self.v_proj = nn.Linear(d_model, d_model, bias=True)
        self.out_proj = nn.Linear(d_model, d_model, bias=True)

    def _heads(self, t: torch.Tensor) -> torch.Tensor:
        batch, seq_len, _ = t.shape
        return t.view(batch, seq_len, self.num_heads, self.head_dim).transpose(1, 2).contiguous()

    def forward(self, x, valid_token_mask=None, causal=False):
        batch, seq_len, _ = x.shape
        q = self._heads(self.q_proj(x))
        k = self._heads(self.k_proj(x))
        v = self._heads(self.v_proj(x))
        scores = torch.matmul(q, k.transpose(-2, -1).contiguous()) * self.scale
        if causal:
            future = torch.ones((seq_len, seq_len), device=x.device, dtype=torch.bool).triu(diagonal=1)
            scores = scores.masked_fill(future, float("-inf"))
        if valid_token_mask is not None:
            scores = scores.masked_fill(~valid_token_mask[:, None, None, :], float("-inf"))
        probs = torch.softmax(scores.float(), dim=-1).to(dtype=x.dtype)
        context = torch.matmul(probs, v).transpose(1, 2).contiguous().view(batch, seq_len, self.d_model)
        output = self.out_proj(context)
        if valid_token_mask is not None:
            output = output.masked_fill(~valid_token_mask[..., None], 0)
        return output


class BaselineTransformerBlock(nn.Module):
    """Pre-LN block (torch_transformer_benchmark.py:125-145)."""

    def __init__(self, d_model: int, num_heads: int, ffn_dim: int) -> None:
        super().__init__()
        self.norm1 = nn.LayerNorm(d_model)
        self.attention = BaselineSelfAttention(d_model, num_heads)
        self.norm2 = nn.LayerNorm(d_model)
        self.ffn_in = nn.Linear(d_model, ffn_dim)
        self.ffn_out = nn.Linear(ffn_dim, d_model)

    def forward(self, x, valid_token_mask, causal):
        x = x + self.attention(self.norm1(x), valid_token_mask, causal)
        x = x + self.ffn_out(F.gelu(self.ffn_in(self.norm2(x)), approximate="none"))
        if valid_token_mask is not None:
            x = x.masked_fill(~valid_token_mask[..., None], 0)
        return x


class BaselineTransformer(nn.Module):
    """Layer stack + final norm (torch_transformer_benchmark.py:148-172)."""

    def __init__(self, config) -> None:
        super().__init__()
        self.config = config
        self.layers = nn.ModuleList(
            [BaselineTransformerBlock(config.d_model, config.num_heads, config.ffn_dim)
             for _ in range(config.num_layers)]
        )
        self.final_norm = nn.LayerNorm(config.d_model)

    def forward(self, x, valid_token_mask=None):
        for layer in self.layers:
            x = layer(x, valid_token_mask, self.config.causal)
        x = self.final_norm(x)
        if valid_token_mask is not None:
            x = x.masked_fill(~valid_token_mask[..., None], 0)
        return x


def copy_model_weights(baseline: nn.Module, optimized: nn.Module, strict: bool = True) -> None:
    """Strict state-dict copy (torch_transformer_benchmark.py:203-213)."""
    optimized.load_state_dict(copy.deepcopy(baseline.state_dict()), strict=strict)


def generate_random_case(config, device, dtype, seed: int, padding_ratio: float,
                         input_scale: float) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """Seeded input and key mask (torch_transformer_benchmark.py:234-272).

    As in the reference submission's wrapper (transformer_opt/submission.py:
    56-75) a zero padding ratio returns ``mask=None``.
    """
    generator = torch.Generator(device=device)
    generator.manual_seed(seed)
    x = torch.randn(config.batch_size, config.seq_len, config.d_model,
                    generator=generator, device=device, dtype=dtype) * input_scale
    if padding_ratio <= 0:
        return x, None
    min_valid = max(1, int(round(config.seq_len * (1.0 - padding_ratio))))
    lengths = torch.randint(low=min_valid, high=config.seq_len + 1, size=(config.batch_size,),
                            generator=generator, device=device)
    valid = torch.arange(config.seq_len, device=device)[None, :] < lengths[:, None]
    x = x.masked_fill(~valid[..., None], 0)
    return x, valid


@dataclass
class AccuracyResult:
    passed: bool
    total_elements: int
    failed_elements: int
    max_abs_error: float
    max_relative_error: float
    mean_abs_error: float
    failed_feature_dims: List[int]
    worst_index: Tuple[int, ...]
    reference_at_worst: float
    optimized_at_worst: float


def compare_outputs(reference: torch.Tensor, optimized: torch.Tensor, rtol: float,
                    atol: float) -> AccuracyResult:
    """Element-wise ``finite and (|d| <= atol or |d| <= rtol*|ref|)``.

    Restates torch_transformer_benchmark.py:289-356: the OR rule, not
    ``isclose``'s ``atol + rtol*|ref|``; every element must pass.
    """
    if reference.shape != optimized.shape:
        raise AssertionError(f"shape mismatch: {tuple(reference.shape)} vs {tuple(optimized.shape)}")
    ref = reference.detach().float().cpu()
    opt = optimized.detach().float().cpu()
    finite = torch.isfinite(ref) & torch.isfinite(opt)
    abs_error = (opt - ref).abs()
    passed = finite & ((abs_error <= atol) | (abs_error <= rtol * ref.abs()))
    failed = ~passed
    failed_elements = int(failed.sum().item())
    flat = abs_error.reshape(-1)
    flat = torch.where(torch.isnan(flat), torch.full_like(flat, float("inf")), flat)
    worst_flat = int(flat.argmax().item()) if flat.numel() else 0
    worst = []
    for size in reversed(reference.shape):
        worst.append(worst_flat % size)
        worst_flat //= size
    worst_index = tuple(reversed(worst))
    relative = abs_error / ref.abs().clamp_min(1e-12)
    if reference.ndim >= 2:
        failed_dims = torch.nonzero(failed.any(dim=tuple(range(reference.ndim - 1)))).flatten().tolist()
    else:
        failed_dims = torch.nonzero(failed).flatten().tolist()
    return AccuracyResult(
        passed=failed_elements == 0,
        total_elements=reference.numel(),
        failed_elements=failed_elements,
        max_abs_error=float(abs_error.max().item()) if abs_error.numel() else 0.0,
        max_relative_error=float(relative.max().item()) if relative.numel() else 0.0,
        mean_abs_error=float(abs_error.mean().item()) if abs_error.numel() else 0.0,
        failed_feature_dims=failed_dims,
        worst_index=worst_index,
        reference_at_worst=float(ref[worst_index].item()) if ref.numel() else 0.0,
        optimized_at_worst=float(opt[worst_index].item()) if opt.numel() else 0.0,
    )
