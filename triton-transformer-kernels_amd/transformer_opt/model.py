"""Module tree of the encoder, with the organizer benchmark's parameter names.

The reference's ``UserOptimizedTransformer`` subclasses the organizer's
``BaselineTransformer`` to inherit its submodules and parameter names
(transformer_opt/submission.py:78-92; benchmarks/torch_transformer_benchmark.
py:59-172), so a strict ``load_state_dict`` copies weights between the two.
This module declares the same tree - ``layers.{i}.norm1``,
``layers.{i}.attention.{q,k,v,out}_proj``, ``layers.{i}.norm2``,
``layers.{i}.ffn_in``, ``layers.{i}.ffn_out``, ``final_norm`` - without the
explicit math: the computation lives in ``submission.UserOptimizedTransformer``
and runs on the HIP kernels.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch.nn as nn


@dataclass(frozen=True)
class TransformerConfig:
    """Same fields and validation as the organizer config (benchmark :29-56)."""

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


class SelfAttention(nn.Module):
    """Projection parameters of one attention layer (benchmark :62-75)."""

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


class TransformerBlock(nn.Module):
    """Parameters of one pre-LN block (benchmark :125-132)."""

    def __init__(self, d_model: int, num_heads: int, ffn_dim: int) -> None:
        super().__init__()
        self.norm1 = nn.LayerNorm(d_model)
        self.attention = SelfAttention(d_model, num_heads)
        self.norm2 = nn.LayerNorm(d_model)
        self.ffn_in = nn.Linear(d_model, ffn_dim)
        self.ffn_out = nn.Linear(ffn_dim, d_model)
