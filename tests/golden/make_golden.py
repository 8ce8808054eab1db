"""Write the float64 golden fixtures under tests/golden/.

Usage: python tests/golden/make_golden.py

The expected outputs are computed here with vectorised float64 numpy written
from the mathematical definitions (masked softmax attention; biased-variance
LayerNorm), independently of both the oracle (oracle/) and the kernels.  The
reference repository holds no golden vectors for this path, so these fixtures
plus the closed forms and library cross-checks in tests/test_oracle.py are
what pin the oracle.  Inputs are float32 (bf16-rounded where noted), stored
exactly; expected values are float64.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np

OUT = Path(__file__).resolve().parent


def _round_bf16(a: np.ndarray) -> np.ndarray:
    """Round float32 to the nearest bf16 (ties to even), returned as float32."""
    bits = a.astype(np.float32).view(np.uint32).astype(np.uint64)
    bits = (bits + 0x7FFF + ((bits >> 16) & 1)) >> 16 << 16
    return bits.astype(np.uint32).view(np.float32)


def attention_f64(q, k, v, mask, causal, scale):
    """Masked softmax attention in float64, one einsum per batch element."""
    q = q.astype(np.float64)
    k = k.astype(np.float64)
    v = v.astype(np.float64)
    batch, seq_len, heads, _ = q.shape
    logits = np.einsum("bshd,bthd->bhst", q, k) * scale
    allowed = np.ones((batch, 1, seq_len, seq_len), dtype=bool)
    if causal:
        allowed &= np.tril(np.ones((seq_len, seq_len), dtype=bool))[None, None]
    if mask is not None:
        allowed &= mask[:, None, None, :]
    logits = np.where(allowed, logits, -np.inf)
    row_max = logits.max(axis=-1, keepdims=True)
    row_max = np.where(np.isfinite(row_max), row_max, 0.0)
    weights = np.where(allowed, np.exp(logits - row_max), 0.0)
    denom = weights.sum(axis=-1, keepdims=True)
    probs = np.divide(weights, denom, out=np.zeros_like(weights), where=denom > 0)
    return np.einsum("bhst,bthd->bshd", probs, v)


def layer_norm_f64(r, w, b, eps):
    r = r.astype(np.float64)
    mean = r.mean(axis=-1, keepdims=True)
    var = ((r - mean) ** 2).mean(axis=-1, keepdims=True)
    y = (r - mean) / np.sqrt(var + eps) * w.astype(np.float64)
    if b is not None:
        y = y + b.astype(np.float64)
    return y


ATTENTION_CASES = [
    # name, B, S, H, D, causal, mask mode, bf16-rounded inputs
    ("tiny_causal_d8", 1, 5, 2, 8, True, "none", False),
    ("prefix_d16", 2, 33, 2, 16, False, "prefix", False),
    ("causal_prefix_d64", 1, 65, 1, 64, True, "prefix", False),
    ("minimum_d32", 2, 17, 1, 32, False, "minimum", False),
    ("causal_d128", 1, 40, 2, 128, True, "none", False),
    ("all_masked_d8", 1, 9, 1, 8, True, "empty", False),
    ("bf16_causal_d64", 1, 48, 2, 64, True, "none", True),
    ("ragged_d64", 1, 130, 2, 64, False, "none", False),
]

LAYER_NORM_CASES = [
    # name, rows, N, bias, mask, zero_residual, zero_normalized
    ("n128_masked_zero_both", 6, 128, True, True, True, True),
    ("n1000_no_bias", 5, 1000, False, False, False, False),
    ("n4096_bias", 4, 4096, True, False, False, False),
    ("n256_masked_zero_residual", 7, 256, True, True, True, False),
]


def _mask(mode, batch, seq_len, rng):
    if mode == "none":
        return None
    if mode == "empty":
        return np.zeros((batch, seq_len), dtype=bool)
    if mode == "minimum":
        lengths = np.ones(batch, dtype=np.int64)
    else:
        lengths = rng.integers(max(1, seq_len // 2), seq_len + 1, size=batch)
    return np.arange(seq_len)[None, :] < lengths[:, None]


def main() -> None:
    rng = np.random.default_rng(20261201)
    arrays = {}
    for name, batch, seq_len, heads, dim, causal, mode, bf16 in ATTENTION_CASES:
        shape = (batch, seq_len, heads, dim)
        q, k, v = (rng.standard_normal(shape).astype(np.float32) for _ in range(3))
        if bf16:
            q, k, v = _round_bf16(q), _round_bf16(k), _round_bf16(v)
        mask = _mask(mode, batch, seq_len, rng)
        scale = dim ** -0.5
        arrays[f"attn/{name}/q"] = q
        arrays[f"attn/{name}/k"] = k
        arrays[f"attn/{name}/v"] = v
        arrays[f"attn/{name}/mask"] = mask if mask is not None else np.zeros((0,), dtype=bool)
        arrays[f"attn/{name}/meta"] = np.array([causal, scale, bf16], dtype=np.float64)
        arrays[f"attn/{name}/expected"] = attention_f64(q, k, v, mask, causal, scale)
    for name, rows, width, bias, masked, zr, zn in LAYER_NORM_CASES:
        x = rng.standard_normal((rows, width)).astype(np.float32)
        u = rng.standard_normal((rows, width)).astype(np.float32)
        w = rng.uniform(0.5, 1.5, width).astype(np.float32)
        b = (rng.standard_normal(width) * 0.1).astype(np.float32) if bias else None
        mask = rng.random(rows) > 0.4 if masked else None
        residual = x + u  # float32 add, exactly the eager residual
        if zr:
            residual = np.where(mask[:, None], residual, np.float32(0))
        normalized = layer_norm_f64(residual, w, b, 1e-5)
        if zn:
            normalized = np.where(mask[:, None], normalized, 0.0)
        arrays[f"ln/{name}/x"] = x
        arrays[f"ln/{name}/u"] = u
        arrays[f"ln/{name}/w"] = w
        arrays[f"ln/{name}/b"] = b if b is not None else np.zeros((0,), dtype=np.float32)
        arrays[f"ln/{name}/mask"] = mask if mask is not None else np.zeros((0,), dtype=bool)
        arrays[f"ln/{name}/meta"] = np.array([1e-5, zr, zn], dtype=np.float64)
        arrays[f"ln/{name}/residual"] = residual.astype(np.float32)
        arrays[f"ln/{name}/normalized"] = normalized
    np.savez_compressed(OUT / "golden_v1.npz", **arrays)
    print(f"wrote {OUT / 'golden_v1.npz'} ({len(arrays)} arrays)")


if __name__ == "__main__":
    main()
