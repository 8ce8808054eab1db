"""HIP fused attention vs the CPU oracle (reference tests/test_gpu_attention.py).

Inputs are generated on the CPU from fixed seeds and copied to the GPU, so the
oracle and the kernel see identical bytes.  Two bounds are asserted:

* the contract, finite on every element and
    - fp32 and fp16: the reference's ``|d| <= 1e-3 or |d| <= 0.01*|ref|``
      (tests/test_gpu_attention.py:53-62);
    - bf16 (no reference route exists, config.py:17-18; bound stated before
      measuring): ``|d| <= 2e-3 or |d| <= 0.02*|ref|``, no mean-error term.
  fp32 outputs are compared with the reference's explicit attention in fp32.
  bf16/fp16 outputs are compared with the same attention evaluated at the
  16-bit kernel's dtype boundaries (fp32 scores, probabilities rounded to the
  input dtype before P.V against an integer reference exponent, fp32 row
  sum; ``oracle.attention.kernel_rounding_attention``), on the same rounded
  inputs.
* a tighter accuracy bound for fp32 that catches systematic mistakes the
  loose contract can hide: ``|d| <= 2e-5 + 2e-5*|ref|`` at the default scale.
"""

from __future__ import annotations

import pytest
import torch

from oracle.attention import (
    _exp2_scale,
    brute_force_attention_f64,
    chunked_kernel_contract_attention,
    kernel_contract_attention,
    kernel_rounding_attention,
)

pytestmark = pytest.mark.gpu

CASES = [
    # (B, S, H, D, dtype, causal, mask mode, input scale) - the reference's
    # CASES (tests/test_gpu_attention.py:18-31) plus bf16 and larger tiles.
    (2, 31, 4, 8, torch.float16, True, "all", 1.0),
    (1, 65, 16, 8, torch.float32, True, "prefix", 1.0),
    (1, 1, 1, 16, torch.float16, False, "none", 1.0),
    (2, 31, 4, 32, torch.float16, True, "all", 1.0),
    (1, 63, 4, 64, torch.float16, False, "prefix", 0.25),
    (2, 64, 2, 64, torch.float16, True, "prefix", 1.0),
    (1, 65, 2, 128, torch.float16, False, "minimum", 1.0),
    (1, 127, 4, 32, torch.float16, True, "none", 3.0),
    (1, 129, 4, 64, torch.float16, True, "prefix", 1.0),
    (1, 257, 2, 32, torch.float16, False, "prefix", 1.0),
    (1, 65, 2, 32, torch.float32, True, "prefix", 1.0),
    (2, 200, 3, 64, torch.float32, False, "none", 1.0),
    (2, 300, 2, 64, torch.float32, True, "none", 1.0),
    (1, 333, 2, 128, torch.float32, True, "prefix", 1.0),
    (1, 190, 2, 16, torch.float32, False, "minimum", 1.0),
    (2, 260, 2, 64, torch.bfloat16, True, "none", 1.0),
    (1, 130, 3, 128, torch.bfloat16, False, "prefix", 1.0),
    (1, 70, 2, 8, torch.bfloat16, True, "none", 1.0),
    (1, 96, 8, 16, torch.bfloat16, False, "all", 2.0),
    # Real key masks (B > 1 prefix lengths) on every head dim of the fp32 path.
    (2, 150, 2, 64, torch.float32, True, "prefix", 1.0),
    (2, 150, 2, 64, torch.float32, False, "prefix", 1.0),
    (2, 150, 2, 128, torch.float32, False, "prefix", 1.0),
    (3, 97, 2, 128, torch.float32, True, "prefix", 1.0),
    (3, 100, 2, 32, torch.float32, True, "prefix", 1.0),
    (3, 100, 2, 64, torch.bfloat16, True, "prefix", 1.0),
    (2, 140, 2, 128, torch.bfloat16, False, "prefix", 1.0),
    # Longer fp32 rows with key masks (several full tiles before the masked
    # diagonal and ragged tiles) and a sequence shorter than one query tile.
    (2, 512, 2, 64, torch.float32, True, "prefix", 1.0),
    (2, 513, 2, 64, torch.float32, True, "prefix", 1.0),
    (2, 700, 2, 64, torch.float32, True, "prefix", 1.0),
    (1, 777, 3, 32, torch.float32, False, "prefix", 1.0),
    (2, 640, 2, 16, torch.float32, True, "prefix", 1.0),
    (3, 64, 4, 64, torch.float32, False, "prefix", 1.0),
]


def make_mask(mode: str, batch: int, seq_len: int):
    if mode == "none":
        return None
    if mode == "all":
        return torch.ones(batch, seq_len, dtype=torch.bool)
    if mode == "minimum":
        lengths = torch.ones(batch, dtype=torch.long)
    elif mode == "prefix":
        lengths = torch.linspace(seq_len, max(1, seq_len // 2), batch).to(torch.long)
    else:  # pragma: no cover
        raise ValueError(mode)
    return torch.arange(seq_len)[None, :] < lengths[:, None]


# |d| <= atol or |d| <= rtol * |ref| on every element, against the oracle of
# the dtype (see ``oracle``): fp32 and fp16 the reference's contract
# (torch_transformer_benchmark.py:309-319), bf16 the bound stated before
# measuring for a dtype the reference has no fused route for.
CONTRACT = {
    torch.float32: (1e-3, 1e-2),
    torch.float16: (1e-3, 1e-2),
    torch.bfloat16: (2e-3, 2e-2),
}


def contract_failures(actual: torch.Tensor, reference: torch.Tensor) -> int:
    """Elements outside the dtype's contract (finite and |d|<=atol or <=rtol*|ref|)."""
    atol, rtol = CONTRACT[actual.dtype]
    a = actual.float().cpu()
    r = reference.float().cpu()
    err = (a - r).abs()
    ok = torch.isfinite(a) & ((err <= atol) | (err <= rtol * r.abs()))
    return int((~ok).sum().item())


def tight_check(actual: torch.Tensor, reference: torch.Tensor, dtype: torch.dtype,
                tol: float = 2e-5) -> None:
    """fp32 only: |d| <= tol + tol*|ref| (low-precision dtypes use the contract)."""
    if dtype != torch.float32:
        return
    a = actual.float().cpu()
    r = reference.float().cpu()
    err = (a - r).abs()
    ok = err <= tol + tol * r.abs()
    assert bool(ok.all()), (
        f"tight bound: failed={int((~ok).sum())}/{ok.numel()} max_abs={err.max().item():.3g}"
    )


def run_hip(q, k, v, mask, causal, scale=None):
    from transformer_opt import attention_forward

    dev = torch.device("cuda")
    with torch.inference_mode():
        out, decision = attention_forward(
            q.to(dev), k.to(dev), v.to(dev),
            None if mask is None else mask.to(dev),
            causal=causal, scale=scale, backend="hip",
        )
    assert decision.selected == "hip"
    return out.cpu()


def test_forced_triton_backend_runs_the_hip_kernel(gpu_ready):
    # Reference callers force backend="triton" (tests/test_gpu_attention.py:
    # 99-180, tests/test_dispatch.py:29); here that route is the HIP kernel.
    from transformer_opt import attention_forward

    g = torch.Generator().manual_seed(5)
    for dtype in (torch.float32, torch.float16, torch.bfloat16):
        q, k, v = (torch.randn(2, 77, 3, 64, generator=g).to(dtype).cuda() for _ in range(3))
        mask = make_mask("prefix", 2, 77)
        with torch.inference_mode():
            out, decision = attention_forward(q, k, v, mask.cuda(), causal=True, backend="triton")
            hip, _ = attention_forward(q, k, v, mask.cuda(), causal=True, backend="hip")
        assert (decision.requested, decision.selected) == ("triton", "hip")
        assert torch.equal(out, hip)
        assert contract_failures(out.cpu(), oracle(q.cpu(), k.cpu(), v.cpu(), mask, True)) == 0
    with torch.inference_mode(), pytest.raises(ValueError, match="Triton attention was forced"):
        bad = torch.randn(1, 8, 2, 48, device="cuda")
        attention_forward(bad, bad, bad, backend="triton")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_reference_route_runs_the_explicit_math_on_the_gpu(gpu_ready, dtype):
    # backend="reference" (reference dispatch.py:69-96, 145-152): explicit
    # torch math on the device, never the kernel.  fp32 agrees with the
    # oracle's restatement on the CPU within float32 rounding; bf16/fp16
    # (scores and probabilities rounded to 8 / 11 bits, as in the reference)
    # within the model-level bound, and with the HIP kernel within it too.
    from oracle.attention import explicit_attention as oracle_explicit
    from transformer_opt import attention_forward

    g = torch.Generator().manual_seed(17)
    q, k, v = (torch.randn(2, 150, 4, 64, generator=g).to(dtype) for _ in range(3))
    mask = make_mask("prefix", 2, 150)
    with torch.inference_mode():
        out, record = attention_forward(q.cuda(), k.cuda(), v.cuda(), mask.cuda(), causal=True,
                                        backend="reference")
        hip, _ = attention_forward(q.cuda(), k.cuda(), v.cuda(), mask.cuda(), causal=True,
                                   backend="hip")
    assert (record.requested, record.selected) == ("reference", "reference")
    expected = oracle_explicit(q.float(), k.float(), v.float(), mask, True)
    atol, rtol = (1e-5, 1e-5) if dtype == torch.float32 else (5e-2, 5e-2)
    for got in (out, hip):
        err = (got.float().cpu() - expected).abs()
        assert bool(((err <= atol) | (err <= rtol * expected.abs())).all()), float(err.max())


def oracle(q, k, v, mask, causal, scale=None):
    """The checker of each dtype, on the (already rounded) inputs.

    fp32: the reference's explicit attention in fp32 with the kernel's
    all-masked-row contract.  bf16/fp16: the same attention with the 16-bit
    kernel's dtype boundaries - fp32 scores, probabilities rounded to the
    input dtype before P.V against an integer reference exponent, fp32 row
    sum (oracle.attention.kernel_rounding_attention) - so the bound measures
    the kernel, not the rounding of P that any 16-bit P.V performs.
    """
    if q.dtype in (torch.bfloat16, torch.float16):
        return kernel_rounding_attention(q, k, v, mask, causal, scale).float()
    return kernel_contract_attention(q.float(), k.float(), v.float(), mask, causal, scale)


@pytest.mark.parametrize("batch,seq_len,heads,head_dim,dtype,causal,mask_mode,input_scale", CASES)
def test_hip_attention_matches_explicit_reference(
    gpu_ready, batch, seq_len, heads, head_dim, dtype, causal, mask_mode, input_scale
):
    for seed in (7, 19):
        g = torch.Generator().manual_seed(seed)
        shape = (batch, seq_len, heads, head_dim)
        q = (torch.randn(shape, generator=g) * input_scale).to(dtype)
        k = (torch.randn(shape, generator=g) * input_scale).to(dtype)
        v = torch.randn(shape, generator=g).to(dtype)
        mask = make_mask(mask_mode, batch, seq_len)
        actual = run_hip(q, k, v, mask, causal)
        reference = oracle(q, k, v, mask, causal)
        assert actual.dtype == dtype and actual.shape == q.shape
        failures = contract_failures(actual, reference)
        assert failures == 0, f"seed={seed} contract failures={failures}"
        tight_check(actual, reference, dtype)


def reference_math_bound_failures(actual, q, k, v, mask, causal, scale=None) -> int:
    """Elements of a 16-bit kernel output outside the rounding bound of the
    reference's explicit math, evaluated in fp32 on the same rounded inputs.

    The reference (dispatch.py:69-96) on fp32 copies of q/k/v gives
    out = sum(p v) / sum(p).  The 16-bit kernel differs from it by (1) the
    rounding of each probability to the input dtype before P.V, w = p(1+e),
    |e| <= u, which moves the output by at most 2u/(1-u) * sum(p|v|)/sum(p)
    (the closed form pinned on the CPU by test_p_rounding_error_is_within_
    its_closed_form_bound), (2) the rounding of the output to the input dtype,
    at most u * |out|, and (3) fp32 summation order, covered by 2e-3.  u is
    the unit roundoff: 2^-8 (bf16), 2^-11 (fp16).  Rows with no allowed key
    are 0 in both (the kernel contract).
    """
    q32, k32, v32 = q.float(), k.float(), v.float()
    if q.shape[0] * q.shape[2] * q.shape[1] ** 2 > (1 << 26):
        ref = chunked_kernel_contract_attention(q32, k32, v32, mask, causal, scale)
        mag = chunked_kernel_contract_attention(q32, k32, v32.abs(), mask, causal, scale)
        batch, seq_len, heads, head_dim = q.shape
        ref = ref.view(batch, heads, seq_len, head_dim).transpose(1, 2)
        mag = mag.view(batch, heads, seq_len, head_dim).transpose(1, 2)
    else:
        ref = kernel_contract_attention(q32, k32, v32, mask, causal, scale)
        mag = kernel_contract_attention(q32, k32, v32.abs(), mask, causal, scale)
    unit = 2.0 ** -8 if q.dtype == torch.bfloat16 else 2.0 ** -11
    bound = 2e-3 + 2 * unit / (1 - unit) * mag + unit * ref.abs()
    err = (actual.float().cpu() - ref).abs()
    return int((~(err <= bound)).sum())


SIXTEEN_BIT_CASES = [c for c in CASES if c[4] != torch.float32] + [
    (1, 4096, 2, 64, torch.bfloat16, True, "none", 1.0),
    (2, 1000, 3, 128, torch.float16, False, "prefix", 2.0),
]


@pytest.mark.parametrize("batch,seq_len,heads,head_dim,dtype,causal,mask_mode,input_scale",
                         SIXTEEN_BIT_CASES)
def test_16bit_attention_within_rounding_bound_of_reference_math(
    gpu_ready, batch, seq_len, heads, head_dim, dtype, causal, mask_mode, input_scale
):
    # The 16-bit kernels against the reference's own explicit math (not the
    # kernel-rounding oracle): fp32 attention on the rounded inputs, held to
    # the closed-form bound of the two roundings a 16-bit kernel performs.
    g = torch.Generator().manual_seed(seq_len * 3 + head_dim)
    shape = (batch, seq_len, heads, head_dim)
    q = (torch.randn(shape, generator=g) * input_scale).to(dtype)
    k = (torch.randn(shape, generator=g) * input_scale).to(dtype)
    v = torch.randn(shape, generator=g).to(dtype)
    mask = make_mask(mask_mode, batch, seq_len)
    actual = run_hip(q, k, v, mask, causal)
    assert reference_math_bound_failures(actual, q, k, v, mask, causal) == 0


def test_16bit_config4_attention_within_rounding_bound_of_reference_math(gpu_ready):
    # Config 4's attention (B=4, S=2048, H=16, D=64, causal, bf16), every
    # element of every head against the reference's explicit math.
    g = torch.Generator().manual_seed(44)
    shape = (4, 2048, 16, 64)
    q, k, v = (torch.randn(shape, generator=g).to(torch.bfloat16) for _ in range(3))
    actual = run_hip(q, k, v, None, True)
    assert reference_math_bound_failures(actual, q, k, v, None, True) == 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("ramp", [3.0, 7.0, 12.0])
@pytest.mark.parametrize("causal", [True, False])
def test_running_max_growth_across_tiles(gpu_ready, dtype, head_dim, ramp, causal):
    # Scores rise along the key axis by about `ramp` (log2 units) per 64-key
    # tile, so every row's running max moves in every tile.  The 16-bit
    # kernel keeps a lagging reference max and rescales only when a row
    # outruns it by more than 2^8: ramps of 3 and 7 rescale every few tiles
    # (P up to 2^8 in between), 12 in every tile.  The fp32 kernel rescales
    # every tile.  Either way the output must match the oracle.
    g = torch.Generator().manual_seed(int(ramp * 10) + head_dim)
    seq_len, heads = 700, 2
    c = head_dim ** -0.5 * 1.4426950408889634
    per_key = ramp / (64 * c)
    keys = torch.arange(seq_len, dtype=torch.float32)
    q = 1.0 + 0.1 * torch.randn(1, seq_len, heads, head_dim, generator=g)
    k = (per_key / head_dim) * keys[None, :, None, None] + 0.1 * torch.randn(1, seq_len, heads, head_dim, generator=g)
    v = torch.randn(1, seq_len, heads, head_dim, generator=g)
    q, k, v = q.to(dtype), k.to(dtype), v.to(dtype)
    actual = run_hip(q, k, v, None, causal)
    reference = oracle(q, k, v, None, causal)
    assert contract_failures(actual, reference) == 0
    tight_check(actual, reference, dtype, tol=1e-4)


@pytest.mark.parametrize("seq_len", [192, 193, 255, 256, 257, 320, 383, 448])
@pytest.mark.parametrize("head_dim", [8, 16, 32, 64, 128])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("causal", [True, False])
def test_pipelined_loop_copy_boundaries(gpu_ready, seq_len, head_dim, dtype, causal):
    # Unmasked 16-bit launches run full key tiles through the two-phase loop,
    # whose K(t+2) / V(t+1) copies are issued between its MFMA groups; where
    # K(t+2) is the ragged last tile or past the query tile's last key tile
    # the copy takes the generic path instead.  These lengths put the loop's
    # end on each side of those cases, for every wavefront of a query tile.
    g = torch.Generator().manual_seed(seq_len * 7 + head_dim)
    shape = (2, seq_len, 3, head_dim)
    q = torch.randn(shape, generator=g).to(dtype)
    k = torch.randn(shape, generator=g).to(dtype)
    v = torch.randn(shape, generator=g).to(dtype)
    actual = run_hip(q, k, v, None, causal)
    reference = oracle(q, k, v, None, causal)
    assert contract_failures(actual, reference) == 0
    tight_check(actual, reference, dtype)


def test_all_keys_masked_is_finite_zero(gpu_ready):
    # Reference tests/test_gpu_attention.py:114-128.
    g = torch.Generator().manual_seed(3)
    for dtype in (torch.float16, torch.float32, torch.bfloat16):
        q = torch.randn(2, 65, 2, 32, generator=g).to(dtype)
        all_masked = torch.zeros(2, 65, dtype=torch.bool)
        for causal in (True, False):
            out = run_hip(q, q, q, all_masked, causal)
            assert torch.isfinite(out).all()
            assert torch.count_nonzero(out) == 0


@pytest.mark.parametrize("seq_len", [31, 32, 33, 63, 64, 65, 127, 128, 129, 257])
@pytest.mark.parametrize("head_dim", [8, 16, 32, 128])
@pytest.mark.parametrize("mask_mode", ["none", "minimum"])
def test_causal_frontier_matches_reference_at_tile_boundaries(gpu_ready, seq_len, head_dim, mask_mode):
    # Reference tests/test_gpu_attention.py:153-169.
    g = torch.Generator().manual_seed(41)
    q = torch.randn(1, seq_len, 2, head_dim, generator=g)
    k, v = torch.randn(q.shape, generator=g), torch.randn(q.shape, generator=g)
    mask = make_mask(mask_mode, 1, seq_len)
    actual = run_hip(q, k, v, mask, True)
    reference = oracle(q, k, v, mask, True)
    assert contract_failures(actual, reference) == 0
    tight_check(actual, reference, torch.float32)


@pytest.mark.parametrize("seq_len", [97, 127, 128, 225, 353, 384])
@pytest.mark.parametrize("head_dim", [8, 16, 32, 64])
@pytest.mark.parametrize("mask_mode", ["none", "drop_last32", "only_last32"])
def test_causal_last_diagonal_sub_block_split_between_wavefronts(gpu_ready, seq_len, head_dim, mask_mode):
    # fp32 causal: in the last key tile of a 128-query tile, the keys
    # [start+96, start+128) of the last 32 query rows are processed by another
    # wavefront and merged (running max, sum and output) into those rows.
    # Sequence lengths leave 1, 31 or 32 valid rows there; the key masks make
    # either side of the merge empty: "drop_last32" removes those keys (the
    # handed-over part sees no key), "only_last32" keeps only them (the rows'
    # own part sees no key, rows before them see none at all -> zeros).
    g = torch.Generator().manual_seed(seq_len + head_dim)
    batch = 2
    q = torch.randn(batch, seq_len, 2, head_dim, generator=g)
    k, v = torch.randn(q.shape, generator=g), torch.randn(q.shape, generator=g)
    keys = torch.arange(seq_len)
    in_last32 = (keys % 128) >= 96
    if mask_mode == "none":
        mask = None
    elif mask_mode == "drop_last32":
        mask = (~in_last32)[None, :].expand(batch, seq_len).clone()
    else:
        mask = in_last32[None, :].expand(batch, seq_len).clone()
    actual = run_hip(q, k, v, mask, True)
    reference = oracle(q, k, v, mask, True)
    assert contract_failures(actual, reference) == 0
    tight_check(actual, reference, torch.float32)
    if mask_mode == "only_last32":
        # Rows before the first allowed key see nothing: exact zeros.
        assert bool((actual[:, :96] == 0).all())


def test_causal_frontier_cannot_observe_future_key_value_tiles(gpu_ready):
    # Reference tests/test_gpu_attention.py:172-181, bitwise.
    g = torch.Generator().manual_seed(43)
    for dtype in (torch.float32, torch.bfloat16):
        q = torch.randn(1, 257, 2, 32, generator=g).to(dtype)
        k, v = torch.randn(q.shape, generator=g).to(dtype), torch.randn(q.shape, generator=g).to(dtype)
        before = run_hip(q, k, v, None, True)
        k2, v2 = k.clone(), v.clone()
        k2[:, 64:] *= 100
        v2[:, 64:] += 100
        after = run_hip(q, k2, v2, None, True)
        assert torch.equal(before[:, :64], after[:, :64])


def test_brute_force_float64_agrees(gpu_ready):
    # The float64 textbook definition, independent of the explicit oracle.
    g = torch.Generator().manual_seed(5)
    q = torch.randn(1, 40, 2, 64, generator=g)
    k, v = torch.randn(q.shape, generator=g), torch.randn(q.shape, generator=g)
    mask = make_mask("prefix", 1, 40)
    for causal in (False, True):
        actual = run_hip(q, k, v, mask, causal).double().numpy()
        expected = brute_force_attention_f64(q.numpy(), k.numpy(), v.numpy(), mask.numpy(), causal)
        assert abs(actual - expected).max() < 2e-5


def test_packed_qkv_views_equal_contiguous_copies_bitwise(gpu_ready):
    # The model passes unbind() views of one [B, S, 3, H, D] projection.
    g = torch.Generator().manual_seed(11)
    for dtype in (torch.float32, torch.bfloat16):
        packed = torch.randn(2, 150, 3, 4, 64, generator=g).to(dtype)
        q, k, v = packed.unbind(dim=2)
        dev = torch.device("cuda")
        from transformer_opt.kernels import hip_attention

        with torch.inference_mode():
            pd = packed.to(dev)
            qv, kv, vv = pd.unbind(dim=2)
            strided = hip_attention(qv, kv, vv, causal=True)
            dense = hip_attention(qv.contiguous(), kv.contiguous(), vv.contiguous(), causal=True)
        assert torch.equal(strided.cpu(), dense.cpu())
        reference = oracle(q, k, v, None, True)
        assert contract_failures(strided, reference) == 0


def test_all_valid_mask_equals_no_mask_bitwise(gpu_ready):
    g = torch.Generator().manual_seed(13)
    q = torch.randn(2, 100, 2, 64, generator=g)
    k, v = torch.randn(q.shape, generator=g), torch.randn(q.shape, generator=g)
    for causal in (False, True):
        a = run_hip(q, k, v, None, causal)
        b = run_hip(q, k, v, torch.ones(2, 100, dtype=torch.bool), causal)
        assert torch.equal(a, b)


def test_closed_forms(gpu_ready):
    g = torch.Generator().manual_seed(17)
    # Identical keys -> uniform weights -> causal row i is the mean of V[0..i].
    q = torch.randn(1, 97, 2, 64, generator=g)
    k = torch.randn(1, 1, 2, 64, generator=g).expand(1, 97, 2, 64).contiguous()
    v = torch.randn(1, 97, 2, 64, generator=g)
    out = run_hip(q, k, v, None, True)
    expected = torch.cumsum(v.double(), dim=1) / torch.arange(1, 98, dtype=torch.float64)[None, :, None, None]
    assert (out.double() - expected).abs().max() < 1e-5
    # Causal row 0 sees only key 0: exactly V[0].
    assert torch.equal(out[:, 0], v[:, 0])
    # One dominant logit -> that key's value.
    q = torch.zeros(1, 8, 1, 32)
    q[..., 0] = 1.0
    k = torch.zeros(1, 8, 1, 32)
    k[0, 5, 0, 0] = 1000.0
    v = torch.randn(1, 8, 1, 32, generator=g)
    out = run_hip(q, k, v, None, False)
    assert torch.allclose(out[0, :, 0], v[0, 5, 0].expand(8, 32), atol=1e-6)


def test_explicit_scale_and_non_power_of_two_batch_heads(gpu_ready):
    g = torch.Generator().manual_seed(23)
    q = torch.randn(3, 77, 5, 64, generator=g)
    k, v = torch.randn(q.shape, generator=g), torch.randn(q.shape, generator=g)
    for scale in (0.3, 1.7):
        actual = run_hip(q, k, v, None, False, scale=scale)
        reference = oracle(q, k, v, None, False, scale=scale)
        assert contract_failures(actual, reference) == 0
        # Logits up to ~14x the default scale: fp32 rounding of the scores
        # grows with |logit|, so the tight bound scales with it.
        tight_check(actual, reference, torch.float32, tol=2e-5 * scale / 0.125)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16], ids=["fp32", "bf16", "fp16"])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("causal", [False, True], ids=["noncausal", "causal"])
@pytest.mark.parametrize("mask_mode", ["none", "prefix"])
def test_negative_zero_and_large_scales(gpu_ready, dtype, head_dim, causal, mask_mode):
    # A negative scale is folded into Q (an exact sign flip for 16-bit inputs,
    # the pre-scale for fp32); scale 0 gives uniform weights, so every output
    # row is the mean of V over its allowed keys (a closed form, checked
    # without the oracle; rows with no allowed key are zero); 0.9 makes
    # logits ~7x the default scale's.
    g = torch.Generator().manual_seed(31 + head_dim)
    shape = (2, 150, 3, head_dim)
    q, k, v = (torch.randn(shape, generator=g).to(dtype) for _ in range(3))
    mask = make_mask(mask_mode, shape[0], shape[1])
    for scale in (-0.4, 0.0, 0.9):
        actual = run_hip(q, k, v, mask, causal, scale=scale)
        reference = oracle(q, k, v, mask, causal, scale=scale)
        # bf16 rounds P and the output to 8 significant bits, so the mean
        # error grows with |out|: at scale 0.9 the softmax is peaked and the
        # outputs are about |v|, not an average over many keys.
        assert contract_failures(actual, reference) == 0, f"scale={scale}"
        if scale == 0.0:
            keys = torch.ones(shape[0], shape[1], dtype=torch.bool) if mask is None else mask
            allowed = keys[:, None, :].expand(shape[0], shape[1], shape[1])  # [b, query, key]
            if causal:
                allowed = allowed & torch.ones(shape[1], shape[1], dtype=torch.bool).tril()[None]
            w = allowed.double()
            counts = w.sum(dim=2, keepdim=True)
            vf = v.double().reshape(shape[0], shape[1], -1)
            mean = torch.matmul(w / counts.clamp(min=1), vf).reshape(shape)
            err = (actual.double() - mean).abs().max().item()
            # P is exactly 1 for every allowed key; the only rounding is the
            # P.V accumulation in fp32 and the output conversion.
            bound = 1e-5 if dtype == torch.float32 else (8e-3 if dtype == torch.bfloat16 else 1e-3)
            assert err <= bound, f"scale=0 mean-of-V error {err:.3g}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16], ids=["fp32", "bf16", "fp16"])
@pytest.mark.parametrize("causal", [False, True], ids=["noncausal", "causal"])
def test_permuted_layouts_and_strided_mask(gpu_ready, dtype, causal):
    # Q is the transpose of a [B, H, S, D] tensor, K a permute of [S, B, H, D]
    # (every B/S/H stride differs from the packed layout), V contiguous, and
    # the key mask a stride-2 view - all built on the GPU so no copy makes
    # them contiguous.  The result must be bitwise the one of contiguous
    # copies and within the contract of the oracle.
    g = torch.Generator().manual_seed(57)
    B, S, H, D = 2, 200, 3, 64
    dev = torch.device("cuda")
    q = torch.randn(B, H, S, D, generator=g).to(dtype).to(dev).transpose(1, 2)
    k = torch.randn(S, B, H, D, generator=g).to(dtype).to(dev).permute(1, 0, 2, 3)
    v = torch.randn(B, S, H, D, generator=g).to(dtype).to(dev)
    mask_full = torch.rand(B, 2 * S, generator=g) > 0.25
    mask_full[:, 0] = True
    mask = mask_full.to(dev)[:, ::2]
    assert not q.is_contiguous() and not k.is_contiguous() and not mask.is_contiguous()
    actual = run_hip(q, k, v, mask, causal)
    again = run_hip(q.contiguous(), k.contiguous(), v, mask.contiguous(), causal)
    assert torch.equal(actual, again)
    reference = oracle(q.cpu(), k.cpu(), v.cpu(), mask.cpu(), causal)
    assert contract_failures(actual, reference) == 0
    tight_check(actual, reference, dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_contiguous_views_at_unaligned_offsets(gpu_ready, dtype):
    # buf[1:].view(B, S, H, D) is contiguous but starts one element past a
    # 16-byte boundary; the wrapper copies it to aligned storage instead of
    # refusing an input the reference accepts.
    from transformer_opt.kernels import hip_attention

    g = torch.Generator().manual_seed(61)
    B, S, H, D = 2, 70, 2, 64
    n = B * S * H * D
    bufs = [torch.randn(n + 1, generator=g).to(dtype).cuda() for _ in range(3)]
    q, k, v = (b[1:].view(B, S, H, D) for b in bufs)
    assert all(t.is_contiguous() and t.data_ptr() % 16 != 0 for t in (q, k, v))
    with torch.inference_mode():
        out = hip_attention(q, k, v, causal=True)
        aligned = hip_attention(q.clone(), k.clone(), v.clone(), causal=True)
    assert torch.equal(out, aligned)
    assert contract_failures(out.cpu(), oracle(q.cpu(), k.cpu(), v.cpu(), None, True)) == 0


def test_empty_batch_returns_empty(gpu_ready):
    for dtype in (torch.float32, torch.bfloat16):
        q = torch.empty(0, 16, 2, 64, dtype=dtype)
        out = run_hip(q, q, q, None, True)
        assert out.shape == (0, 16, 2, 64) and out.dtype == dtype


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16], ids=["fp32", "bf16", "fp16"])
@pytest.mark.parametrize("head_dim", [64, 128])
def test_left_padding_with_causal_mask(gpu_ready, dtype, head_dim):
    # Left padding: the first keys of each sequence are masked, so under the
    # causal bound the first rows have no allowed key (exact zeros) while
    # later rows of the same wavefront start their running max in the same
    # tiles.  The 16-bit kernel once rescaled those empty rows by
    # exp2(-inf - (-inf)) = NaN when another row of the wavefront moved its
    # reference.
    g = torch.Generator().manual_seed(71 + head_dim)
    batch, seq_len, heads = 3, 230, 2
    q, k, v = (torch.randn(batch, seq_len, heads, head_dim, generator=g).to(dtype) for _ in range(3))
    pad = torch.tensor([1, 5, 70])  # masked keys at the start of each sequence
    mask = torch.arange(seq_len)[None, :] >= pad[:, None]
    actual = run_hip(q, k, v, mask, True)
    reference = oracle(q, k, v, mask, True)
    assert bool(torch.isfinite(actual.float()).all())
    assert contract_failures(actual, reference) == 0
    tight_check(actual, reference, dtype)
    for b in range(batch):
        assert bool((actual[b, : int(pad[b])] == 0).all())


@pytest.mark.parametrize("head_dim", [64, 32, 16, 8])
def test_paired_grid_with_key_masks(gpu_ready, head_dim):
    # The fp32 paired schedule (a workgroup runs query tiles nq-1-i and i) is
    # chosen only for grids that fill every workgroup slot, e.g. the config-2
    # shape B=8, S=1024, H=16; together with the diagonal hand-off and the
    # priority alternation it is checked here under key masks: left padding
    # of varying length (rows with no allowed key) and random holes.  Three
    # heads of every batch element are compared with the oracle.
    g = torch.Generator().manual_seed(91 + head_dim)
    batch, seq_len, heads = 8, 1024, 16
    q, k, v = (torch.randn(batch, seq_len, heads, head_dim, generator=g) for _ in range(3))
    positions = torch.arange(seq_len)[None, :]
    pad = torch.tensor([0, 1, 3, 40, 100, 130, 0, 500])[:, None]
    mask = positions >= pad
    mask[6] &= torch.rand(seq_len, generator=g) > 0.3  # holes
    mask[7] &= torch.rand(seq_len, generator=g) > 0.5
    actual = run_hip(q, k, v, mask, True)
    for hh in (0, 7, 15):
        sl = slice(hh, hh + 1)
        reference = oracle(q[:, :, sl], k[:, :, sl], v[:, :, sl], mask, True)
        assert contract_failures(actual[:, :, sl], reference) == 0, f"head {hh}"
        tight_check(actual[:, :, sl], reference, torch.float32)
    for b in range(batch):
        assert bool((actual[b, : int(pad[b])] == 0).all())


@pytest.mark.parametrize("batch,seq_len,heads,head_dim,mask_mode", [
    (8, 512, 16, 64, "holes"),   # config 2 at S=512: 4 query tiles x 128 heads = 512 workgroups
    (3, 400, 32, 64, "prefix"),  # 384 workgroups, ragged last tile
    (2, 700, 24, 32, "none"),    # 6 query tiles x 48 heads = 288 workgroups
    (5, 600, 13, 64, "holes"),   # B*H = 65: no XCD swizzle; 5 query tiles, 325 workgroups
    (4, 500, 32, 16, "holes"),   # head_dim 16 (16x16x4 P.V): 4 query tiles x 128 heads
])
def test_folded_grid_one_round(gpu_ready, batch, seq_len, heads, head_dim, mask_mode):
    # An unpaired causal fp32 grid that is resident in one round (more
    # workgroups than CUs, at most two per CU) runs its query tiles in folded
    # order - heavy tiles descending, then light tiles ascending - so the two
    # workgroups of a CU carry tiles of opposite weight.  Every head is
    # compared with the oracle.
    rng = torch.Generator().manual_seed(seq_len + heads)
    shape = (batch, seq_len, heads, head_dim)
    q, k, v = (torch.randn(shape, generator=rng) for _ in range(3))
    if mask_mode == "holes":
        mask = torch.rand(batch, seq_len, generator=rng) > 0.3
        mask[1, :200] = False  # left padding: rows with no allowed key
    else:
        mask = make_mask(mask_mode, batch, seq_len)
    actual = run_hip(q, k, v, mask, True)
    reference = oracle(q, k, v, mask, True)
    assert contract_failures(actual, reference) == 0
    tight_check(actual, reference, torch.float32)
    if mask_mode == "holes":
        assert bool((actual[1, :200] == 0).all())


@pytest.mark.parametrize("case_seed", range(24))
def test_randomized_grid_filling_shapes(gpu_ready, case_seed):
    # Random shapes large enough for the fp32 schedules that only appear on
    # full grids: the paired grid (ceil(nq/2)*B*H >= 2 workgroups per CU),
    # the folded one-round grid (CUs < nq*B*H <= 2*CUs) and the plain
    # heaviest-first grid, with causal or not, key masks with left padding
    # and holes, head dims 8-64 and BSHD or packed layouts.  Two heads (the
    # first and a random one) of every batch element go to the oracle.
    rng = torch.Generator().manual_seed(7000 + case_seed)
    pick = lambda seq: seq[int(torch.randint(len(seq), (1,), generator=rng))]  # noqa: E731
    batch = int(torch.randint(2, 9, (1,), generator=rng))
    heads = int(torch.randint(12, 41, (1,), generator=rng))
    seq_len = int(torch.randint(300, 1301, (1,), generator=rng))
    head_dim = pick([8, 16, 32, 64])
    causal = bool(torch.randint(4, (1,), generator=rng)) != 0  # mostly causal
    layout = pick(["contiguous", "packed"])
    q, k, v = _layout_inputs((batch, seq_len, heads, head_dim), layout, rng)
    pad = torch.randint(0, seq_len // 3, (batch, 1), generator=rng)
    mask = (torch.arange(seq_len)[None, :] >= pad) & (torch.rand(batch, seq_len, generator=rng) > 0.15)
    actual = run_hip(q, k, v, mask, causal)
    other = int(torch.randint(1, heads, (1,), generator=rng))
    for hh in (0, other):
        sl = slice(hh, hh + 1)
        reference = oracle(q[:, :, sl].cpu(), k[:, :, sl].cpu(), v[:, :, sl].cpu(), mask, causal)
        assert contract_failures(actual[:, :, sl], reference) == 0, (
            f"B={batch} S={seq_len} H={heads} D={head_dim} causal={causal} layout={layout} head={hh}")
        tight_check(actual[:, :, sl], reference, torch.float32)


def _layout_inputs(shape, layout: str, rng: torch.Generator, dtype=torch.float32):
    """q, k, v on the GPU as contiguous BSHD, permuted BHSD views or packed-QKV views."""
    batch, seq_len, heads, head_dim = shape
    dev = torch.device("cuda")
    if layout == "packed":
        packed = torch.randn(batch, seq_len, 3, heads, head_dim, generator=rng).to(dtype).to(dev)
        return packed.unbind(dim=2)
    if layout == "bhsd":
        return tuple(torch.randn(batch, heads, seq_len, head_dim, generator=rng).to(dtype).to(dev).transpose(1, 2)
                     for _ in range(3))
    return tuple(torch.randn(shape, generator=rng).to(dtype).to(dev) for _ in range(3))


@pytest.mark.parametrize("batch,seq_len,heads,head_dim,mask_mode,layout", [
    (3, 64, 3, 64, "holes", "contiguous"),  # B*H = 9: the last workgroup has one pair
    (1, 1, 1, 64, "none", "contiguous"),
    (2, 33, 5, 32, "prefix", "bhsd"),
    (5, 17, 1, 16, "holes", "packed"),
    (4, 64, 2, 8, "none", "packed"),
    (1, 64, 7, 64, "prefix", "bhsd"),
    (2, 32, 3, 64, "holes", "contiguous"),
    (2, 50, 3, 128, "holes", "bhsd"),      # head_dim 128: 64-key tiles when non-causal
])
def test_twin_grid_short_sequences(gpu_ready, batch, seq_len, heads, head_dim, mask_mode, layout):
    # fp32 non-causal attention with S <= 64 (one key tile; a 128-query tile
    # has rows for two of its four wavefronts) runs two (batch, head) pairs
    # per workgroup, wavefronts 0-1 on pair 2i and 2-3 on pair 2i + 1, each
    # pair's keys in its own LDS buffer.  Odd B*H leaves the second pair of
    # the last workgroup empty.  Every head is compared with the oracle.
    rng = torch.Generator().manual_seed(batch * 1000 + seq_len * 10 + heads + head_dim)
    q, k, v = _layout_inputs((batch, seq_len, heads, head_dim), layout, rng)
    if mask_mode == "holes":
        mask = torch.rand(batch, seq_len, generator=rng) > 0.4
        mask[0, :] = False  # one batch element with no valid key: zero rows
    else:
        mask = make_mask(mask_mode, batch, seq_len)
    for scale in (None, 0.3):
        actual = run_hip(q, k, v, mask, False, scale)
        reference = oracle(q.cpu(), k.cpu(), v.cpu(), mask, False, scale)
        assert contract_failures(actual, reference) == 0, f"scale={scale}"
        tight_check(actual, reference, torch.float32)
    if mask_mode == "holes":
        assert bool((actual[0] == 0).all())


@pytest.mark.parametrize("batch,seq_len,heads,head_dim,mask_mode,layout", [
    (512, 64, 8, 64, "none", "packed"),    # config 5b: 8192 items, 4 per wavefront
    (64, 40, 41, 32, "none", "contiguous"),  # ragged S, items not a multiple of the grid
    (96, 32, 23, 64, "none", "bhsd"),      # S = 32: one 32-query half per head
    (40, 9, 61, 64, "prefix", "packed"),   # S < 32 with key masks
    (33, 64, 65, 32, "holes", "bhsd"),
])
def test_short_sequence_persistent_grid(gpu_ready, batch, seq_len, heads, head_dim, mask_mode, layout):
    # fp32 non-causal S <= 64 with head_dim 32 / 64: one wavefront per (batch,
    # head, 32-query half), operands loaded straight into registers, a
    # persistent grid whose wavefronts walk several items and prefetch the
    # next one.  Every head against the oracle; a second call must agree
    # bitwise (the schedule is static).
    rng = torch.Generator().manual_seed(batch * 7 + seq_len * 3 + heads + head_dim)
    q, k, v = _layout_inputs((batch, seq_len, heads, head_dim), layout, rng)
    if mask_mode == "holes":
        mask = torch.rand(batch, seq_len, generator=rng) > 0.4
        mask[1, :] = False
    else:
        mask = make_mask(mask_mode, batch, seq_len)
    actual = run_hip(q, k, v, mask, False)
    reference = oracle(q.cpu(), k.cpu(), v.cpu(), mask, False)
    assert contract_failures(actual, reference) == 0
    tight_check(actual, reference, torch.float32)
    assert torch.equal(run_hip(q, k, v, mask, False), actual)
    if mask_mode == "holes":
        assert bool((actual[1] == 0).all())


def _short_case(rng: torch.Generator):
    """One randomized fp32 non-causal case with S <= 64 (the short-sequence kernel)."""
    pick = lambda seq: seq[int(torch.randint(len(seq), (1,), generator=rng))]  # noqa: E731
    batch = int(torch.randint(1, 41, (1,), generator=rng))
    seq_len = int(torch.randint(1, 65, (1,), generator=rng))
    heads = int(torch.randint(1, 41, (1,), generator=rng))
    head_dim = pick([32, 64])
    mask_mode = pick(["none", "none", "prefix", "holes"])
    layout = pick(["contiguous", "bhsd", "packed"])
    scale = pick([None, None, 0.05, 0.3])
    return batch, seq_len, heads, head_dim, mask_mode, layout, scale


@pytest.mark.parametrize("case_seed", range(48))
def test_randomized_short_sequences(gpu_ready, case_seed):
    # Seeded random sweep of the short-sequence kernel's envelope: B and H up
    # to 40 (up to 3200 items, so some wavefronts walk two), S from 1 to 64
    # (one or two 32-query halves, ragged key ends), head dims 32 and 64,
    # every layout, prefix and holed masks, default and explicit scales.
    rng = torch.Generator().manual_seed(7000 + case_seed)
    batch, seq_len, heads, head_dim, mask_mode, layout, scale = _short_case(rng)
    q, k, v = _layout_inputs((batch, seq_len, heads, head_dim), layout, rng)
    if mask_mode == "holes":
        mask = torch.rand(batch, seq_len, generator=rng) > 0.35
    else:
        mask = make_mask(mask_mode, batch, seq_len)
    actual = run_hip(q, k, v, mask, False, scale=scale)
    reference = oracle(q.cpu(), k.cpu(), v.cpu(), mask, False, scale=scale)
    label = f"case {case_seed}: {(batch, seq_len, heads, head_dim)} mask={mask_mode} layout={layout} scale={scale}"
    assert contract_failures(actual, reference) == 0, label
    tight_check(actual, reference, torch.float32)
    if mask is not None:
        empty = ~mask.any(dim=1)
        assert bool((actual[empty] == 0).all()), label


def test_twin_grid_config5b_shape_with_padding(gpu_ready):
    # Config 5b's attention (fp32, B=512, S=64, H=8, D=64, non-causal) with
    # right padding of every length 1..64 and random holes, every head
    # against the oracle.
    rng = torch.Generator().manual_seed(55)
    batch, seq_len, heads, head_dim = 512, 64, 8, 64
    q, k, v = _layout_inputs((batch, seq_len, heads, head_dim), "packed", rng)
    lengths = torch.arange(batch) % seq_len + 1
    mask = torch.arange(seq_len)[None, :] < lengths[:, None]
    mask[::7] &= torch.rand(mask[::7].shape, generator=rng) > 0.25
    actual = run_hip(q, k, v, mask, False)
    reference = oracle(q.cpu(), k.cpu(), v.cpu(), mask, False)
    assert contract_failures(actual, reference) == 0
    tight_check(actual, reference, torch.float32)


def _random_case(rng: torch.Generator, max_len: int = 300):
    """One randomized attention case: shapes, dtype, layout, mask and scale."""
    pick = lambda seq: seq[int(torch.randint(len(seq), (1,), generator=rng))]  # noqa: E731
    batch = int(torch.randint(1, 4, (1,), generator=rng))
    seq_len = int(torch.randint(1, max_len + 1, (1,), generator=rng))
    heads = int(torch.randint(1, 5, (1,), generator=rng))
    head_dim = pick([8, 16, 32, 64, 128])
    dtype = pick([torch.float32, torch.bfloat16, torch.float16])
    causal = bool(torch.randint(2, (1,), generator=rng))
    mask_mode = pick(["none", "prefix", "holes"])
    layout = pick(["contiguous", "bhsd", "packed"])
    scale = pick([None, None, 0.05, 0.3])
    return batch, seq_len, heads, head_dim, dtype, causal, mask_mode, layout, scale


@pytest.mark.parametrize("case_seed", list(range(120)) + list(range(5000, 5060)))
def test_randomized_shapes_layouts_and_masks(gpu_ready, case_seed):
    # Seeded random sweep over everything the contract admits at small sizes:
    # head dims, dtypes, causal or not, ragged lengths, default or explicit
    # scales, contiguous / permuted (BHSD strides) / packed-QKV layouts, and
    # key masks as prefixes or with random holes (valid and invalid keys
    # interleaved inside tiles).  Seeds from 5000 draw lengths up to 1100, so
    # the steady multi-tile loop meets the masks too.
    rng = torch.Generator().manual_seed(1000 + case_seed)
    batch, seq_len, heads, head_dim, dtype, causal, mask_mode, layout, scale = _random_case(
        rng, 1100 if case_seed >= 5000 else 300)
    shape = (batch, seq_len, heads, head_dim)
    dev = torch.device("cuda")
    if layout == "packed":
        packed = torch.randn(batch, seq_len, 3, heads, head_dim, generator=rng).to(dtype).to(dev)
        q, k, v = packed.unbind(dim=2)
    elif layout == "bhsd":
        q, k, v = (torch.randn(batch, heads, seq_len, head_dim, generator=rng).to(dtype).to(dev).transpose(1, 2)
                   for _ in range(3))
    else:
        q, k, v = (torch.randn(shape, generator=rng).to(dtype).to(dev) for _ in range(3))
    if mask_mode == "holes":
        mask = torch.rand(batch, seq_len, generator=rng) > 0.35
    else:
        mask = make_mask(mask_mode, batch, seq_len)
    actual = run_hip(q, k, v, mask, causal, scale=scale)
    reference = oracle(q.cpu(), k.cpu(), v.cpu(), mask, causal, scale=scale)
    label = f"case {case_seed}: {shape} {dtype} causal={causal} mask={mask_mode} layout={layout} scale={scale}"
    assert actual.shape == shape and actual.dtype == dtype, label
    assert contract_failures(actual, reference) == 0, label
    if scale is None:
        tight_check(actual, reference, dtype)
    if mask is not None:
        # Rows with no allowed key are exact zeros.
        allowed = mask[:, None, :].expand(batch, seq_len, seq_len)
        if causal:
            allowed = allowed & torch.ones(seq_len, seq_len, dtype=torch.bool).tril()[None]
        empty = ~allowed.any(dim=2)
        assert bool((actual[empty] == 0).all()), label


@pytest.mark.parametrize("seq_len", [1024, 4096])
def test_baseline_size_every_head_matches_chunked_oracle(gpu_ready, seq_len):
    # BASELINE config 2 geometry (B=8, H=16, D=64, fp32), causal and not:
    # the chunked oracle evaluates all 128 (batch, head) pairs, so every
    # output element of the full-size launch is compared.
    g = torch.Generator().manual_seed(29)
    shape = (8, seq_len, 16, 64)
    q, k, v = (torch.randn(shape, generator=g) for _ in range(3))
    for causal in (True, False):
        out = run_hip(q, k, v, None, causal)
        reference = chunked_kernel_contract_attention(q, k, v, None, causal)
        actual = out.permute(0, 2, 1, 3).reshape(8 * 16, seq_len, 64)
        assert contract_failures(actual, reference) == 0, f"causal={causal}"
        tight_check(actual, reference, torch.float32)


def test_determinism_bitwise(gpu_ready):
    g = torch.Generator().manual_seed(31)
    q = torch.randn(2, 1000, 8, 64, generator=g)
    k, v = torch.randn(q.shape, generator=g), torch.randn(q.shape, generator=g)
    a = run_hip(q, k, v, None, True)
    b = run_hip(q, k, v, None, True)
    assert torch.equal(a, b)


def _causal_rounding_attention_fp32_gpu(q, k, v, chunk=2048):
    """``kernel_rounding_attention`` for causal launches, restated in fp32
    torch on the GPU so that every row of a full-size launch can be checked:
    one head and one block of query rows at a time, keys up to the block's
    last row.  fp32 products and sums stand in for the model's exact
    products rounded once (a relative difference of ~1e-6, far inside the
    contract); the callers pin it against the float64 model on sampled rows.
    Returns float32 [B, S, H, D] on q's device."""
    batch, seq_len, heads, head_dim = q.shape
    sign, c = _exp2_scale(head_dim, None)
    dev = q.device
    out = torch.empty(q.shape, dtype=torch.float32, device=dev)
    keys = torch.arange(seq_len, device=dev)
    for b in range(batch):
        for h in range(heads):
            qh = q[b, :, h, :].float() * sign
            kt = k[b, :, h, :].float().t().contiguous()
            vh = v[b, :, h, :].float().contiguous()
            for start in range(0, seq_len, chunk):
                end = min(seq_len, start + chunk)
                s = qh[start:end] @ kt[:, :end]
                s = s.masked_fill(keys[None, :end] > keys[start:end, None], float("-inf"))
                ref = torch.ceil(s.max(dim=1).values * c)
                rounded = torch.exp2(s * c - ref[:, None]).to(q.dtype).float()
                out[b, start:end, h] = (rounded @ vh[:end]) / rounded.sum(dim=1, keepdim=True)
    return out


def test_config5a_long_sequence_bf16_rows_and_memory(gpu_ready):
    # BASELINE config 5a: causal bf16, B=1, H=32, S=16384, D=128, run at full
    # size.  The float64 rounding model on every head at four row blocks -
    # start, middle and end of the sequence, where the rows meet 128 to 16384
    # keys - and its fp32 GPU restatement on every row of every head.
    # Memory: the kernel keeps no workspace, so with a caller-owned output a
    # launch allocates nothing at all.
    from transformer_opt.kernels import hip_attention

    batch, seq_len, heads, head_dim = 1, 16384, 32, 128
    g = torch.Generator().manual_seed(37)
    q, k, v = (torch.randn(batch, seq_len, heads, head_dim, generator=g).to(torch.bfloat16)
               for _ in range(3))
    dev = torch.device("cuda")
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    out = torch.empty_like(qd)
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    before = torch.cuda.memory_allocated()
    with torch.inference_mode():
        hip_attention(qd, kd, vd, causal=True, out=out)
    torch.cuda.synchronize()
    assert torch.cuda.max_memory_allocated() == before
    result = out.cpu()
    assert torch.isfinite(result).all()
    pairs = [(0, h) for h in range(heads)]
    atol, rtol = CONTRACT[torch.bfloat16]
    with torch.inference_mode():
        every_row = _causal_rounding_attention_fp32_gpu(qd, kd, vd)
    for rows in (slice(0, 128), slice(5000, 5128), slice(8128, 8256), slice(16256, 16384)):
        reference = kernel_rounding_attention(q, k, v, None, True, heads=pairs, query_rows=rows)
        actual = torch.stack([result[b, rows, h, :] for b, h in pairs])
        assert contract_failures(actual, reference) == 0, f"rows {rows}"
        # The fp32 GPU restatement meets the contract against the float64 model
        # on these rows, and stays close on average (its fp32 score sums flip
        # the bf16 rounding of a few probabilities, as the kernel's do).
        restated = torch.stack([every_row[b, rows, h, :] for b, h in pairs]).double().cpu()
        gap = (restated - reference).abs()
        assert bool(((gap <= atol) | (gap <= rtol * reference.abs())).all()), f"rows {rows}"
        assert gap.mean().item() < 5e-5, f"rows {rows}: mean gap {gap.mean().item():.3g}"
    # Every row of every head against the restatement, under the same contract.
    err = (out.float() - every_row).abs()
    ok = torch.isfinite(out.float()) & ((err <= atol) | (err <= rtol * every_row.abs()))
    assert bool(ok.all()), f"failed={int((~ok).sum())}/{ok.numel()} max_abs={err.max().item():.3g}"


# ------------------------------------------------------------------ key split --
def _abi_attention(q, k, v, mask, causal, workspace=None):
    """One launch through the C ABI: ttk_attention_fwd, or ttk_attention_fwd_ws
    with ``workspace`` (a uint8 device tensor) when given."""
    from transformer_opt import _native
    from transformer_opt.kernels.attention import _DTYPE_CODE

    lib = _native.load()
    out = torch.empty_like(q)
    B, S, H, D = q.shape
    args = [q.data_ptr(), k.data_ptr(), v.data_ptr(), None if mask is None else mask.data_ptr(),
            out.data_ptr(), _DTYPE_CODE[q.dtype], B, S, H, D,
            _native.strides3(q.stride()[:3]), _native.strides3(k.stride()[:3]),
            _native.strides3(v.stride()[:3]),
            None if mask is None else _native.strides2(mask.stride()),
            _native.strides3(out.stride()[:3]), D ** -0.5, 1 if causal else 0]
    stream = torch.cuda.current_stream().cuda_stream
    if workspace is None:
        status = lib.ttk_attention_fwd(*args, stream)
    else:
        status = lib.ttk_attention_fwd_ws(*args, workspace.data_ptr(), workspace.numel(), stream)
    _native.check(status, "attention")
    return out


@pytest.mark.parametrize("batch,seq_len,heads,head_dim,dtype,mask_mode", [
    (1, 4096, 4, 64, torch.bfloat16, "none"),
    (1, 1024, 2, 64, torch.float16, "prefix"),
    (2, 1300, 3, 32, torch.bfloat16, "holes"),
    (1, 2048, 2, 128, torch.bfloat16, "none"),
    (1, 777, 5, 16, torch.float16, "none"),
    (1, 3000, 1, 8, torch.bfloat16, "prefix"),
])
def test_key_split_schedule_matches_oracle_and_unsplit_launch(gpu_ready, batch, seq_len, heads,
                                                              head_dim, dtype, mask_mode):
    # A causal 16-bit launch with few resident rounds splits its heavy query
    # tiles into key chunks whose partial states the last chunk merges.  The
    # split launch, the unsplit one (no workspace) and the oracle agree, the
    # arrival counters are zero again afterwards and a second split launch is
    # bitwise identical (the merge sums the chunks in a fixed order).
    from transformer_opt import _native

    lib = _native.load()
    nbytes = lib.ttk_attention_workspace_size(1 if dtype == torch.bfloat16 else 2, batch, seq_len,
                                              heads, head_dim, 1)
    assert nbytes > 0, "the shape should take the key-split schedule"
    g = torch.Generator().manual_seed(seq_len + head_dim)
    shape = (batch, seq_len, heads, head_dim)
    q, k, v = (torch.randn(shape, generator=g).to(dtype) for _ in range(3))
    mask = None
    if mask_mode == "prefix":
        mask = make_mask("prefix", batch, seq_len)
    elif mask_mode == "holes":
        mask = torch.rand(batch, seq_len, generator=g) > 0.2
        mask[:, 0] = True
    dev = torch.device("cuda")
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    md = None if mask is None else mask.to(dev)
    workspace = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
    with torch.inference_mode():
        split = _abi_attention(qd, kd, vd, md, True, workspace)
        again = _abi_attention(qd, kd, vd, md, True, workspace)
        whole = _abi_attention(qd, kd, vd, md, True)
    torch.cuda.synchronize()
    assert int(workspace[:_native.ATTENTION_WS_COUNTER_BYTES].count_nonzero()) == 0
    assert torch.equal(split, again)
    reference = oracle(q, k, v, mask, True)
    assert contract_failures(split.cpu(), reference) == 0
    assert contract_failures(whole.cpu(), reference) == 0


@pytest.mark.parametrize("seq_len,dtype,causal,mask_mode", [
    (4096, torch.bfloat16, True, "none"),
    (4096, torch.float16, False, "prefix"),
    (4097, torch.bfloat16, True, "none"),
    (4097, torch.float16, True, "prefix"),
    (4160, torch.float16, False, "prefix"),
    (4223, torch.bfloat16, True, "prefix"),
    (1024, torch.bfloat16, False, "none"),
    (1025, torch.float16, False, "none"),
    (2100, torch.bfloat16, False, "none"),
])
def test_head_dim_128_tile_size_switch(gpu_ready, seq_len, dtype, causal, mask_mode):
    # 16-bit head_dim 128 runs 32-key tiles (three workgroups per CU) up to
    # S = 4096 when causal or key-masked and up to 1024 otherwise, and 64-key
    # tiles, two workgroups per CU, above that (without a workspace: no key
    # split).  Both sides of each switch, with and without key masks, ragged
    # last tiles of either size.
    g = torch.Generator().manual_seed(seq_len + (7 if causal else 0))
    shape = (2, seq_len, 1, 128)
    q, k, v = (torch.randn(shape, generator=g).to(dtype) for _ in range(3))
    mask = make_mask(mask_mode, 2, seq_len)
    dev = torch.device("cuda")
    with torch.inference_mode():
        actual = _abi_attention(q.to(dev), k.to(dev), v.to(dev),
                                None if mask is None else mask.to(dev), causal)
    reference = oracle(q, k, v, mask, causal)
    assert contract_failures(actual.cpu(), reference) == 0


@pytest.mark.parametrize("seq_len,head_dim,dtype,mask_mode", [
    (1024, 64, torch.bfloat16, "none"),
    (1025, 64, torch.bfloat16, "none"),
    (1000, 64, torch.float16, "none"),
    (2048, 64, torch.float16, "prefix"),
    (2049, 64, torch.bfloat16, "prefix"),
    (1500, 64, torch.bfloat16, "prefix"),
    (1024, 32, torch.bfloat16, "none"),
    (1025, 32, torch.float16, "none"),
    (333, 32, torch.bfloat16, "none"),
    (700, 32, torch.float16, "prefix"),
])
def test_causal_small_head_dim_tile_size_switch(gpu_ready, seq_len, head_dim, dtype, mask_mode):
    # Causal 16-bit head_dim 64 and 32 run 32-key tiles (four workgroups per
    # CU) up to S = 1024 (head_dim 64 with a key mask: 2048) and 64-key
    # tiles otherwise (without a workspace: no key split).  Both sides of
    # each switch.
    g = torch.Generator().manual_seed(seq_len + head_dim)
    shape = (2, seq_len, 2, head_dim)
    q, k, v = (torch.randn(shape, generator=g).to(dtype) for _ in range(3))
    mask = make_mask(mask_mode, 2, seq_len)
    dev = torch.device("cuda")
    with torch.inference_mode():
        actual = _abi_attention(q.to(dev), k.to(dev), v.to(dev),
                                None if mask is None else mask.to(dev), True)
    reference = oracle(q, k, v, mask, True)
    assert contract_failures(actual.cpu(), reference) == 0


# Split shapes in an order whose split plans grow and then shrink (more
# split slots, larger partial states, then fewer): each launch finds the
# previous launch's partial states in the workspace.
SPLIT_SEQUENCE = [
    (1, 2048, 2, 64, torch.bfloat16),
    (1, 4096, 4, 64, torch.bfloat16),
    (1, 4096, 4, 128, torch.bfloat16),
    (1, 4096, 16, 32, torch.float16),
    (2, 4096, 4, 64, torch.bfloat16),
    (1, 1024, 2, 64, torch.float16),
]


def _split_inputs(shape, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    return tuple(torch.randn(shape, generator=g).to(dtype) for _ in range(3))


def test_key_split_one_workspace_across_shapes(gpu_ready):
    # One caller workspace, sized for the largest plan, serves every shape in
    # turn: each split launch equals the same launch on a fresh zero-filled
    # workspace bitwise, and the counter block is zero after every launch.
    from transformer_opt import _native

    lib = _native.load()
    sizes = []
    for (b, s, h, d, dtype) in SPLIT_SEQUENCE:
        code = 1 if dtype == torch.bfloat16 else 2
        sizes.append(lib.ttk_attention_workspace_size(code, b, s, h, d, 1))
        assert sizes[-1] > 0, (b, s, h, d)
    shared = torch.zeros(max(sizes), dtype=torch.uint8, device="cuda")
    for i, (b, s, h, d, dtype) in enumerate(SPLIT_SEQUENCE):
        q, k, v = (t.cuda() for t in _split_inputs((b, s, h, d), dtype, 40 + i))
        with torch.inference_mode():
            got = _abi_attention(q, k, v, None, True, shared)
            fresh = _abi_attention(q, k, v, None, True,
                                   torch.zeros(sizes[i], dtype=torch.uint8, device="cuda"))
        torch.cuda.synchronize()
        assert torch.equal(got, fresh), (b, s, h, d)
        assert int(shared[:_native.ATTENTION_WS_COUNTER_BYTES].count_nonzero()) == 0


def test_key_split_through_the_wrapper_across_shapes(gpu_ready):
    # The product wrapper keeps one workspace per stream and reuses it for
    # every shape: its outputs equal fresh-workspace launches bitwise, and
    # the smaller shapes stay within the oracle's bound.
    from transformer_opt.kernels.attention import hip_attention
    from transformer_opt import _native

    lib = _native.load()
    for i, (b, s, h, d, dtype) in enumerate(SPLIT_SEQUENCE):
        cpu = _split_inputs((b, s, h, d), dtype, 60 + i)
        q, k, v = (t.cuda() for t in cpu)
        code = 1 if dtype == torch.bfloat16 else 2
        nbytes = lib.ttk_attention_workspace_size(code, b, s, h, d, 1)
        with torch.inference_mode():
            got = hip_attention(q, k, v, causal=True)
            fresh = _abi_attention(q, k, v, None, True,
                                   torch.zeros(nbytes, dtype=torch.uint8, device="cuda"))
        torch.cuda.synchronize()
        assert torch.equal(got, fresh), (b, s, h, d)
        if s * h <= 8192:
            reference = oracle(*cpu, None, True)
            assert contract_failures(got.cpu(), reference) == 0, (b, s, h, d)


def test_key_split_workspace_rules(gpu_ready):
    # Too small a workspace runs the unsplit schedule (same result as no
    # workspace, bitwise); an unaligned one is rejected before any launch.
    from transformer_opt import _native

    lib = _native.load()
    g = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn(1, 1024, 2, 64, generator=g).to(torch.bfloat16).cuda() for _ in range(3))
    nbytes = lib.ttk_attention_workspace_size(1, 1, 1024, 2, 64, 1)
    assert nbytes > 0 and lib.ttk_attention_workspace_size(1, 1, 1024, 2, 64, 0) == 0
    small = torch.zeros(nbytes - 256, dtype=torch.uint8, device="cuda")
    with torch.inference_mode():
        assert torch.equal(_abi_attention(q, k, v, None, True, small), _abi_attention(q, k, v, None, True))
        big = torch.zeros(nbytes + 512, dtype=torch.uint8, device="cuda")
        with pytest.raises(ValueError, match="256-byte aligned"):
            _abi_attention(q, k, v, None, True, big[16:])
