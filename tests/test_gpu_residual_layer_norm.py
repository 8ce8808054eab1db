"""HIP fused residual + LayerNorm vs the CPU oracle.

Mirrors the reference tests/test_gpu_residual_layer_norm.py: the residual must
be BITWISE equal to the eager ``x + u`` (:75), the normalized output within
1e-5 of ``F.layer_norm`` (:76-81), all four mask/zeroing combinations
(:18-26) and the no-bias form (:84-113) - plus every width of BASELINE
config 3, the vector and fallback kernels, and bf16/fp16 rows.
"""

from __future__ import annotations

import pytest
import torch

from oracle.layernorm import brute_force_layer_norm_f64, explicit_residual_layer_norm

pytestmark = pytest.mark.gpu


def run_hip(x, u, w, b, eps, mask, zr=False, zn=False):
    from transformer_opt.kernels import fused_residual_layer_norm

    dev = torch.device("cuda")
    with torch.inference_mode():
        r, y = fused_residual_layer_norm(
            x.to(dev), u.to(dev), w.to(dev), None if b is None else b.to(dev), eps,
            None if mask is None else mask.to(dev),
            zero_invalid_residual=zr, zero_invalid_normalized=zn,
        )
    return r.cpu(), y.cpu()


@pytest.mark.parametrize(
    "masked,zero_residual,zero_normalized",
    [(False, False, False), (True, False, False), (True, True, False), (True, True, True)],
)
def test_fused_residual_layer_norm_matches_explicit_operations(gpu_ready, masked, zero_residual,
                                                               zero_normalized):
    g = torch.Generator().manual_seed(7018)
    x = torch.randn(2, 17, 128, generator=g)
    u = torch.randn(x.shape, generator=g)
    w = torch.randn(128, generator=g)
    b = torch.randn(128, generator=g)
    mask = None
    if masked:
        mask = torch.arange(17)[None, :] < torch.tensor([[17], [9]])
    er, ey = explicit_residual_layer_norm(x, u, w, b, 1e-5, mask,
                                          zero_invalid_residual=zero_residual,
                                          zero_invalid_normalized=zero_normalized)
    r, y = run_hip(x, u, w, b, 1e-5, mask, zero_residual, zero_normalized)
    torch.testing.assert_close(r, er, rtol=0, atol=0)
    torch.testing.assert_close(y, ey, rtol=1e-5, atol=1e-5)


def test_fused_residual_layer_norm_supports_layer_norm_without_bias(gpu_ready):
    g = torch.Generator().manual_seed(7019)
    x = torch.randn(3, 5, 128, generator=g)
    u = torch.randn(x.shape, generator=g)
    w = torch.randn(128, generator=g)
    er, ey = explicit_residual_layer_norm(x, u, w, None, 1e-5)
    r, y = run_hip(x, u, w, None, 1e-5, None)
    torch.testing.assert_close(r, er, rtol=0, atol=0)
    torch.testing.assert_close(y, ey, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("hidden", [32, 96, 128, 256, 512, 768, 1000, 1024, 2048, 3072, 4096, 5120, 8192, 65536])
def test_widths_vector_and_fallback_paths(gpu_ready, hidden):
    # 1000 and 5120/8192 (fp32) exercise the block-per-row fallback.
    g = torch.Generator().manual_seed(hidden)
    rows = 37 if hidden < 65536 else 3
    x = torch.randn(rows, hidden, generator=g)
    u = torch.randn(x.shape, generator=g)
    w = torch.rand(hidden, generator=g) + 0.5
    b = torch.randn(hidden, generator=g) * 0.1
    mask = torch.rand(rows, generator=g) > 0.3
    er, ey = explicit_residual_layer_norm(x, u, w, b, 1e-5, mask,
                                          zero_invalid_residual=True, zero_invalid_normalized=True)
    r, y = run_hip(x, u, w, b, 1e-5, mask, True, True)
    torch.testing.assert_close(r, er, rtol=0, atol=0)
    torch.testing.assert_close(y, ey, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("hidden", [32, 64, 128, 1024, 1000])
def test_low_precision_rows(gpu_ready, dtype, hidden):
    g = torch.Generator().manual_seed(99)
    x = torch.randn(50, hidden, generator=g).to(dtype)
    u = torch.randn(x.shape, generator=g).to(dtype)
    w = (torch.rand(hidden, generator=g) + 0.5).to(dtype)
    b = (torch.randn(hidden, generator=g) * 0.1).to(dtype)
    er, ey = explicit_residual_layer_norm(x, u, w, b, 1e-5)
    r, y = run_hip(x, u, w, b, 1e-5, None)
    # The residual is the eager low-precision add: bitwise.
    torch.testing.assert_close(r, er, rtol=0, atol=0)
    # Normalized: within one output rounding step of the CPU reference.
    tol = 1.6e-2 if dtype == torch.bfloat16 else 2e-3
    torch.testing.assert_close(y.float(), ey.float(), rtol=tol, atol=tol)


def test_config3_rows_against_float64(gpu_ready):
    # rows = 32768, gamma ~ U(0.5, 1.5), beta ~ N(0, 0.1).
    g = torch.Generator().manual_seed(3)
    for hidden in (256, 4096):
        x = torch.randn(32768, hidden, generator=g)
        u = torch.randn(x.shape, generator=g)
        w = torch.rand(hidden, generator=g) + 0.5
        b = torch.randn(hidden, generator=g) * 0.1
        r, y = run_hip(x, u, w, b, 1e-5, None)
        assert torch.equal(r, x + u)
        # Every row (in blocks of 2048 rows, to bound host memory).
        for start in range(0, 32768, 2048):
            rows = slice(start, start + 2048)
            expected = brute_force_layer_norm_f64(r[rows].numpy(), w.numpy(), b.numpy(), 1e-5)
            assert abs(y[rows].double().numpy() - expected).max() < 1e-5, (hidden, start)


def test_constant_and_two_value_rows_closed_forms(gpu_ready):
    hidden = 256
    w = torch.linspace(0.5, 1.5, hidden)
    b = torch.linspace(-1, 1, hidden)
    x = torch.zeros(2, hidden)
    x[0] = 3.25  # constant row -> y = b exactly
    a = 0.75
    x[1, ::2] = a
    x[1, 1::2] = -a
    u = torch.zeros_like(x)
    _, y = run_hip(x, u, w, b, 1e-5, None)
    assert torch.equal(y[0], b)
    expected = torch.where(torch.arange(hidden) % 2 == 0, 1.0, -1.0) * a / (a * a + 1e-5) ** 0.5 * w + b
    assert (y[1] - expected).abs().max() < 1e-6


def test_layer_norm_only_entry(gpu_ready):
    from transformer_opt.kernels import layer_norm

    g = torch.Generator().manual_seed(5)
    x = torch.randn(4, 33, 512, generator=g)
    w = torch.randn(512, generator=g)
    b = torch.randn(512, generator=g)
    with torch.inference_mode():
        y = layer_norm(x.cuda(), w.cuda(), b.cuda(), 1e-5).cpu()
    torch.testing.assert_close(y, torch.nn.functional.layer_norm(x, (512,), w, b, 1e-5),
                               rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16], ids=["fp32", "bf16", "fp16"])
@pytest.mark.parametrize("hidden", [1, 3, 5, 33, 77, 255])
def test_odd_widths_take_the_unaligned_path(gpu_ready, dtype, hidden):
    # Rows that are not whole 16-byte vectors use the block-per-row kernel.
    # Width 1 has zero variance, so the normalized output is beta exactly.
    g = torch.Generator().manual_seed(hidden + 7)
    rows = 41
    x = torch.randn(rows, hidden, generator=g).to(dtype)
    u = torch.randn(x.shape, generator=g).to(dtype)
    w = (torch.rand(hidden, generator=g) + 0.5).to(dtype)
    b = (torch.randn(hidden, generator=g) * 0.1).to(dtype)
    mask = torch.rand(rows, generator=g) > 0.3
    er, ey = explicit_residual_layer_norm(x, u, w, b, 1e-5, mask,
                                          zero_invalid_residual=True, zero_invalid_normalized=True)
    r, y = run_hip(x, u, w, b, 1e-5, mask, True, True)
    torch.testing.assert_close(r, er, rtol=0, atol=0)
    tol = {torch.float32: 1e-5, torch.bfloat16: 1.6e-2, torch.float16: 2e-3}[dtype]
    torch.testing.assert_close(y.float(), ey.float(), rtol=tol, atol=tol)
    if hidden == 1:
        assert torch.equal(y[mask], b.expand(rows, 1)[mask])
        assert bool((y[~mask] == 0).all())


def test_zero_rows_return_empty_outputs(gpu_ready):
    from transformer_opt.kernels import layer_norm

    for dtype in (torch.float32, torch.bfloat16):
        x = torch.empty(0, 64, dtype=dtype)
        w = torch.ones(64, dtype=dtype)
        r, y = run_hip(x, x, w, None, 1e-5, None)
        assert r.shape == (0, 64) and y.shape == (0, 64)
        with torch.inference_mode():
            assert layer_norm(x.cuda(), w.cuda(), None, 1e-5).shape == (0, 64)


@pytest.mark.parametrize("rows", [1, 7, 8, 9, 4099])
@pytest.mark.parametrize("bias", [True, False])
def test_short_layer_norm_width_32(gpu_ready, rows, bias):
    # The reference's width-32 entry point (residual_layer_norm.py:129-156):
    # within float32 rounding of F.layer_norm, including row counts that are
    # not a multiple of the eight rows a wavefront takes.
    from transformer_opt.kernels import short_layer_norm

    g = torch.Generator().manual_seed(rows)
    x = torch.randn(rows, 32, generator=g) * 3.0
    w = torch.randn(32, generator=g)
    b = torch.randn(32, generator=g) if bias else None
    with torch.inference_mode():
        y = short_layer_norm(x.cuda(), w.cuda(), None if b is None else b.cuda(), 3e-4).cpu()
    torch.testing.assert_close(y, torch.nn.functional.layer_norm(x, (32,), w, b, 3e-4), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("case_seed", range(40))
def test_randomized_rows_widths_masks_and_flags(gpu_ready, case_seed):
    # Seeded random sweep: widths 1..6000 (vector and block-per-row kernels),
    # dtypes, leading shapes, row masks with both zeroing flags, optional
    # bias and eps.
    rng = torch.Generator().manual_seed(300 + case_seed)
    pick = lambda seq: seq[int(torch.randint(len(seq), (1,), generator=rng))]  # noqa: E731
    hidden = pick([1, 7, 32, 64, 96, 250, 512, 768, 1000, 1024, 2048, 4096, 6000])
    dtype = pick([torch.float32, torch.bfloat16, torch.float16])
    lead = pick([(3,), (2, 5), (1, 1, 7), (33,)])
    with_bias = bool(torch.randint(2, (1,), generator=rng))
    eps = pick([1e-5, 1e-6, 3e-4])
    masked = bool(torch.randint(2, (1,), generator=rng))
    zr = masked and bool(torch.randint(2, (1,), generator=rng))
    zn = masked and bool(torch.randint(2, (1,), generator=rng))
    x = (torch.randn(*lead, hidden, generator=rng) * 3).to(dtype)
    u = torch.randn(x.shape, generator=rng).to(dtype)
    w = (torch.rand(hidden, generator=rng) + 0.5).to(dtype)
    b = (torch.randn(hidden, generator=rng) * 0.1).to(dtype) if with_bias else None
    mask = (torch.rand(lead, generator=rng) > 0.3) if masked else None
    er, ey = explicit_residual_layer_norm(x, u, w, b, eps, mask, zero_invalid_residual=zr,
                                          zero_invalid_normalized=zn)
    r, y = run_hip(x, u, w, b, eps, mask, zr, zn)
    label = f"case {case_seed}: {tuple(x.shape)} {dtype} bias={with_bias} eps={eps} mask={masked} zr={zr} zn={zn}"
    torch.testing.assert_close(r, er, rtol=0, atol=0, msg=label)
    tol = {torch.float32: 1e-5, torch.bfloat16: 1.6e-2, torch.float16: 2e-3}[dtype]
    torch.testing.assert_close(y.float(), ey.float(), rtol=tol, atol=tol, msg=label)
