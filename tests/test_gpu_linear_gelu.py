"""Fused Linear + exact GELU (HIP) vs a float32 CPU reference.

The reference computes gelu(x @ w.T + b) with the exact erf GELU in float32 on
the same bf16/fp16-rounded inputs, as the model's
``F.gelu(layer.ffn_in(...), approximate="none")`` (reference
transformer_opt/submission.py:507) does in spirit.  The kernel accumulates in
fp32 and rounds once to the storage type, so every element must lie within
one rounding of the float32 value: ``|d| <= 2^-8 * |ref|`` (bf16) or
``2^-10 * |ref|`` (fp16), plus 1e-4 absolute for values near zero (fp32
summation order over K terms).
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu

REL = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -10}


def reference(x, w, b):
    y = x.float() @ w.float().T
    if b is not None:
        y = y + b.float()
    return F.gelu(y, approximate="none")


def run(x, w, b):
    from transformer_opt.kernels import linear_gelu

    dev = torch.device("cuda")
    with torch.inference_mode():
        out = linear_gelu(x.to(dev), w.to(dev), None if b is None else b.to(dev))
    return out.cpu()


def check(actual, ref, dtype):
    err = (actual.float() - ref).abs()
    bound = 1e-4 + REL[dtype] * ref.abs()
    bad = ~(err <= bound)
    assert torch.isfinite(actual.float()).all()
    assert not bool(bad.any()), f"{int(bad.sum())} elements out of bound, max_abs={err.max().item():.3g}"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,n,k,bias", [
    (1, 4, 64, True),
    (300, 260, 128, True),     # partial tiles in both M and N
    (256, 256, 64, False),     # one exact tile, no bias
    (513, 1024, 512, True),
    (64, 2048, 1024, True),
])
def test_linear_gelu_matches_float32_reference(gpu_ready, dtype, m, n, k, bias):
    g = torch.Generator().manual_seed(m * 7 + n + k)
    x = torch.randn(m, k, generator=g).to(dtype)
    w = (torch.randn(n, k, generator=g) * k ** -0.5).to(dtype)
    b = (torch.randn(n, generator=g) * 0.1).to(dtype) if bias else None
    check(run(x, w, b), reference(x, w, b), dtype)


def test_config4_ffn_in_full_size(gpu_ready):
    # The config-4 encoder's FFN input projection: tokens 4*2048, d=1024 ->
    # 4096, bf16, [B, S, d] input; rows sampled across the whole output.
    g = torch.Generator().manual_seed(5)
    x = torch.randn(4, 2048, 1024, generator=g).to(torch.bfloat16)
    w = (torch.randn(4096, 1024, generator=g) * 1024 ** -0.5).to(torch.bfloat16)
    b = (torch.randn(4096, generator=g) * 0.1).to(torch.bfloat16)
    out = run(x, w, b)
    assert out.shape == (4, 2048, 4096) and out.dtype == torch.bfloat16
    rows = torch.tensor([0, 1, 255, 256, 2047, 4100, 6000, 8191])
    flat = x.reshape(-1, 1024)
    check(out.reshape(-1, 4096)[rows], reference(flat[rows], w, b), torch.bfloat16)


@pytest.mark.parametrize("n,ldy_pad", [(260, 4), (260, 0), (512, 8)])
def test_strided_operands_through_the_c_abi(gpu_ready, n, ldy_pad):
    # Row strides wider than the rows: x and w as column slices of wider
    # buffers, y written into a wider buffer whose pad columns must stay
    # untouched.  n=260 with ldy=264 takes the 16-byte store path with a
    # 4-feature tail; ldy=260 takes the 8-byte path.
    from transformer_opt import _native

    lib = _native.load()
    m, k = 300, 192
    g = torch.Generator().manual_seed(n + ldy_pad)
    xs = torch.randn(m, k + 64, generator=g).to(torch.bfloat16)
    ws = (torch.randn(n, k + 8, generator=g) * k ** -0.5).to(torch.bfloat16)
    b = (torch.randn(n, generator=g) * 0.1).to(torch.bfloat16)
    dev = torch.device("cuda")
    xd, wd, bd = xs.to(dev), ws.to(dev), b.to(dev)
    ld_y = n + ldy_pad
    yd = torch.full((m, ld_y), 7.0, device=dev, dtype=torch.bfloat16)
    status = lib.ttk_linear_gelu_fwd(xd.data_ptr(), wd.data_ptr(), bd.data_ptr(), yd.data_ptr(), 1,
                                     m, n, k, k + 64, k + 8, ld_y, torch.cuda.current_stream().cuda_stream)
    _native.check(status, "linear_gelu")
    y = yd.cpu()
    check(y[:, :n], reference(xs[:, :k], ws[:, :k], b), torch.bfloat16)
    assert bool((y[:, n:] == 7.0).all())


def test_unsupported_inputs_raise(gpu_ready):
    from transformer_opt.kernels import linear_gelu, linear_gelu_supported

    x = torch.randn(4, 96, device="cuda", dtype=torch.bfloat16)
    w = torch.randn(8, 96, device="cuda", dtype=torch.bfloat16)
    assert not linear_gelu_supported(x, w, None)
    with pytest.raises(ValueError):
        linear_gelu(x, w)
    x32 = torch.randn(4, 64, device="cuda")
    assert not linear_gelu_supported(x32, torch.randn(8, 64, device="cuda"), None)
