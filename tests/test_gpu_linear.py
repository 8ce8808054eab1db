"""Fused Linear + exact GELU (``ttk_linear_fwd``) against float64 references.

The reference computes the encoder FFN's input in 16-bit torch as
``F.gelu(F.linear(x, W, b))`` (transformer_opt/submission.py:507): the linear
output rounded to the dtype, the exact GELU of that rounded value rounded
again.  The checker here is the same computation in float64 on the CPU:
``pre = round(x @ W^T + b)``, ``y = round(pre * Phi(pre))`` with
``Phi(v) = erfc(-v / sqrt 2) / 2``.

Bounds: the kernel accumulates in fp32, so its rounded pre-activation can
differ from the float64 one by one unit in the last place (ulp(pre) <=
2^-7 |pre| in bf16, 2^-10 |pre| in fp16) where the exact sum lies near a
rounding boundary, and where the sum cancels (a result far smaller than
its terms) the fp32 accumulation error itself, ~sqrt(K) * 2^-24 * sum|x w|
(the library GEMM gives the same values there).  GELU's slope is at most
1.13, so an output may move by 1.13 times that plus one output rounding
step (ulp(y) <= 2^-7 |y|, 2^-10 |y|):
|d| <= 1.2 (q |pre| + 4 sqrt(K) 2^-24 sum|x w|) + q |y| + 1e-6 with q = 2^-7
(bf16) or 2^-10 (fp16), and at least 97 % of the outputs must be bit-exact.
The epilogue's GELU itself is checked bit for bit over every bf16 input.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _gelu64(v: torch.Tensor) -> torch.Tensor:
    return v * 0.5 * torch.special.erfc(-v / math.sqrt(2.0))


def _round_to(v: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Round float64 to bf16/fp16 directly (nearest, ties to even), no float32
    detour: significand scaled to the target's precision, then np.rint."""
    bits = 8 if dtype == torch.bfloat16 else 11
    a = v.numpy()
    m, e = np.frexp(a)
    if dtype == torch.float16:
        # Below fp16's normal range the quantum stays 2^-24.
        e = np.maximum(e, -13)
        m = np.ldexp(a, -e)
    q = np.ldexp(np.rint(np.ldexp(m, bits)), e - bits)
    return torch.from_numpy(q).to(dtype)


def _reference(x, w, b, gelu: bool):
    """(y, pre, acc): the float64 checker's output, its rounded pre-activation
    and the fp32 accumulation error scale 4 sqrt(K) 2^-24 sum_k |x_k w_k|."""
    pre = x.double() @ w.double().T
    if b is not None:
        pre = pre + b.double()
    acc = (x.double().abs() @ w.double().abs().T) * (4 * math.sqrt(x.shape[-1]) * 2.0 ** -24)
    pre = _round_to(pre, x.dtype)
    if not gelu:
        return pre, pre, acc
    return _round_to(_gelu64(pre.double()), x.dtype), pre, acc


def _check(actual, reference, dtype):
    expected, pre, acc = reference
    a = actual.float().cpu()
    e = expected.float()
    q = 2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -10
    err = (a - e).abs()
    ok = err <= 1.2 * (q * pre.float().abs() + acc.float()) + q * e.abs() + 1e-6
    assert bool(ok.all()), f"failed={int((~ok).sum())}/{ok.numel()} max_abs={err.max().item():.3g}"
    exact = float((a == e).float().mean())
    assert exact > 0.97, f"only {exact:.4f} of the outputs are bit-exact"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("gelu", [True, False])
@pytest.mark.parametrize("rows,out_features,in_features,bias", [
    (300, 96, 256, True),       # partial tiles in both directions, one feature tile
    (512, 4096, 1024, True),    # config 4's FFN input widths
    (777, 288, 384, False),     # ragged rows, 288 features (one full + one partial tile)
    (2048, 1024, 4096, True),   # config 4's FFN output widths
])
def test_linear_matches_float64(gpu_ready, dtype, gelu, rows, out_features, in_features, bias):
    from transformer_opt.kernels.linear import linear, linear_gelu

    g = torch.Generator().manual_seed(rows + out_features)
    x = torch.randn(rows, in_features, generator=g).to(dtype)
    w = (torch.randn(out_features, in_features, generator=g) * in_features ** -0.5).to(dtype)
    b = (torch.randn(out_features, generator=g) * 0.5).to(dtype) if bias else None
    with torch.inference_mode():
        fn = linear_gelu if gelu else linear
        y = fn(x.cuda(), w.cuda(), None if b is None else b.cuda())
    assert y.shape == (rows, out_features) and y.dtype == dtype
    _check(y, _reference(x, w, b, gelu), dtype)


def test_config4_ffn_input_every_element(gpu_ready):
    # The full config-4 FFN input: [8192, 1024] x [4096, 1024]^T + b, bf16,
    # every output against the float64 reference; the unfused route (library
    # GEMM, then the elementwise GELU kernel) is held to the same bound.
    from transformer_opt.kernels.gelu import gelu_
    from transformer_opt.kernels.linear import linear_gelu

    g = torch.Generator().manual_seed(4)
    x = torch.randn(8192, 1024, generator=g).to(torch.bfloat16)
    w = (torch.rand(4096, 1024, generator=g) * 2 - 1).mul(math.sqrt(6 / 5120)).to(torch.bfloat16)
    b = (torch.randn(4096, generator=g) * 0.02).to(torch.bfloat16)
    with torch.inference_mode():
        xd, wd, bd = x.cuda(), w.cuda(), b.cuda()
        fused = linear_gelu(xd, wd, bd)
        unfused = gelu_(torch.nn.functional.linear(xd, wd, bd))
    expected = _reference(x, w, b, True)
    _check(fused, expected, torch.bfloat16)
    _check(unfused, expected, torch.bfloat16)


def test_gelu_epilogue_on_every_bf16_input(gpu_ready):
    # Row m of X holds the bf16 value with bit pattern m in column 0 (zeros
    # elsewhere) and W has ones in column 0, so the linear output of row m is
    # that value exactly.  Inside the table the epilogue must return the
    # correctly rounded exact GELU (the table itself, checked against float64
    # on the CPU in test_oracle.py); outside it, the elementwise GELU kernel's
    # result bit for bit.
    from transformer_opt.kernels.gelu import gelu
    from transformer_opt.kernels.linear import linear_gelu

    bits = torch.arange(65536, dtype=torch.int32).to(torch.int16)
    values = bits.view(torch.bfloat16)
    x = torch.zeros(65536, 256, dtype=torch.bfloat16)
    x[:, 0] = values
    w = torch.zeros(32, 256, dtype=torch.bfloat16)
    w[:, 0] = 1
    with torch.inference_mode():
        y = linear_gelu(x.cuda(), w.cuda()).cpu()
        elementwise = gelu(values.cuda()).cpu()
    same = (y == y[:, :1]) | (y.isnan() & y[:, :1].isnan())
    assert bool(same.all())
    got = y[:, 0]
    mag = bits.to(torch.int32) & 0x7FFF
    in_table = (mag >= 0x3780) & (mag < 0x3780 + 2432)
    v64 = values.double()
    table_expected = _round_to(_gelu64(v64[in_table]), torch.bfloat16)
    assert torch.equal(got[in_table].view(torch.int16), table_expected.view(torch.int16))
    # Denormal inputs: GELU(x) = x/2 + O(x^2); the epilogue evaluates it in
    # fp32, where Phi(x) is 1/2 exactly, so the result is x/2 rounded to the
    # bf16 denormal grid - within one quantum (2^-133) of the exact value.
    denormal = ((bits.to(torch.int32) >> 7) & 0xFF) == 0
    half = values[denormal].double() / 2
    assert bool(((got[denormal].double() - half).abs() <= 2.0 ** -133).all())
    outside = ~in_table & ~values.isnan() & ~denormal
    assert torch.equal(got[outside].view(torch.int16), elementwise[outside].view(torch.int16))
    assert bool(got[values.isnan()].isnan().all())


def test_linear_rejects_what_it_cannot_run(gpu_ready):
    from transformer_opt.kernels.linear import linear_gelu, linear_supported

    x = torch.randn(16, 256, device="cuda", dtype=torch.bfloat16)
    assert linear_supported(x, torch.randn(64, 256, device="cuda", dtype=torch.bfloat16), None) is None
    for w, why in ((torch.randn(64, 200, device="cuda", dtype=torch.bfloat16), "in_features"),
                   (torch.randn(40, 256, device="cuda", dtype=torch.bfloat16), "multiple of 32"),
                   (torch.randn(64, 256, device="cuda"), "bfloat16")):
        with pytest.raises(ValueError, match=why):
            linear_gelu(x, w)
    with pytest.raises(ValueError, match="multiple of 128"):
        linear_gelu(x[:, :128].contiguous(), torch.randn(64, 128, device="cuda", dtype=torch.bfloat16))


@pytest.mark.parametrize("case_seed", range(12))
def test_random_shapes_against_float64(gpu_ready, case_seed):
    # Seeded sweep over the envelope: M from 1 to 1500 (ragged token tiles),
    # N a multiple of 32 up to 1184 (partial feature tiles), K a multiple of
    # 128 from 256 to 1536, with and without bias, both activations and both
    # dtypes, inputs scaled by a random factor.
    from transformer_opt.kernels.linear import linear, linear_gelu

    rng = np.random.default_rng(1000 + case_seed)
    rows = int(rng.integers(1, 1501))
    out_features = 32 * int(rng.integers(1, 38))
    in_features = 128 * int(rng.integers(2, 13))
    dtype = (torch.bfloat16, torch.float16)[case_seed % 2]
    gelu = bool(rng.integers(0, 2))
    bias = bool(rng.integers(0, 2))
    scale = float(rng.choice([0.25, 1.0, 3.0]))
    g = torch.Generator().manual_seed(case_seed)
    x = (torch.randn(rows, in_features, generator=g) * scale).to(dtype)
    w = (torch.randn(out_features, in_features, generator=g) * in_features ** -0.5).to(dtype)
    b = (torch.randn(out_features, generator=g) * 0.5).to(dtype) if bias else None
    with torch.inference_mode():
        fn = linear_gelu if gelu else linear
        y = fn(x.cuda(), w.cuda(), None if b is None else b.cuda())
    assert y.shape == (rows, out_features)
    _check(y, _reference(x, w, b, gelu), dtype)
