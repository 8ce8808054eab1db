"""Output projection + residual + LayerNorm in one kernel
(``ttk_linear_residual_ln_fwd``) against the unfused route.

The reference computes ``x, h = fused_residual_layer_norm(x, out_proj(ctx),
norm2)`` (transformer_opt/submission.py:497-505): the projection rounded to
the dtype, the residual sum rounded again, the LayerNorm of that rounded sum.
Checks:

* the packed weight is the documented fragment order, element for element;
* r is bit for bit ``round(x + P)`` where P is this library's own linear
  kernel on the same operands (``ttk_linear_fwd``: the same MFMA sequence
  over k, so the same fp32 sums) - and P itself is held to the float64
  bound of ``test_gpu_linear.py``;
* y against the float64 LayerNorm of that r: |d| <= one output rounding
  step (2^-8 |y| bf16, 2^-11 |y| fp16) + the fp32 statistics error,
  and bit for bit the residual+LN kernel's y on at least 99 % of elements
  (the two sum the row statistics in different orders);
* determinism, the workspace left zero, ragged rows, padded and strided
  inputs, no bias / no LN bias, and hipGraph replay.
"""

from __future__ import annotations

import math

import numpy as np

import pytest
import torch

from transformer_opt import _native

pytestmark = pytest.mark.gpu


def _inputs(rows, in_features, dtype, seed, bias=True, ln_bias=True):
    g = torch.Generator().manual_seed(seed)
    a = torch.randn(rows, in_features, generator=g).to(dtype)
    w = (torch.randn(1024, in_features, generator=g) * in_features ** -0.5).to(dtype)
    b = (torch.randn(1024, generator=g) * 0.1).to(dtype) if bias else None
    x = torch.randn(rows, 1024, generator=g).to(dtype)
    gamma = (torch.rand(1024, generator=g) + 0.5).to(dtype)
    beta = (torch.randn(1024, generator=g) * 0.1).to(dtype) if ln_bias else None
    dev = torch.device("cuda")
    move = lambda t: None if t is None else t.to(dev)  # noqa: E731
    return tuple(move(t) for t in (a, w, b, x, gamma, beta))


def _layer_norm64(r, gamma, beta, eps):
    r64 = r.double().cpu()
    mean = r64.mean(dim=-1, keepdim=True)
    var = ((r64 - mean) ** 2).mean(dim=-1, keepdim=True)
    y = (r64 - mean) / torch.sqrt(var + eps) * gamma.double().cpu()
    return y if beta is None else y + beta.double().cpu()


def _check_against_unfused(a, w, b, x, gamma, beta, eps, r, y):
    from transformer_opt.kernels import fused_residual_layer_norm
    from transformer_opt.kernels.linear import linear

    with torch.inference_mode():
        proj = linear(a, w, b)
        expect_r = (x.float() + proj.float()).to(x.dtype)
        ln_r, ln_y = fused_residual_layer_norm(x, proj, gamma, beta, eps)
    assert torch.equal(r, expect_r), "r differs from round(x + own linear kernel)"
    assert torch.equal(ln_r, r)
    # y against float64 LayerNorm of the same r.
    q = 2.0 ** -8 if x.dtype == torch.bfloat16 else 2.0 ** -11
    y64 = _layer_norm64(r, gamma, beta, eps)
    err = (y.double().cpu() - y64).abs()
    bound = q * y64.abs() + 1e-5 * (1 + gamma.double().abs().max().item())
    assert bool((err <= bound).all()), f"y: max err {err.max().item():.3g}, failed {int((err > bound).sum())}"
    same = float((y == ln_y).float().mean())
    assert same >= 0.99, f"only {same:.4f} of y equals the residual+LN kernel's"
    return proj


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,in_features,bias,ln_bias", [
    (64, 256, True, True),       # one row block, two stage pairs
    (300, 1024, True, True),     # ragged last block
    (129, 256, False, True),     # no projection bias
    (200, 384, True, False),     # no LayerNorm bias
    (2048, 4096, True, True),    # FFN-output-like depth
])
def test_matches_unfused_route(gpu_ready, dtype, rows, in_features, bias, ln_bias):
    from transformer_opt.kernels.linear_ln import linear_residual_layer_norm, pack_weight

    a, w, b, x, gamma, beta = _inputs(rows, in_features, dtype, rows + in_features, bias, ln_bias)
    with torch.inference_mode():
        wp = pack_weight(w)
        r, y = linear_residual_layer_norm(a, wp, b, x, gamma, beta, 1e-5)
    _check_against_unfused(a, w, b, x, gamma, beta, 1e-5, r, y)


def test_config4_block_every_element_and_determinism(gpu_ready):
    # Config 4's shapes: 8192 tokens, d_model 1024, bf16, Xavier-uniform
    # weights; every element checked, two launches bitwise equal, the
    # workspace zero afterwards.
    from transformer_opt.kernels import linear_ln
    from transformer_opt.kernels.linear_ln import linear_residual_layer_norm, pack_weight

    dtype = torch.bfloat16
    g = torch.Generator().manual_seed(41)
    bound = math.sqrt(6 / 2048)
    a = torch.randn(8192, 1024, generator=g).to(dtype).cuda()
    w = ((torch.rand(1024, 1024, generator=g) * 2 - 1) * bound).to(dtype).cuda()
    b = (torch.randn(1024, generator=g) * 0.02).to(dtype).cuda()
    x = torch.randn(8192, 1024, generator=g).to(dtype).cuda()
    gamma = torch.ones(1024, dtype=dtype, device="cuda")
    beta = torch.zeros(1024, dtype=dtype, device="cuda")
    with torch.inference_mode():
        wp = pack_weight(w)
        r, y = linear_residual_layer_norm(a, wp, b, x, gamma, beta, 1e-5)
        r2, y2 = linear_residual_layer_norm(a, wp, b, x, gamma, beta, 1e-5)
    torch.cuda.synchronize()
    assert torch.equal(r, r2) and torch.equal(y, y2)
    counter_bytes = _native.LINEAR_LN_WS_COUNTER_BYTES
    for ws in linear_ln._WORKSPACES.values():
        assert int(ws[:counter_bytes].count_nonzero()) == 0
    proj = _check_against_unfused(a, w, b, x, gamma, beta, 1e-5, r, y)
    # The projection itself against float64 (rows sampled: 8192 x 1024 x 1024).
    rows = slice(0, 8192, 37)
    p64 = a[rows].double().cpu() @ w.double().cpu().T + b.double().cpu()
    err = (proj[rows].double().cpu() - p64).abs()
    acc = (a[rows].double().abs().cpu() @ w.double().abs().cpu().T) * (4 * math.sqrt(1024) * 2.0 ** -24)
    assert bool((err <= 2.0 ** -8 * p64.abs() + acc + 1e-6).all())


@pytest.mark.parametrize("rows,in_features,dtype", [
    (64, 256, torch.bfloat16), (300, 1024, torch.bfloat16), (8192, 1024, torch.bfloat16),
    (200, 384, torch.float16),
])
def test_hand_over_route_gives_the_same_bits(gpu_ready, rows, in_features, dtype):
    # max_polls = 0: the first workgroup of every row block hands its half to
    # the second without waiting, which then normalises the whole block from
    # the r it reads back.  Same bits as the default route; counters zero after.
    from transformer_opt.kernels import linear_ln
    from transformer_opt.kernels.linear_ln import linear_residual_layer_norm, pack_weight

    a, w, b, x, gamma, beta = _inputs(rows, in_features, dtype, 3 * rows + in_features)
    with torch.inference_mode():
        wp = pack_weight(w)
        r0, y0 = linear_residual_layer_norm(a, wp, b, x, gamma, beta, 1e-5)
        r1, y1 = linear_residual_layer_norm(a, wp, b, x, gamma, beta, 1e-5, max_polls=0)
        r2, y2 = linear_residual_layer_norm(a, wp, b, x, gamma, beta, 1e-5, max_polls=1)
    torch.cuda.synchronize()
    assert torch.equal(r0, r1) and torch.equal(r0, r2)
    if not (torch.equal(y0, y1) and torch.equal(y0, y2)):
        from transformer_opt.kernels import fused_residual_layer_norm
        _, ln_y = fused_residual_layer_norm(x, (r0.float() - x.float()).to(x.dtype), gamma, beta, 1e-5)
        report = []
        for name, yy in (("default", y0), ("polls=0", y1), ("polls=1", y2)):
            far = (yy.float() - ln_y.float()).abs() > 0.02 * (1 + ln_y.float().abs())
            rows_far = far.any(dim=1).nonzero().flatten()
            blocks = sorted(set((rows_far // 64).tolist()))
            halves = [int(far[:, :512].sum()), int(far[:, 512:].sum())]
            report.append(f"{name}: far={int(far.sum())} blocks={blocks[:12]} halves={halves}")
        raise AssertionError("routes differ; " + "; ".join(report))
    counter_bytes = _native.LINEAR_LN_WS_COUNTER_BYTES
    for ws in linear_ln._WORKSPACES.values():
        assert int(ws[:counter_bytes].count_nonzero()) == 0
    _check_against_unfused(a, w, b, x, gamma, beta, 1e-5, r1, y1)


def test_shapes_in_any_order_share_one_workspace(gpu_ready):
    # One workspace per stream serves launches of every size: a small launch
    # (whose statistics follow the counter block) before and after large
    # ones leaves the large launches' counters intact.
    from transformer_opt.kernels.linear_ln import linear_residual_layer_norm, pack_weight

    cases = [_inputs(rows, 256, torch.bfloat16, rows) for rows in (300, 8192, 64, 8192, 4100)]
    with torch.inference_mode():
        for a, w, b, x, gamma, beta in cases:
            wp = pack_weight(w)
            r, y = linear_residual_layer_norm(a, wp, b, x, gamma, beta, 1e-5)
            r1, y1 = linear_residual_layer_norm(a, wp, b, x, gamma, beta, 1e-5, max_polls=0)
            torch.cuda.synchronize()
            assert torch.equal(r, r1) and torch.equal(y, y1), a.shape
            _check_against_unfused(a, w, b, x, gamma, beta, 1e-5, r, y)


def test_packed_weight_layout(gpu_ready):
    from transformer_opt.kernels.linear_ln import pack_weight

    g = torch.Generator().manual_seed(5)
    w = torch.randn(1024, 256, generator=g).to(torch.bfloat16).cuda()
    packed = pack_weight(w).cpu()
    # chunk (fb * K/16 + q) * 64 + l holds W[32 fb + l % 32][16 q + 8 (l // 32) .. + 7]
    expected = w.cpu().view(32, 32, 16, 2, 8).permute(0, 2, 3, 1, 4).reshape(-1)
    assert torch.equal(packed, expected)


def test_strided_and_offset_operands(gpu_ready):
    # Views with padded rows and an offset start are copied to aligned
    # contiguous operands by the wrapper; the result matches contiguous inputs.
    from transformer_opt.kernels.linear_ln import linear_residual_layer_norm, pack_weight

    a, w, b, x, gamma, beta = _inputs(160, 256, torch.bfloat16, 7)
    big_a = torch.zeros(161, 264, dtype=a.dtype, device=a.device)
    big_a[1:, 4:260] = a
    big_x = torch.zeros(161, 1032, dtype=x.dtype, device=x.device)
    big_x[1:, 8:] = x
    with torch.inference_mode():
        wp = pack_weight(w)
        r, y = linear_residual_layer_norm(big_a[1:, 4:260], wp, b, big_x[1:, 8:], gamma, beta, 1e-5)
        r0, y0 = linear_residual_layer_norm(a, wp, b, x, gamma, beta, 1e-5)
    assert torch.equal(r, r0) and torch.equal(y, y0)


def test_graph_replay_matches_eager(gpu_ready):
    from transformer_opt.kernels.linear_ln import linear_residual_layer_norm, pack_weight

    a, w, b, x, gamma, beta = _inputs(512, 1024, torch.bfloat16, 11)
    with torch.inference_mode():
        wp = pack_weight(w)
        r_eager, y_eager = linear_residual_layer_norm(a, wp, b, x, gamma, beta, 1e-5)
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            linear_residual_layer_norm(a, wp, b, x, gamma, beta, 1e-5)  # warm-up on the stream
        torch.cuda.current_stream().wait_stream(stream)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            r_g, y_g = linear_residual_layer_norm(a, wp, b, x, gamma, beta, 1e-5)
        for _ in range(3):
            graph.replay()
            # Eager work on the same inputs between replays.
            linear_residual_layer_norm(a, wp, b, x, gamma, beta, 1e-5)
            torch.cuda.synchronize()
            assert torch.equal(r_g, r_eager) and torch.equal(y_g, y_eager)


def test_rejects_what_it_cannot_run(gpu_ready):
    from transformer_opt.kernels.linear_ln import linear_ln_supported, linear_residual_layer_norm, pack_weight

    a, w, b, x, gamma, beta = _inputs(64, 256, torch.bfloat16, 3)
    wp = pack_weight(w)
    assert linear_ln_supported(a, wp, b, x, gamma, beta) is None
    with pytest.raises(ValueError, match="width"):
        linear_residual_layer_norm(a, wp, b, x[:, :512], gamma[:512], beta[:512], 1e-5)
    with pytest.raises(ValueError, match="multiple of 128"):
        linear_residual_layer_norm(a[:, :192], wp, b, x, gamma, beta, 1e-5)
    with pytest.raises(ValueError, match="dtype"):
        linear_residual_layer_norm(a.float(), wp, b, x, gamma, beta, 1e-5)


@pytest.mark.parametrize("case_seed", range(8))
def test_random_shapes_against_unfused_route(gpu_ready, case_seed):
    # Seeded sweep: M from 1 to 2500 (ragged row blocks), K a multiple of 128
    # up to 2048, bias and LayerNorm bias present or not, both dtypes, both
    # the default and the hand-over route (the same bits).
    from transformer_opt.kernels.linear_ln import linear_residual_layer_norm, pack_weight

    rng = np.random.default_rng(2000 + case_seed)
    rows = int(rng.integers(1, 2501))
    in_features = 128 * int(rng.integers(1, 17))
    dtype = (torch.bfloat16, torch.float16)[case_seed % 2]
    bias, ln_bias = bool(rng.integers(0, 2)), bool(rng.integers(0, 2))
    a, w, b, x, gamma, beta = _inputs(rows, in_features, dtype, 7 * case_seed + 1, bias, ln_bias)
    with torch.inference_mode():
        wp = pack_weight(w)
        r, y = linear_residual_layer_norm(a, wp, b, x, gamma, beta, 1e-5)
        r1, y1 = linear_residual_layer_norm(a, wp, b, x, gamma, beta, 1e-5, max_polls=0)
    assert torch.equal(r, r1) and torch.equal(y, y1)
    if in_features >= 256:  # the comparison route's linear kernel takes K >= 256
        _check_against_unfused(a, w, b, x, gamma, beta, 1e-5, r, y)
    else:
        q = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11
        y64 = _layer_norm64(r, gamma, beta, 1e-5)
        err = (y.double().cpu() - y64).abs()
        assert bool((err <= q * y64.abs() + 1e-5 * (1 + gamma.double().abs().max().item())).all())
