"""Host-side contract of the product surface (reference tests/test_dispatch.py,
tests/test_correctness.py and tests/test_cuda_graph_inference.py, CPU parts).

No kernel runs here: every call either validates and raises, or inspects
metadata.  Where the reference fell back to SDPA or explicit math on CPU, the
HIP build raises instead (there is no fallback in the product path).
"""

from __future__ import annotations

import copy
import sys
from pathlib import Path

import pytest
import torch

from transformer_opt import ATTENTION_BACKENDS, attention_forward, hip_attention_support
from transformer_opt.config import attention_launch_config, triton_attention_support
from transformer_opt.kernels import fused_residual_layer_norm, layer_norm
from transformer_opt.submission import TransformerConfig, UserOptimizedTransformer

REPO = Path(__file__).resolve().parent.parent


def _cpu_qkv(dtype=torch.float32):
    q = torch.randn(1, 8, 2, 16, dtype=dtype)
    return q, torch.randn_like(q), torch.randn_like(q)


def test_backends_are_the_hip_routes_and_the_explicit_reference():
    # "triton" is the reference's forced fused route (config.py:11,
    # dispatch.py:119-132); here it names the HIP kernel that replaces it.
    # "reference" is the reference's explicit-math route (dispatch.py:69-96).
    assert ATTENTION_BACKENDS == ("auto", "hip", "triton", "reference")
    assert triton_attention_support is hip_attention_support


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("causal", [False, True])
def test_reference_route_is_the_explicit_math(dtype, causal):
    # Forced only: recorded as "reference", plain torch operations (it runs
    # here on the CPU), equal to the oracle's restatement of the reference's
    # explicit attention (dispatch.py:69-96) on the same inputs, all-masked
    # rows NaN as there.
    from oracle.attention import explicit_attention as oracle_explicit

    g = torch.Generator().manual_seed(7)
    q, k, v = (torch.randn(2, 37, 3, 16, generator=g, dtype=dtype) for _ in range(3))
    mask = torch.arange(37)[None, :] < torch.tensor([[37], [20]])
    out, record = attention_forward(q, k, v, mask, causal=causal, scale=0.3, backend="reference")
    assert (record.requested, record.selected) == ("reference", "reference")
    expected = oracle_explicit(q, k, v, mask, causal, 0.3)
    assert out.shape == q.shape and out.dtype == dtype and out.is_contiguous()
    torch.testing.assert_close(out, expected, rtol=1e-6, atol=1e-6)
    empty = torch.zeros(2, 37, dtype=torch.bool)
    empty[0] = True
    out, _ = attention_forward(q, k, v, empty, causal=causal, backend="reference")
    assert bool(out[1].isnan().all()) and bool(out[0].isfinite().all())


def test_invalid_backend_is_rejected():
    q, k, v = _cpu_qkv()
    with pytest.raises(ValueError, match="attention backend"):
        attention_forward(q, k, v, backend="mystery")
    with pytest.raises(ValueError, match="attention backend"):
        attention_forward(q, k, v, backend="sdpa")


def test_cpu_tensors_fail_loudly_instead_of_falling_back():
    q, k, v = _cpu_qkv()
    for backend in ("auto", "hip"):
        with pytest.raises((RuntimeError, ValueError), match="HIP attention was"):
            attention_forward(q, k, v, backend=backend)


def test_forced_triton_route_fails_like_the_reference_on_cpu():
    # Reference tests/test_dispatch.py:27-29 matches this wording.
    q, k, v = _cpu_qkv()
    with pytest.raises((RuntimeError, ValueError), match="Triton attention was forced"):
        attention_forward(q, k, v, backend="triton")


@pytest.mark.parametrize("bad,reason", [
    (lambda q: (q, q, q, torch.ones(1, 7, dtype=torch.bool)), "shape [batch, sequence]"),
    (lambda q: (q[0], q[0], q[0], None), "shape [batch, sequence, heads, head_dim]"),
    (lambda q: (q, q[:, :4], q, None), "identical shapes"),
    (lambda q: (q, q.double(), q, None), "identical dtypes"),
    (lambda q: (q.transpose(2, 3).contiguous().transpose(2, 3), q, q, None), "head-dimension stride"),
    (lambda q: (q, q, q, torch.ones(1, 8)), "dtype torch.bool"),
    (lambda q: (q, q, q, None), "ROCm device"),
])
def test_support_check_explains_refusals(bad, reason):
    q = torch.randn(1, 8, 2, 16)
    result = hip_attention_support(*bad(q))
    assert not result.supported
    assert reason in result.reason


def test_launch_config_is_the_fixed_gfx950_tile():
    assert attention_launch_config(64, torch.float32) == attention_launch_config(64)
    fp32_64 = attention_launch_config(64, torch.float32)
    assert (fp32_64.block_m, fp32_64.block_n, fp32_64.num_waves, fp32_64.lds_stages) == (128, 64, 4, 2)
    assert attention_launch_config(128, torch.float32).block_n == 32
    assert attention_launch_config(128, torch.bfloat16).block_n == 64
    assert attention_launch_config(8, torch.float16).block_m == 128
    with pytest.raises(ValueError, match="head_dim=48"):
        attention_launch_config(48)


def test_fused_layer_norm_contract_errors():
    x = torch.randn(2, 5, 16)
    w = torch.ones(16)
    with pytest.raises(ValueError, match="ROCm device"):
        fused_residual_layer_norm(x, x, w, None, 1e-5)
    with pytest.raises(ValueError, match="same rank-two-or-higher shape"):
        fused_residual_layer_norm(x, x[:, :4], w, None, 1e-5)
    with pytest.raises(ValueError, match="same rank-two-or-higher shape"):
        fused_residual_layer_norm(x[0, 0], x[0, 0], w, None, 1e-5)
    with pytest.raises(ValueError):
        layer_norm(x, w, None, 1e-5)


def test_zeroing_without_mask_is_rejected_before_device_checks():
    # The reference raises this ValueError too (residual_layer_norm.py:200-201).
    x = torch.randn(2, 5, 16)
    if torch.cuda.is_available():
        x = x.cuda()
    w = torch.ones(16, device=x.device)
    if x.is_cuda:
        with pytest.raises(ValueError, match="requires valid_token_mask"):
            fused_residual_layer_norm(x, x, w, None, 1e-5, zero_invalid_residual=True)


def test_model_constructor_validation_and_state_surface():
    cfg = TransformerConfig(1, 128, 128, 4, 128, 4, True)
    with pytest.raises(ValueError, match="execution_mode"):
        UserOptimizedTransformer(cfg, execution_mode="invalid")
    with pytest.raises(ValueError, match="attention_backend"):
        UserOptimizedTransformer(cfg, attention_backend="sdpa")
    for backend in ("triton", "reference"):
        forced = UserOptimizedTransformer(cfg, attention_backend=backend).eval()
        assert forced._replay_refusal(torch.randn(1, 128, 128), None) == "attention backend is forced"
    model = UserOptimizedTransformer(cfg).eval()
    assert model.attention_backend_counts == {"hip": 0, "reference": 0}
    assert model.fused_residual_layer_norm_calls == 0 and model.cuda_graph_replays == 0
    cloned = copy.deepcopy(model)
    assert cloned.state_dict().keys() == model.state_dict().keys()
    assert cloned._inference_graph is None
    with torch.inference_mode():
        assert not model._can_replay_cuda_graph(torch.randn(1, 128, 128), None)
    keys = set(model.state_dict().keys())
    assert "layers.0.attention.q_proj.weight" in keys and "final_norm.bias" in keys
    assert not any("packed" in key for key in keys)


def test_model_is_freed_without_the_cyclic_collector():
    # The operand layout cached in the model's replay cache must not refer
    # back to the model: a model in a reference cycle is freed only by the
    # cyclic collector, which may run inside another model's graph capture
    # and there destroy this model's captured graphs (not allowed during a
    # capture; the error aborts the process).
    import gc
    import weakref

    cfg = TransformerConfig(1, 16, 32, 2, 64, 2, False)
    model = UserOptimizedTransformer(cfg).eval()
    ops = model._operands()
    assert ops.fingerprint is not None and model._replay.layout is not None
    ref = weakref.ref(model)
    collecting = gc.isenabled()
    gc.disable()
    try:
        del model, ops
        assert ref() is None, "the model survived its last reference (reference cycle)"
    finally:
        if collecting:
            gc.enable()


def test_model_forward_on_cpu_fails_loudly():
    cfg = TransformerConfig(1, 16, 32, 2, 64, 1, False)
    model = UserOptimizedTransformer(cfg).eval()
    with torch.inference_mode(), pytest.raises((RuntimeError, ValueError)):
        model(torch.randn(1, 16, 32))


def test_config_validation():
    TransformerConfig(1, 1, 8, 2, 8, 1, False).validate()
    with pytest.raises(ValueError, match="divisible"):
        TransformerConfig(1, 1, 10, 3, 8, 1, False).validate()
    with pytest.raises(ValueError, match="positive"):
        TransformerConfig(0, 1, 8, 2, 8, 1, False).validate()


def test_product_never_imports_the_oracle():
    pkg = REPO / "triton-transformer-kernels_amd"
    for path in pkg.rglob("*.py"):
        text = path.read_text()
        assert "import oracle" not in text and "from oracle" not in text, path
    for path in (pkg / "csrc").glob("*"):
        if path.is_file():
            assert "oracle" not in path.read_text(), path


def test_bench_rejects_multi_gpu_requests():
    import subprocess

    out = subprocess.run([sys.executable, str(REPO / "bench.py"), "--gpus", "8"],
                         capture_output=True, text=True, timeout=300)
    assert out.returncode == 2
    assert "one MI355X" in out.stderr


def test_reference_entry_point_names_are_present():
    # Callers written against the reference import these names
    # (transformer_opt/kernels/__init__.py, kernels/residual_layer_norm.py:129,
    # submission.py:56 and 726).
    from transformer_opt import kernels, submission

    assert kernels.triton_attention is kernels.hip_attention
    assert kernels.triton_available is kernels.hip_available
    assert callable(kernels.short_layer_norm)
    assert callable(submission.generate_random_case) and callable(submission.run_accuracy_tests)


def test_short_layer_norm_contract_errors():
    from transformer_opt.kernels import short_layer_norm

    with torch.no_grad():
        with pytest.raises(ValueError, match="width 32"):
            short_layer_norm(torch.empty(4, 33), torch.ones(33), None, 1e-5)
        with pytest.raises(ValueError, match="width 32"):
            short_layer_norm(torch.empty(4, 32, dtype=torch.float16), torch.ones(32), None, 1e-5)
        with pytest.raises(ValueError, match="width 32"):
            short_layer_norm(torch.empty(32), torch.ones(32), None, 1e-5)
        with pytest.raises(ValueError, match="width 32"):  # CPU tensor: no host fallback
            short_layer_norm(torch.empty(4, 32), torch.ones(32), None, 1e-5)


def test_harness_case_generator_matches_the_oracle_restatement():
    from oracle.model import generate_random_case as organizer_case
    from transformer_opt.submission import generate_random_case

    cfg = TransformerConfig(3, 40, 16, 2, 32, 1, False)
    for padding in (0.0, 0.3, 0.9):
        x, mask = generate_random_case(cfg, torch.device("cpu"), torch.float32, 11, padding, 1.5)
        ex, emask = organizer_case(cfg, torch.device("cpu"), torch.float32, 11, padding, 1.5)
        assert torch.equal(x, ex)
        assert (mask is None and emask is None) or torch.equal(mask, emask)


def test_harness_accuracy_loop_uses_the_or_rule(capsys):
    from oracle.model import BaselineTransformer, compare_outputs
    from transformer_opt.submission import _or_rule, run_accuracy_tests

    # The OR rule agrees with the oracle's comparator element for element,
    # including non-finite values.
    g = torch.Generator().manual_seed(2)
    ref = torch.randn(3, 7, 9, generator=g)
    got = ref + torch.randn(ref.shape, generator=g) * 2e-3
    got[0, 0, 0] = float("nan")
    got[1, 2, 3] = ref[1, 2, 3] * 1.009  # relative error below 1 %
    mine = _or_rule(ref, got, rtol=0.01, atol=1e-3)
    theirs = compare_outputs(ref, got, rtol=0.01, atol=1e-3)
    assert mine["failed"] == theirs.failed_elements and mine["passed"] == theirs.passed
    assert mine["feature_dims"] == theirs.failed_feature_dims

    # The loop passes a model against itself and fails a perturbed copy.
    cfg = TransformerConfig(2, 12, 16, 2, 32, 1, True)
    torch.manual_seed(0)
    model = BaselineTransformer(cfg).eval()

    class Shifted(torch.nn.Module):
        def __init__(self, inner, shift):
            super().__init__()
            self.inner, self.shift = inner, shift

        def forward(self, x, mask):
            return self.inner(x, mask) + self.shift

    args = dict(config=cfg, device=torch.device("cpu"), dtype=torch.float32, trials=2, seed=5,
                padding_ratio=0.3, input_scale=1.0, rtol=0.01, atol=1e-3)
    assert run_accuracy_tests(model, model, **args)
    assert not run_accuracy_tests(model, Shifted(model, 0.5), **args)
    out = capsys.readouterr().out
    assert "trial 01/2: PASS" in out and "summary: FAIL" in out and "worst_index=" in out


def test_fused_out_projection_norm_route_contract():
    # The opt-in projection + residual + LayerNorm route: off by default,
    # never packs a weight the kernel cannot take (a CPU weight here), packs
    # nothing while the route is off, and its support check explains refusals
    # before any device work.
    from transformer_opt.kernels.linear_ln import linear_ln_supported, pack_weight
    from transformer_opt.replay import PackedOut

    cfg = TransformerConfig(1, 16, 1024, 8, 64, 1, False)
    model = UserOptimizedTransformer(cfg).to(torch.bfloat16).eval()
    assert model.fuse_out_projection_norm is False
    ops = model._operands()
    assert all(block.out_packed is None for block in ops.blocks) and not model._replay.out_packs
    model.fuse_out_projection_norm = True
    ops = model._operands()
    assert all(block.out_packed is None for block in ops.blocks)  # CPU weights: nothing to pack
    assert PackedOut(torch.zeros(1024, 1024, dtype=torch.bfloat16)).packed is None
    a = torch.zeros(16, 1024, dtype=torch.bfloat16)
    x = torch.zeros(16, 1024, dtype=torch.bfloat16)
    g = torch.ones(1024, dtype=torch.bfloat16)
    assert "ROCm" in linear_ln_supported(a, torch.zeros(1024 * 1024, dtype=torch.bfloat16), None, x, g, None)
    with pytest.raises(ValueError, match="ROCm"):
        pack_weight(torch.zeros(1024, 1024, dtype=torch.bfloat16))
