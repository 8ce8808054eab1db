"""Encoder model on the gfx950 HIP kernels (the reference's submission surface).

``UserOptimizedTransformer`` keeps the reference's public surface
(transformer_opt/submission.py:78-723): constructor flags
``attention_backend`` / ``execution_mode``, the counters
``attention_backend_counts`` / ``fused_residual_layer_norm_calls`` /
``cuda_graph_replays``, ``reset_attention_backend_counts()``,
``clear_cuda_graph()``, ``_can_replay_cuda_graph()``, a state-dict key set
identical to the organizer baseline, a non-persistent packed-QKV projection
cache invalidated by parameter versions, and bounded graph replay.

What is MI355X-specific:

* every attention runs on the HIP kernel (fp32, bf16, fp16) - the
  reference's per-shape routing policy between Triton, SDPA and explicit math
  (submission.py:235-321) is gone, and so is the SDPA counter;
* every LayerNorm runs on the HIP fused residual + LayerNorm kernel, in the
  reference's fused order (submission.py:481-525) for all shapes: one
  standalone norm, then two fused residual+norm calls per layer;
* the packed QKV projection is used for every width and dtype
  (submission.py:184-190 restricted it to measured widths);
* graph replay (torch.cuda.CUDAGraph, i.e. a hipGraph on ROCm) is eligible for
  every supported shape and dtype instead of an exact measured shape set
  (submission.py:582-590), and up to ``max_cuda_graphs`` captures (one per
  input geometry: shape, dtype, mask presence, inference mode) are kept, so a
  caller alternating between shapes replays instead of recapturing.

Projections and the FFN stay library GEMMs (hipBLASLt through F.linear); the
FFN's exact GELU runs in place on the HIP elementwise kernel (the fused
Linear + GELU kernel, kernels.linear_gelu, measured no faster in the model).
The model is forward-inference only: a call with gradients enabled on
parameters that require them raises, as there is no backward kernel.
"""

from __future__ import annotations

import threading
from collections import OrderedDict
from typing import Dict, Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from .config import ATTENTION_BACKENDS, SUPPORTED_DTYPES
from .dispatch import attention_forward
from .kernels.gelu import gelu_
from .kernels.residual_layer_norm import fused_residual_layer_norm, layer_norm
from .model import SelfAttention, TransformerBlock, TransformerConfig

__all__ = ["TransformerConfig", "UserOptimizedTransformer", "generate_random_case", "run_accuracy_tests"]

_EXECUTION_MODES = ("auto", "eager")


class UserOptimizedTransformer(nn.Module):
    """Pre-LN encoder whose attention and LayerNorms run on gfx950 HIP kernels."""

    def __init__(self, config, attention_backend: str = "auto", execution_mode: str = "auto",
                 max_cuda_graphs: int = 4) -> None:
        super().__init__()
        if not isinstance(max_cuda_graphs, int) or max_cuda_graphs < 1:
            raise ValueError("max_cuda_graphs must be a positive integer")
        if attention_backend not in ATTENTION_BACKENDS:
            raise ValueError(
                f"attention_backend must be one of {ATTENTION_BACKENDS}, got {attention_backend!r}"
            )
        if execution_mode not in _EXECUTION_MODES:
            raise ValueError("execution_mode must be 'auto' or 'eager'")
        self.config = config
        self.layers = nn.ModuleList(
            [TransformerBlock(config.d_model, config.num_heads, config.ffn_dim)
             for _ in range(config.num_layers)]
        )
        self.final_norm = nn.LayerNorm(config.d_model)
        self.attention_backend = attention_backend
        self.execution_mode = execution_mode
        # Captured forwards keyed by input geometry, least recently used first;
        # all of them belong to one model state (``_graph_model_key``).
        self.max_cuda_graphs = max_cuda_graphs
        self._inference_graphs: "OrderedDict[tuple, _InferenceGraph]" = OrderedDict()
        self._graph_model_key = None
        self._inference_graph = None  # the entry used last
        self._inference_graph_lock = threading.RLock()
        self.cuda_graph_replays = 0
        self.attention_backend_counts: Dict[str, int] = {"hip": 0}
        self.fused_residual_layer_norm_calls = 0
        # Derived, non-persistent packed projection weights keyed by module id;
        # kept out of the state dict so its keys equal the baseline's.
        self._packed_qkv_cache: Dict[int, Tuple[tuple, torch.Tensor, torch.Tensor]] = {}

    # -- counters / pickling -------------------------------------------------
    def reset_attention_backend_counts(self) -> None:
        self.attention_backend_counts = {"hip": 0}
        self.fused_residual_layer_norm_calls = 0
        self.cuda_graph_replays = 0

    def __getstate__(self):
        state = super().__getstate__().copy()
        state["_inference_graph"] = None
        state["_inference_graphs"] = OrderedDict()
        state["_graph_model_key"] = None
        state.pop("_inference_graph_lock", None)
        return state

    def __setstate__(self, state):
        super().__setstate__(state)
        self._inference_graph_lock = threading.RLock()

    # -- projections -----------------------------------------------------------
    @staticmethod
    def _qkv_signature(attn: SelfAttention) -> tuple:
        tensors = (attn.q_proj.weight, attn.k_proj.weight, attn.v_proj.weight,
                   attn.q_proj.bias, attn.k_proj.bias, attn.v_proj.bias)
        return tuple((t.data_ptr(), t._version, t.device, t.dtype) for t in tensors if t is not None)

    def _project_qkv(self, attn: SelfAttention, x: torch.Tensor):
        """One packed GEMM -> strided [B, S, H, D] views of Q, K and V.

        Same cache contract as the reference (submission.py:145-217): the
        concatenated weight is rebuilt whenever any projection parameter's
        pointer, version counter, device or dtype changes.
        """
        batch, seq_len, _ = x.shape
        signature = self._qkv_signature(attn)
        cached = self._packed_qkv_cache.get(id(attn))
        if cached is None or cached[0] != signature:
            packed_weight = torch.cat(
                (attn.q_proj.weight, attn.k_proj.weight, attn.v_proj.weight), dim=0).detach()
            packed_bias = torch.cat(
                (attn.q_proj.bias, attn.k_proj.bias, attn.v_proj.bias), dim=0).detach()
            cached = (signature, packed_weight, packed_bias)
            self._packed_qkv_cache[id(attn)] = cached
        projected = F.linear(x, cached[1], cached[2])
        qkv = projected.view(batch, seq_len, 3, attn.num_heads, attn.head_dim)
        return qkv.unbind(dim=2)

    def _attention(self, attn: SelfAttention, x: torch.Tensor,
                   valid_token_mask: Optional[torch.Tensor], causal: bool) -> torch.Tensor:
        batch, seq_len, _ = x.shape
        q, k, v = self._project_qkv(attn, x)
        context, dispatch = attention_forward(
            q, k, v, valid_token_mask, causal=causal, scale=attn.scale,
            backend=self.attention_backend,
        )
        self.attention_backend_counts[dispatch.selected] += 1
        return attn.out_proj(context.reshape(batch, seq_len, attn.d_model))

    def _fused_residual_norm(self, x, update, norm: nn.LayerNorm, valid_token_mask, *,
                             zero_invalid_residual=False, zero_invalid_normalized=False):
        residual, normalized = fused_residual_layer_norm(
            x, update, norm.weight, norm.bias, norm.eps, valid_token_mask,
            zero_invalid_residual=zero_invalid_residual,
            zero_invalid_normalized=zero_invalid_normalized,
        )
        self.fused_residual_layer_norm_calls += 1
        return residual, normalized

    # -- forward -----------------------------------------------------------------
    def _forward_eager(self, x: torch.Tensor,
                       valid_token_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Fused order of the reference (submission.py:481-525).

        LN(x) once; then per layer: attention, (x, ffn_in) = x + attn,
        LN2(x + attn); FFN; (x, next_in) = x + ffn, next LN, with invalid rows
        of x zeroed (the baseline's per-block masked_fill) and invalid rows of
        the final output zeroed.  Invalid rows never reach a valid row: their
        keys are masked in every attention and all other ops are row-wise.
        """
        if valid_token_mask is not None and not valid_token_mask.is_contiguous():
            valid_token_mask = valid_token_mask.contiguous()
        x = x.contiguous()
        causal = self.config.causal
        first = self.layers[0].norm1
        normalized = layer_norm(x, first.weight, first.bias, first.eps)
        last_index = len(self.layers) - 1
        for index, layer in enumerate(self.layers):
            attn_out = self._attention(layer.attention, normalized, valid_token_mask, causal)
            del normalized
            x, ffn_input = self._fused_residual_norm(x, attn_out, layer.norm2, valid_token_mask)
            del attn_out
            ffn_out = layer.ffn_out(gelu_(layer.ffn_in(ffn_input)))
            del ffn_input
            is_last = index == last_index
            next_norm = self.final_norm if is_last else self.layers[index + 1].norm1
            x, normalized = self._fused_residual_norm(
                x, ffn_out, next_norm, valid_token_mask,
                zero_invalid_residual=valid_token_mask is not None,
                zero_invalid_normalized=is_last and valid_token_mask is not None,
            )
            del ffn_out
        return normalized

    def forward(self, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        if self._graph_input_supported(x, valid_token_mask):
            with self._inference_graph_lock:
                signature = self._graph_signature(x, valid_token_mask)
                if signature is not None:
                    model_key, geometry = signature
                    if model_key != self._graph_model_key:
                        # Parameters, modules or attention settings changed:
                        # every capture is stale (and would pin old storage).
                        self._drop_graphs()
                        self._graph_model_key = model_key
                    entry = self._inference_graphs.get(geometry)
                    if entry is None:
                        entry = _InferenceGraph(self, x, valid_token_mask, signature)
                        self._inference_graphs[geometry] = entry
                        while len(self._inference_graphs) > self.max_cuda_graphs:
                            self._inference_graphs.popitem(last=False)
                    else:
                        self._inference_graphs.move_to_end(geometry)
                    self._inference_graph = entry
                    output = entry.replay(x, valid_token_mask)
                    for backend, count in entry.backend_counts.items():
                        self.attention_backend_counts[backend] += count
                    self.fused_residual_layer_norm_calls += entry.fused_calls
                    self.cuda_graph_replays += 1
                    return output
        return self._forward_eager(x, valid_token_mask)

    # -- graph replay ------------------------------------------------------------
    def _can_replay_cuda_graph(self, x, valid_token_mask) -> bool:
        return (self._graph_input_supported(x, valid_token_mask)
                and self._graph_signature(x, valid_token_mask) is not None)

    def _graph_input_supported(self, x, valid_token_mask) -> bool:
        """Capture eligibility (reference submission.py:561-601, minus the
        measured-shape whitelist): eval-mode inference on one ROCm device with a
        supported dtype, no autograd, no autocast, no hooks, not already
        capturing."""
        if (
            self.execution_mode != "auto"
            or self.attention_backend != "auto"
            or not x.is_cuda
            or x.dtype not in SUPPORTED_DTYPES
            or x.ndim != 3
            or not x.is_contiguous()
            or torch.is_grad_enabled()
            or self.training
            or torch.compiler.is_compiling()
            or torch.cuda.current_device() != x.device.index
            or torch.cuda.is_current_stream_capturing()
            or torch.is_autocast_enabled("cuda")
        ):
            return False
        if x.shape[2] != self.config.d_model or x.numel() == 0:
            return False
        if x.dtype != self.final_norm.weight.dtype or x.device != self.final_norm.weight.device:
            return False
        if valid_token_mask is not None and not (
            valid_token_mask.shape == x.shape[:2]
            and valid_token_mask.device == x.device
            and valid_token_mask.dtype == torch.bool
            and valid_token_mask.is_contiguous()
        ):
            return False
        if nn.modules.module._global_forward_hooks or nn.modules.module._global_forward_pre_hooks:
            return False
        return True

    def _graph_signature(self, x, valid_token_mask):
        """Everything a captured graph bakes in (reference submission.py:603-641),
        as ``(model_key, geometry)``: the model key holds parameter
        storage/version/device/dtype, module eps and shapes, hooks, training
        flags and the attention config; the geometry holds the input's device,
        shape and dtype, mask presence and the inference-mode context.  None
        means "do not capture"."""
        stack = [self]
        seen_modules, seen_parameters = set(), set()
        modules, parameters = [], []
        while stack:
            module = stack.pop()
            identity = id(module)
            if identity in seen_modules:
                continue
            seen_modules.add(identity)
            if module.training or module._forward_hooks or module._forward_pre_hooks:
                return None
            modules.append((identity, getattr(module, "eps", None),
                            getattr(module, "normalized_shape", None)))
            for parameter in module._parameters.values():
                if parameter is None or id(parameter) in seen_parameters:
                    continue
                seen_parameters.add(id(parameter))
                if parameter.is_inference():
                    return None
                parameters.append((id(parameter), parameter.data_ptr(), parameter._version,
                                   parameter.device, parameter.dtype))
            stack.extend(child for child in reversed(tuple(module._modules.values()))
                         if child is not None)
        attention_config = tuple(
            (layer.attention.d_model, layer.attention.num_heads,
             layer.attention.head_dim, layer.attention.scale)
            for layer in self.layers
        )
        model_key = (tuple(parameters), tuple(modules), attention_config, self.config,
                     self.attention_backend, torch.backends.cuda.matmul.allow_tf32)
        geometry = (x.device, tuple(x.shape), x.dtype, valid_token_mask is not None,
                    torch.is_inference_mode_enabled())
        return model_key, geometry

    def _drop_graphs(self) -> None:
        self._inference_graphs.clear()
        self._inference_graph = None
        self._graph_model_key = None

    def clear_cuda_graph(self) -> None:
        """Release every cached capture; a later eligible call rebuilds what it needs."""
        with self._inference_graph_lock:
            self._drop_graphs()

    def _apply(self, fn, recurse=True):
        # Device/dtype moves must not keep the old graph pool or packed weights.
        self.clear_cuda_graph()
        self._packed_qkv_cache.clear()
        return super()._apply(fn, recurse=recurse)


class _InferenceGraph:
    """One captured forward with static input buffers (reference submission.py:
    674-723): warm up on a side stream, capture ``_forward_eager``, record the
    backend counts the capture performed, and on replay copy fresh inputs in,
    replay, and return a clone so earlier results are never overwritten."""

    def __init__(self, model: UserOptimizedTransformer, x, mask, signature):
        # Warm-up and capture run with inference mode off.  torch allocates the
        # generator's graph-safe RNG state tensors at the first capture and
        # updates them in place at every later one; allocated inside inference
        # mode they would become inference tensors and a later capture outside
        # it would fail.  Replay clones the output in the caller's context, so
        # returned tensors still follow the caller's mode.
        with torch.inference_mode(False), torch.no_grad():
            self._capture(model, x, mask, signature)

    def _capture(self, model: UserOptimizedTransformer, x, mask, signature):
        self.signature = signature
        self.x = x.clone()
        self.mask = mask.clone() if mask is not None else None
        # Keep captured parameter storage alive across state/device changes.
        self.parameters = tuple(parameter.detach() for parameter in model.parameters())
        before = dict(model.attention_backend_counts)
        fused_before = model.fused_residual_layer_norm_calls
        stream = torch.cuda.Stream(device=x.device)
        current = torch.cuda.current_stream(x.device)
        stream.wait_stream(current)
        try:
            with torch.cuda.stream(stream):
                for _ in range(3):
                    model._forward_eager(self.x, self.mask)
            current.wait_stream(stream)
            capture_before = dict(model.attention_backend_counts)
            capture_fused_before = model.fused_residual_layer_norm_calls
            self.graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self.graph, stream=stream):
                self.output = model._forward_eager(self.x, self.mask)
            current.wait_stream(stream)
            self.backend_counts = {
                backend: count - capture_before.get(backend, 0)
                for backend, count in model.attention_backend_counts.items()
            }
            self.fused_calls = model.fused_residual_layer_norm_calls - capture_fused_before
            self.packed = tuple(model._packed_qkv_cache.values())
            self.complete = torch.cuda.Event()
            self.complete.record(current)
        finally:
            # Warm-up and capture are set-up, not user-visible forwards.
            model.attention_backend_counts = before
            model.fused_residual_layer_norm_calls = fused_before

    def replay(self, x, mask):
        current = torch.cuda.current_stream(x.device)
        current.wait_event(self.complete)
        self.x.copy_(x)
        if self.mask is not None:
            self.mask.copy_(mask)
        self.graph.replay()
        output = self.output.clone()
        self.complete.record(current)
        return output


# ---------------------------------------------------------------------------
# Harness entry points.  The reference keeps its case generator and accuracy
# loop in this module (transformer_opt/submission.py:56-75, 726-800) and its
# tests import them from here.  They drive a caller-supplied baseline module
# against the optimized one; nothing on the compute path uses them.
# ---------------------------------------------------------------------------


def generate_random_case(
    config: TransformerConfig,
    device: torch.device,
    dtype: torch.dtype,
    seed: int,
    padding_ratio: float,
    input_scale: float,
) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """Seeded input and key-padding mask of one accuracy trial.

    Draws in the order of the organizer's generator
    (benchmarks/torch_transformer_benchmark.py:234-272): ``randn`` input times
    ``input_scale``, then per-sequence valid lengths in
    ``[round(S * (1 - padding_ratio)), S]`` from the same generator, padded
    positions zeroed - so a seed gives the reference's case.  Without padding
    the mask is ``None`` (reference submission.py:56-75).
    """
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    shape = (config.batch_size, config.seq_len, config.d_model)
    x = torch.randn(shape, generator=gen, device=device, dtype=dtype) * input_scale
    if padding_ratio <= 0:
        return x, None
    shortest = max(1, int(round(config.seq_len * (1.0 - padding_ratio))))
    lengths = torch.randint(low=shortest, high=config.seq_len + 1, size=(config.batch_size,),
                            generator=gen, device=device)
    valid = torch.arange(config.seq_len, device=device)[None, :] < lengths[:, None]
    return x.masked_fill(~valid[..., None], 0), valid


def _or_rule(reference: torch.Tensor, candidate: torch.Tensor, rtol: float, atol: float) -> dict:
    """The organizer's element rule ``finite and (|d| <= atol or |d| <= rtol*|ref|)``
    (torch_transformer_benchmark.py:289-356) with the statistics the loop prints."""
    ref = reference.detach().float()
    got = candidate.detach().float()
    diff = (got - ref).abs()
    ok = torch.isfinite(ref) & torch.isfinite(got) & ((diff <= atol) | (diff <= rtol * ref.abs()))
    bad = ~ok
    ranked = torch.nan_to_num(diff, nan=float("inf")).reshape(-1)
    worst = tuple(int(i) for i in torch.unravel_index(ranked.argmax(), ref.shape)) if ref.numel() else ()
    feature_dims = torch.nonzero(bad.reshape(-1, ref.shape[-1]).any(dim=0)).flatten().tolist() if ref.numel() else []
    return {
        "passed": not bool(bad.any()),
        "failed": int(bad.sum()),
        "total": ref.numel(),
        "max_abs": float(diff.max()) if ref.numel() else 0.0,
        "max_rel": float((diff / ref.abs().clamp_min(1e-12)).max()) if ref.numel() else 0.0,
        "worst": worst,
        "ref_at_worst": float(ref[worst]) if ref.numel() else 0.0,
        "got_at_worst": float(got[worst]) if ref.numel() else 0.0,
        "feature_dims": feature_dims,
    }


def run_accuracy_tests(
    baseline: nn.Module,
    optimized: nn.Module,
    config: TransformerConfig,
    device: torch.device,
    dtype: torch.dtype,
    trials: int,
    seed: int,
    padding_ratio: float,
    input_scale: float,
    rtol: float,
    atol: float,
) -> bool:
    """The organizer's accuracy loop (reference submission.py:726-800).

    For each trial: one seeded case (seed + trial), the baseline's output
    (cloned, as a replayed graph may reuse its buffer), the optimized
    output, and the OR rule on every element; prints one line per trial
    and a summary, and returns whether every element of every trial passed.
    """
    print("\n=== Accuracy check ===")
    print(f"criterion: abs_error <= {atol:g} OR relative_error <= {rtol:.2%}")
    all_passed = True
    max_abs = max_rel = 0.0
    failed = total = 0
    with torch.inference_mode():
        for trial in range(trials):
            x, mask = generate_random_case(config=config, device=device, dtype=dtype, seed=seed + trial,
                                           padding_ratio=padding_ratio, input_scale=input_scale)
            expected = baseline(x, mask).clone()
            result = _or_rule(expected, optimized(x, mask), rtol, atol)
            all_passed &= result["passed"]
            max_abs = max(max_abs, result["max_abs"])
            max_rel = max(max_rel, result["max_rel"])
            failed += result["failed"]
            total += result["total"]
            print(f"trial {trial + 1:02d}/{trials}: {'PASS' if result['passed'] else 'FAIL'} | "
                  f"max_abs={result['max_abs']:.6g} | max_rel={result['max_rel']:.6g} | "
                  f"failed={result['failed']}/{result['total']}")
            if not result["passed"]:
                dims = result["feature_dims"]
                more = "..." if len(dims) > 16 else ""
                print(f"  worst_index={result['worst']}, baseline={result['ref_at_worst']:.8g}, "
                      f"optimized={result['got_at_worst']:.8g}")
                print(f"  failed output feature dims={dims[:16]}{more}")
    print(f"summary: {'PASS' if all_passed else 'FAIL'} | max_abs={max_abs:.6g} | "
          f"max_rel={max_rel:.6g} | failed={failed}/{total}")
    return all_passed
