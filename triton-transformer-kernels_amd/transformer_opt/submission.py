"""Encoder model on the gfx950 HIP kernels (the reference's submission surface).

``UserOptimizedTransformer`` keeps the reference's public surface
(transformer_opt/submission.py:78-723): constructor flags
``attention_backend`` / ``execution_mode``, the counters
``attention_backend_counts`` / ``fused_residual_layer_norm_calls`` /
``cuda_graph_replays``, ``reset_attention_backend_counts()``,
``clear_cuda_graph()``, ``_can_replay_cuda_graph()``, a state-dict key set
identical to the organizer baseline, a non-persistent packed-QKV projection
and hipGraph replay.

How a forward runs here:

1. ``_operands()`` reads, once, every tensor and scalar the forward uses -
   LayerNorm weights and eps, the packed QKV projection, attention heads and
   scale, the output and FFN projections - into a flat ``_Operands`` record,
   and fingerprints that read set (tensor identity, storage and version;
   the scalars; module training flags and hooks).  The fingerprint is the
   capture key: a capture is stale exactly when something it read changed.
2. ``_encode(ops, x, mask, tally)`` is the forward over those operands: one
   standalone LayerNorm, then per block attention, a fused residual +
   LayerNorm, the FFN, and a fused residual + LayerNorm that also produces
   the next block's (or the final) normalised input - the fused order of the
   reference (submission.py:481-525).  Every kernel launch is reported to
   ``tally``.
3. ``forward`` either runs ``_encode`` eagerly or replays a hipGraph of it
   from ``replay.ReplayCache``; ``_replay_refusal`` names the rule that keeps
   a call eager.

What is MI355X-specific: every attention runs on the HIP kernel (fp32,
bf16, fp16) and every LayerNorm on the HIP residual + LayerNorm kernel - the
reference's per-shape routing between Triton, SDPA and explicit math
(submission.py:235-321) is gone, and so is the SDPA counter.  The counters
are ``{"hip": n, "reference": n}``: a model built with
``attention_backend="reference"`` runs the explicit-math attention route of
the dispatcher (never chosen otherwise) and counts it there; the packed QKV
projection is used for every width and dtype (submission.py:184-190
restricted it); graph replay is eligible for every supported shape and dtype
instead of a measured shape set (submission.py:582-590), with up to
``max_cuda_graphs`` captures kept, one per input geometry.  Projections are
library GEMMs (hipBLASLt through ``F.linear``); in bf16 the FFN's input
projection and exact GELU are one HIP kernel (GELU in the GEMM epilogue),
otherwise the GELU runs in place on the HIP elementwise kernel.  The model is
forward-inference only: with gradients enabled on parameters that require
them the kernels raise, as there is no backward kernel.
"""

from __future__ import annotations

from typing import Dict, NamedTuple, Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from .config import ATTENTION_BACKENDS, SUPPORTED_DTYPES
from .dispatch import attention_forward
from .kernels.gelu import gelu_
from .kernels.linear import linear_gelu, linear_supported
from .kernels.linear_ln import linear_ln_supported, linear_residual_layer_norm
from .kernels.linear_ln import workspace_bytes as linear_ln_workspace_bytes
from .kernels.residual_layer_norm import fused_residual_layer_norm, layer_norm
from .model import TransformerBlock, TransformerConfig
from .replay import CapturedForward, ReplayCache

__all__ = ["TransformerConfig", "UserOptimizedTransformer", "generate_random_case", "run_accuracy_tests"]

_EXECUTION_MODES = ("auto", "eager")


class _Norm(NamedTuple):
    weight: torch.Tensor
    bias: Optional[torch.Tensor]
    eps: float


class _Block(NamedTuple):
    """Operands of one encoder block, read from its modules."""

    qkv_weight: torch.Tensor  # [3 * d_model, d_model]
    qkv_bias: torch.Tensor
    num_heads: int
    head_dim: int
    scale: float
    out_weight: torch.Tensor
    out_bias: Optional[torch.Tensor]
    norm2: _Norm
    ffn_in_weight: torch.Tensor
    ffn_in_bias: Optional[torch.Tensor]
    ffn_out_weight: torch.Tensor
    ffn_out_bias: Optional[torch.Tensor]
    exit_norm: _Norm  # the next block's norm1, or the final norm
    # out_weight packed for the fused projection + residual + LayerNorm
    # kernel, or None when that kernel cannot take it.
    out_packed: Optional[torch.Tensor]


class _Operands(NamedTuple):
    entry_norm: _Norm  # the first block's norm1
    blocks: Tuple[_Block, ...]
    # Hashable summary of everything above (None: the read set cannot be
    # fingerprinted - inference-tensor parameters, training mode or hooks).
    fingerprint: Optional[tuple]
    keepalive: tuple  # tensors a capture reads by address


class _Layout:
    """Where the forward's operands sit in the module tree, read once.

    ``slots`` holds one ``(dict, key, object)`` triple per edge the forward
    walks - child modules and parameters - so ``intact()`` is a single
    identity pass.  ``tensors`` are the parameters whose stamps key a
    capture; ``modules`` the submodules whose training flag and hooks do (the
    root's are read from the model itself: the layout lives in the model's
    replay cache, and a reference back to the model would make a cycle that
    only the cyclic garbage collector frees - possibly in the middle of
    another model's graph capture, where destroying this model's captured
    graphs is not allowed).
    """

    __slots__ = ("epoch", "slots", "modules", "tensors", "norms", "attentions", "layers",
                 "final_norm")

    def __init__(self, model: "UserOptimizedTransformer", epoch: int) -> None:
        self.epoch = epoch
        slots, modules, tensors = [], [], []

        def child(parent: nn.Module, name: str) -> nn.Module:
            module = parent._modules[name]
            slots.append((parent._modules, name, module))
            modules.append(module)
            return module

        def param(owner: nn.Module, name: str) -> Optional[torch.Tensor]:
            tensor = owner._parameters.get(name)
            slots.append((owner._parameters, name, tensor))
            if tensor is not None:
                tensors.append(tensor)
            return tensor

        stack = child(model, "layers")
        self.layers = []
        self.norms = []
        self.attentions = []
        for name in list(stack._modules):
            layer = child(stack, name)
            norm1, attn = child(layer, "norm1"), child(layer, "attention")
            projections = [child(attn, p) for p in ("q_proj", "k_proj", "v_proj", "out_proj")]
            norm2, ffn_in, ffn_out = (child(layer, n) for n in ("norm2", "ffn_in", "ffn_out"))
            entry = {
                "norm1": (param(norm1, "weight"), param(norm1, "bias")),
                "qkv": tuple(param(p, "weight") for p in projections[:3])
                + tuple(param(p, "bias") for p in projections[:3]),
                "out": (param(projections[3], "weight"), param(projections[3], "bias")),
                "norm2": (param(norm2, "weight"), param(norm2, "bias")),
                "ffn_in": (param(ffn_in, "weight"), param(ffn_in, "bias")),
                "ffn_out": (param(ffn_out, "weight"), param(ffn_out, "bias")),
            }
            self.layers.append(entry)
            self.norms += [norm1, norm2]
            self.attentions.append(attn)
        final = child(model, "final_norm")
        self.final_norm = (param(final, "weight"), param(final, "bias"))
        self.norms.append(final)
        self.slots = tuple(slots)
        self.modules = tuple(modules)
        self.tensors = tuple(tensors)

    def intact(self) -> bool:
        return all(d.get(k) is v for d, k, v in self.slots)

    def scalars(self) -> tuple:
        return (tuple([n.eps for n in self.norms]),
                tuple([(a.num_heads, a.head_dim, a.d_model, a.scale) for a in self.attentions]))

    def resolve(self, cache: ReplayCache, fuse_out: bool) -> _Operands:
        """Operands of every block; the out-projection weights are packed for
        the fused projection + residual + LayerNorm kernel only with
        ``fuse_out`` (otherwise the packs are dropped)."""
        eps = [n.eps for n in self.norms]
        exits = [_Norm(*entry["norm1"], eps[2 * i]) for i, entry in enumerate(self.layers)]
        exits.append(_Norm(*self.final_norm, eps[-1]))
        blocks = []
        for index, (entry, attn) in enumerate(zip(self.layers, self.attentions)):
            qkv = entry["qkv"]
            pack = cache.pack_for(index, qkv[:3], qkv[3:])
            out_packed = cache.out_pack_for(index, entry["out"][0]).packed if fuse_out else None
            blocks.append(_Block(
                pack.weight, pack.bias, attn.num_heads, attn.head_dim, attn.scale,
                *entry["out"], _Norm(*entry["norm2"], eps[2 * index + 1]),
                *entry["ffn_in"], *entry["ffn_out"], exits[index + 1], out_packed,
            ))
        if not fuse_out:
            cache.out_packs.clear()
        keepalive = (self.tensors, tuple(cache.packs.values()),
                     tuple(p.packed for p in cache.out_packs.values()))
        return _Operands(exits[0], tuple(blocks), None, keepalive)


class _ModelTally:
    """Adapter that reports launches straight into the model's counters."""

    __slots__ = ("model",)

    def __init__(self, model: "UserOptimizedTransformer") -> None:
        self.model = model

    def count_attention(self, selected: str) -> None:
        counts = self.model.attention_backend_counts
        counts[selected] = counts.get(selected, 0) + 1

    def count_fused_norm(self) -> None:
        self.model.fused_residual_layer_norm_calls += 1


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
        self.cuda_graph_replays = 0
        self.attention_backend_counts: Dict[str, int] = {"hip": 0, "reference": 0}
        self.fused_residual_layer_norm_calls = 0
        # True: in bf16/fp16 models of width 1024, each block's attention
        # output projection and its first residual + LayerNorm run as one HIP
        # kernel.  Off by default: at config 4 the library GEMM plus the
        # residual + LayerNorm kernel is faster.
        self.fuse_out_projection_norm = False
        # Captures, packed projections and the lock: derived inference state,
        # outside the state dict and not copied with the module.
        self._replay = ReplayCache(max_cuda_graphs)

    # -- surface ---------------------------------------------------------------
    @property
    def max_cuda_graphs(self) -> int:
        return self._replay.capacity

    @property
    def _inference_graph(self) -> Optional[CapturedForward]:
        """The capture the last replayed forward used (None after a drop)."""
        return self._replay.last

    @property
    def _inference_graphs(self):
        return self._replay.entries

    @property
    def _packed_qkv_cache(self) -> dict:
        return dict(self._replay.packs)

    def reset_attention_backend_counts(self) -> None:
        self.attention_backend_counts = {"hip": 0, "reference": 0}
        self.fused_residual_layer_norm_calls = 0
        self.cuda_graph_replays = 0

    def clear_cuda_graph(self) -> None:
        """Release every cached capture; a later eligible call rebuilds what it needs."""
        with self._replay.lock:
            self._replay.drop_captures()

    def _apply(self, fn, recurse=True):
        # A device or dtype move replaces every parameter's storage: release
        # captures (and their graph pools) and packed weights now rather than
        # at the next forward.
        self._replay.reset()
        return super()._apply(fn, recurse=recurse)

    # -- operand resolution ----------------------------------------------------------
    def _operands(self) -> _Operands:
        """Operands for ``_encode`` and the fingerprint of everything they hold.

        The tree layout (which module and parameter objects sit where) is
        read once and re-checked per call with one identity pass; tensor
        stamps (storage pointer, version) and the scalar settings (eps,
        heads, scale) are re-read per call.  Operands are rebuilt only when
        one of these moved.
        """
        cache = self._replay
        layout = cache.layout
        if layout is None or not layout.intact():
            layout = _Layout(self, cache.layout_epoch + 1)
            cache.layout, cache.layout_epoch, cache.operands = layout, layout.epoch, None
        try:
            stamps = tuple([(t.data_ptr(), t._version) for t in layout.tensors])
        except RuntimeError:  # inference tensors carry no version counter
            stamps = None
        scalars = layout.scalars()
        settled = not any(m.training or m._forward_hooks or m._forward_pre_hooks
                          for m in (self,) + layout.modules)
        fuse_out = bool(self.fuse_out_projection_norm)
        key = (layout.epoch, stamps, scalars, fuse_out)
        ops = cache.operands
        if ops is None or stamps is None or cache.operands_key != key:
            ops = layout.resolve(cache, fuse_out)
            cache.operands, cache.operands_key = ops, key
        fingerprint = None
        if stamps is not None and settled:
            fingerprint = key + (self.config, torch.backends.cuda.matmul.allow_tf32)
        return ops._replace(fingerprint=fingerprint)

    # -- the forward ----------------------------------------------------------------
    def _encode(self, ops: _Operands, x: torch.Tensor, mask: Optional[torch.Tensor],
                tally) -> torch.Tensor:
        """Pre-LN encoder over resolved operands; returns the final normalised output.

        ``x`` carries the residual stream, ``h`` the normalised input of the
        next sublayer.  Each block's second fused residual + LayerNorm zeroes
        the invalid rows of the residual stream (the organizer block's
        masked_fill, benchmark :142-144) and the last one zeroes the invalid
        rows of the output (benchmark :169-171).  Padded rows never reach a
        valid row: their keys are masked in every attention and everything
        else is row-wise.
        """
        masked = mask is not None
        h = layer_norm(x, *ops.entry_norm)
        last = len(ops.blocks) - 1
        workspace = None
        for index, block in enumerate(ops.blocks):
            context = self._attend(block, h, mask, tally)
            norm = block.norm2
            if (self.fuse_out_projection_norm and block.out_packed is not None
                    and linear_ln_supported(context, block.out_packed, block.out_bias, x,
                                            norm.weight, norm.bias) is None):
                # One zeroed workspace serves the forward's launches in turn
                # (each leaves its counters zero); under capture it comes
                # from the graph's pool and is cleared inside the graph.
                if workspace is None:
                    workspace = torch.zeros(linear_ln_workspace_bytes(x.numel() // x.shape[-1]),
                                            dtype=torch.uint8, device=x.device)
                # The block's first residual + LayerNorm zeroes nothing, so
                # the key mask does not enter it.
                x, h = linear_residual_layer_norm(context, block.out_packed, block.out_bias, x,
                                                  norm.weight, norm.bias, norm.eps,
                                                  workspace=workspace)
                tally.count_fused_norm()
            else:
                update = F.linear(context, block.out_weight, block.out_bias)
                x, h = self._fused_norm(x, update, norm, mask, tally)
            x, h = self._fused_norm(x, self._feed_forward(block, h), block.exit_norm, mask, tally,
                                    zero_residual=masked, zero_output=masked and index == last)
        return h

    def _attend(self, block: _Block, h: torch.Tensor, mask, tally) -> torch.Tensor:
        """Multi-head attention of one block up to its output projection:
        the context ``[B, S, width]`` that out_proj maps."""
        batch, seq_len, width = h.shape
        qkv = F.linear(h, block.qkv_weight, block.qkv_bias)
        q, k, v = qkv.view(batch, seq_len, 3, block.num_heads, block.head_dim).unbind(2)
        context, record = attention_forward(q, k, v, mask, causal=self.config.causal,
                                            scale=block.scale, backend=self.attention_backend)
        tally.count_attention(record.selected)
        return context.view(batch, seq_len, width)

    @staticmethod
    def _feed_forward(block: _Block, h: torch.Tensor) -> torch.Tensor:
        """FFN: ``ffn_out(gelu(ffn_in(h)))`` (reference submission.py:506-508).

        bf16: the input projection and its exact GELU are one HIP kernel, the
        GELU in the GEMM's epilogue (same dtype boundaries: the projection is
        rounded to bf16, its GELU rounded again).  Otherwise, and for widths
        that kernel does not take, the library GEMM writes the projection and
        the HIP elementwise GELU runs in place on it.
        """
        w, b = block.ffn_in_weight, block.ffn_in_bias
        if h.dtype == torch.bfloat16 and linear_supported(h, w, b) is None:
            inner = linear_gelu(h, w, b)
        else:
            inner = gelu_(F.linear(h, w, b))
        return F.linear(inner, block.ffn_out_weight, block.ffn_out_bias)

    @staticmethod
    def _fused_norm(x, update, norm: _Norm, mask, tally, *, zero_residual=False,
                    zero_output=False):
        pair = fused_residual_layer_norm(x, update, norm.weight, norm.bias, norm.eps, mask,
                                         zero_invalid_residual=zero_residual,
                                         zero_invalid_normalized=zero_output)
        tally.count_fused_norm()
        return pair

    def _forward_eager(self, x: torch.Tensor,
                       valid_token_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        mask = valid_token_mask
        if mask is not None and not mask.is_contiguous():
            mask = mask.contiguous()
        # Operand resolution updates the shared cache: under the lock, like
        # every capture and replay; the eager forward itself runs outside it.
        with self._replay.lock:
            ops = self._operands()
        return self._encode(ops, x.contiguous(), mask, _ModelTally(self))

    def forward(self, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        if self._replay_refusal(x, valid_token_mask) is None:
            # Resolve, fingerprint and replay under one hold of the lock, so
            # another thread cannot move the cached operands in between.
            with self._replay.lock:
                ops = self._operands()
                if ops.fingerprint is not None:
                    return self._replay_forward(ops, x, valid_token_mask)
        return self._forward_eager(x, valid_token_mask)

    # -- graph replay -------------------------------------------------------------
    def _replay_forward(self, ops: _Operands, x, mask) -> torch.Tensor:
        geometry = (x.device, tuple(x.shape), x.dtype, mask is not None,
                    torch.is_inference_mode_enabled())
        cache = self._replay
        # The lock orders host-side capture and replay; the capture's event
        # orders its static buffers between caller streams.
        with cache.lock:
            captured = cache.entry(
                (ops.fingerprint, self.attention_backend), geometry,
                lambda: CapturedForward(lambda xs, ms, t: self._encode(ops, xs, ms, t), x, mask,
                                        ops.keepalive),
            )
            result = captured.replay(x, mask)
            for selected, count in captured.tally.attention.items():
                self.attention_backend_counts[selected] = (
                    self.attention_backend_counts.get(selected, 0) + count)
            self.fused_residual_layer_norm_calls += captured.tally.fused_norms
            self.cuda_graph_replays += 1
        return result

    def _can_replay_cuda_graph(self, x, valid_token_mask) -> bool:
        if self._replay_refusal(x, valid_token_mask) is not None:
            return False
        with self._replay.lock:
            return self._operands().fingerprint is not None

    def _replay_refusal(self, x: torch.Tensor, mask: Optional[torch.Tensor]) -> Optional[str]:
        """The first rule that keeps this call eager, or None if it may replay.

        Eligibility follows the reference's (submission.py:561-601) without its
        measured-shape whitelist: eval-mode inference of a supported dtype on
        the current ROCm device, no autograd, autocast, compilation, capture
        in progress or global module hooks; the input must match the model's
        width, dtype and device.
        """
        if self.execution_mode != "auto":
            return "execution_mode='eager'"
        if self.attention_backend != "auto":
            return "attention backend is forced"
        if self.training:
            return "training mode"
        if torch.is_grad_enabled():
            return "autograd enabled"
        if not x.is_cuda:
            return "input not on a ROCm device"
        if x.ndim != 3 or x.shape[2] != self.config.d_model or x.numel() == 0:
            return "input is not a non-empty [batch, seq, d_model] tensor"
        if not x.is_contiguous():
            return "input not contiguous"
        if x.dtype not in SUPPORTED_DTYPES:
            return "unsupported dtype"
        if x.dtype != self.final_norm.weight.dtype or x.device != self.final_norm.weight.device:
            return "input dtype or device differs from the model's"
        if torch.cuda.current_device() != x.device.index:
            return "input not on the current device"
        if torch.cuda.is_current_stream_capturing():
            return "caller is capturing a graph"
        if torch.is_autocast_enabled("cuda"):
            return "autocast enabled"
        if torch.compiler.is_compiling():
            return "inside torch.compile"
        if nn.modules.module._global_forward_hooks or nn.modules.module._global_forward_pre_hooks:
            return "global module hooks registered"
        if mask is not None and (mask.shape != x.shape[:2] or mask.dtype is not torch.bool
                                 or mask.device != x.device or not mask.is_contiguous()):
            return "mask is not a contiguous [batch, seq] bool tensor on the input's device"
        return None


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
