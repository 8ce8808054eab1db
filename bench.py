#!/usr/bin/env python3
"""Benchmark of the MI355X hot path: fused attention, residual+LayerNorm, encoder.

Driver contract: ``python bench.py --gpus N --steps K --warmup W`` prints ONE
JSON line.  A "step" is one fused-attention launch over the BASELINE config-2
workload (fp32, Q/K/V [B=8, S=1024, H=16, D=64] in the reference's BSHD
layout, causal, scale 1/sqrt(D), inputs resident in HBM).  ``value`` is the
whole-job throughput in TFLOP/s of algorithmic causal FLOPs
(4*B*H*D*S(S+1)/2 - masked or skipped pairs are not counted) over the wall
clock of exactly K steps bracketed by device synchronisation.

Also reported in the same line:
* ``roofline``: the attention kernel's achieved TFLOP/s from HIP events on
  the launch stream around the K back-to-back launches (elapsed / K = the
  average launch duration), against the 157.3 TFLOP/s fp32 MFMA peak;
  ``traffic`` (HBM bytes per launch) comes from the committed rocprofv3 PMC
  summary in profiles/traffic.json when present, else null;
* ``cpu_baseline``: the reference's explicit PyTorch attention (the oracle's
  restatement, kind "port") timed on this host's cores on a bounded sample of
  the same workload (``value``), plus the explicit residual+LayerNorm (GB/s)
  and the explicit encoder (tokens/s, configs 1 and 4) beside it;
* ``clock_settle``: untimed launches of the step for ``--settle-s`` seconds
  before the W warm-up steps, so the K timed steps do not include the GPU's
  clock ramp;
* ``secondary``: the S sweep {256..4096} causal/non-causal (config 2), the
  residual+LayerNorm HBM GB/s per hidden size with rotating input sets larger
  than the 256 MB MALL (config 3), bf16 long-sequence attention (config 5a),
  the config-4 FFN input in bf16 as the fused Linear + exact-GELU kernel
  against the library GEMM plus the GELU kernel, and encoder tokens/s with
  hipGraph replay (config 4, fp32 and bf16).  Each
  figure there follows 1 s of untimed calls of its own workload (the clock
  follows the power draw of the work in flight), and each kernel figure is
  the average launch over back-to-back launches between two events, as for
  ``roofline``.  ``--quick`` skips the secondary block.

One GPU only: ``--gpus`` other than 1 exits with a message.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "triton-transformer-kernels_amd"))

METRIC = "fused-attn TFLOP/s + model tokens/s on 1 MI355X; residual+LN HBM GB/s"
FP32_MFMA_PEAK_TFLOPS = 157.3
BF16_MFMA_PEAK_TFLOPS = 2516.6  # dense (no sparsity)
HBM_PEAK_GBPS = 8000.0
MALL_BYTES = 256 * 1024 * 1024


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def attention_flops(batch: int, heads: int, seq_len: int, head_dim: int, causal: bool) -> float:
    """4*B*H*D per allowed (query, key) pair: Q.K and P.V multiply-adds."""
    pairs = seq_len * (seq_len + 1) / 2 if causal else float(seq_len) * seq_len
    return 4.0 * batch * heads * head_dim * pairs


def layer_norm_bytes(rows: int, hidden: int, elem: int = 4) -> float:
    """Read x and u, write r and y (rows*hidden each) plus gamma and beta."""
    return float(rows) * hidden * elem * 4 + 2.0 * hidden * elem


def time_launches(fn, steps: int, warmup: int):
    """Warm up, then time `steps` calls; returns (wall seconds, per-call event ms)."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        starts[i].record(stream)
        fn()
        ends[i].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return wall, [s.elapsed_time(e) for s, e in zip(starts, ends)]


def make_qkv(batch, seq_len, heads, head_dim, dtype, seed):
    import torch

    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    shape = (batch, seq_len, heads, head_dim)
    return tuple(torch.randn(shape, generator=g, device="cuda", dtype=torch.float32).to(dtype)
                 for _ in range(3))


# Seconds of untimed calls of a secondary workload before its warm-up: the
# GPU's clock follows the power draw of the work in flight with a lag of
# tens of milliseconds or more, so a short measurement taken right after a
# different workload (or idling) runs at that workload's clock.
SECONDARY_SETTLE_S = 1.0


def settle(fn, seconds: float) -> None:
    """Call `fn` for about `seconds` of wall time (synchronising every 10 calls)."""
    import torch

    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(10):
            fn()
        torch.cuda.synchronize()


def back_to_back_ms(fn, steps: int, warmup: int, settle_s: float = SECONDARY_SETTLE_S) -> float:
    """Average time per call (ms) of `steps` back-to-back calls between two
    events on the current stream, after `settle_s` seconds and `warmup` more
    untimed calls: the launch duration rocprofv3 --stats averages (an event
    pair around every launch adds microseconds of its own to a ~50 us
    kernel)."""
    import torch

    settle(fn, settle_s)
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    begin = torch.cuda.Event(enable_timing=True)
    finish = torch.cuda.Event(enable_timing=True)
    begin.record(stream)
    for _ in range(steps):
        fn()
    finish.record(stream)
    torch.cuda.synchronize()
    return begin.elapsed_time(finish) / steps


def ffn_input_operands():
    """The config-4 encoder's FFN input projection in bf16: activations
    [8192, 1024] ~ N(0, 1), Xavier-uniform weight [4096, 1024], bias ~ N(0, 0.02)."""
    import torch

    g = torch.Generator(device="cuda").manual_seed(4)
    x = torch.randn(8192, 1024, device="cuda", generator=g).to(torch.bfloat16)
    bound = (6.0 / (1024 + 4096)) ** 0.5
    w = ((torch.rand(4096, 1024, device="cuda", generator=g) * 2 - 1) * bound).to(torch.bfloat16)
    b = (torch.randn(4096, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    return x, w, b


def out_projection_norm_operands():
    """The config-4 encoder's attention output projection and the residual +
    LayerNorm after it, bf16: context and residual [8192, 1024] ~ N(0, 1),
    Xavier-uniform weight [1024, 1024], biases ~ N(0, 0.02), gamma ~ U(0.5,
    1.5), beta ~ N(0, 0.1)."""
    import torch

    g = torch.Generator(device="cuda").manual_seed(5)
    a = torch.randn(8192, 1024, device="cuda", generator=g).to(torch.bfloat16)
    bound = (6.0 / 2048) ** 0.5
    w = ((torch.rand(1024, 1024, device="cuda", generator=g) * 2 - 1) * bound).to(torch.bfloat16)
    b = (torch.randn(1024, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    x = torch.randn(8192, 1024, device="cuda", generator=g).to(torch.bfloat16)
    gamma = (torch.rand(1024, device="cuda", generator=g) + 0.5).to(torch.bfloat16)
    beta = (torch.randn(1024, device="cuda", generator=g) * 0.1).to(torch.bfloat16)
    return a, w, b, x, gamma, beta


def ffn_input_ab(steps: int = 50, warmup: int = 10) -> dict:
    """Per-call times (us) of the config-4 FFN input in bf16: the fused Linear +
    exact-GELU kernel against what it replaces (library GEMM, then the
    elementwise GELU kernel in place), alternating twice, best of each."""
    import torch
    import torch.nn.functional as F

    from transformer_opt.kernels import gelu_, linear_gelu

    x, w, b = ffn_input_operands()
    routes = {"fused_linear_gelu": lambda: linear_gelu(x, w, b),
              "library_gemm_then_gelu": lambda: gelu_(F.linear(x, w, b)),
              "library_gemm_only": lambda: F.linear(x, w, b)}
    best = {}
    with torch.inference_mode():
        for _ in range(2):
            for name, fn in routes.items():
                us = back_to_back_ms(fn, steps, warmup) * 1e3
                best[name] = min(best.get(name, us), us)
    flop = 2.0 * 8192 * 4096 * 1024
    out = {name: {"us": round(us, 2), "tflops": round(flop / us / 1e6, 1)} for name, us in best.items()}
    out["fused_speedup_vs_pair"] = round(best["library_gemm_then_gelu"] / best["fused_linear_gelu"], 3)
    return out


def out_projection_norm_ab(steps: int = 50, warmup: int = 10) -> dict:
    """Per-call times (us) of the config-4 attention output projection and the
    residual + LayerNorm after it, bf16: the fused kernel (an opt-in model
    route) against the library GEMM followed by the residual + LayerNorm
    kernel (the model's default), alternating twice, best of each."""
    import torch
    import torch.nn.functional as F

    from transformer_opt.kernels import fused_residual_layer_norm
    from transformer_opt.kernels.linear_ln import linear_residual_layer_norm, pack_weight

    a, w, b, x, gamma, beta = out_projection_norm_operands()
    best = {}
    with torch.inference_mode():
        wp = pack_weight(w)
        routes = {"fused_linear_residual_ln": lambda: linear_residual_layer_norm(a, wp, b, x, gamma, beta, 1e-5),
                  "library_gemm_then_residual_ln": lambda: fused_residual_layer_norm(
                      x, F.linear(a, w, b), gamma, beta, 1e-5)}
        for _ in range(2):
            for name, fn in routes.items():
                us = back_to_back_ms(fn, steps, warmup) * 1e3
                best[name] = min(best.get(name, us), us)
    out = {name: {"us": round(us, 2)} for name, us in best.items()}
    out["fused_speedup_vs_pair"] = round(best["library_gemm_then_residual_ln"] / best["fused_linear_residual_ln"], 3)
    return out


def attention_tflops(batch, seq_len, heads, head_dim, causal, dtype, steps=10, warmup=3):
    from transformer_opt.kernels import hip_attention

    q, k, v = make_qkv(batch, seq_len, heads, head_dim, dtype, seed=seq_len)
    out = q.new_empty(q.shape)

    def run():
        hip_attention(q, k, v, causal=causal, out=out)

    ms = back_to_back_ms(run, steps, warmup)
    return attention_flops(batch, heads, seq_len, head_dim, causal) / (ms * 1e-3) / 1e12, ms


def packed_attention_5b_us(steps: int = 50, warmup: int = 5) -> float:
    """Average launch (us) of the config-5b encoder's attention: fp32, non-causal,
    [512, 64, 8, 64] on the unbind views of one packed [512, 64, 3, 8, 64]
    projection, between two events around ``steps`` back-to-back launches."""
    import torch

    from transformer_opt.kernels import hip_attention

    g = torch.Generator(device="cuda").manual_seed(7)
    packed = torch.randn(512, 64, 3, 8, 64, device="cuda", generator=g)
    q, k, v = packed.unbind(dim=2)
    out = torch.empty(512, 64, 8, 64, device="cuda")
    return back_to_back_ms(lambda: hip_attention(q, k, v, causal=False, out=out), steps, warmup) * 1e3


def layer_norm_gbps(hidden: int, rows: int = 32768, steps: int = 50, warmup: int = 5):
    """Config 3: rotate input sets so their total exceeds the 256 MB MALL.

    The time per call is the average over `steps` back-to-back launches between
    two events on the launch stream (a per-launch event pair adds microseconds
    of its own to a ~20 us kernel)."""
    import torch

    from transformer_opt.kernels import fused_residual_layer_norm

    g = torch.Generator(device="cuda")
    g.manual_seed(hidden)
    set_bytes = rows * hidden * 4 * 4
    nsets = max(3, -(-2 * MALL_BYTES // set_bytes))
    sets = []
    for _ in range(nsets):
        x = torch.randn(rows, hidden, generator=g, device="cuda")
        u = torch.randn(rows, hidden, generator=g, device="cuda")
        sets.append((x, u))
    w = torch.rand(hidden, generator=g, device="cuda") + 0.5
    b = torch.randn(hidden, generator=g, device="cuda") * 0.1
    counter = [0]

    def run():
        x, u = sets[counter[0] % nsets]
        counter[0] += 1
        fused_residual_layer_norm(x, u, w, b, 1e-5)

    with torch.inference_mode():
        ms = back_to_back_ms(run, steps, warmup)
    return layer_norm_bytes(rows, hidden) / (ms * 1e-3) / 1e9, ms, nsets


# TransformerConfig fields: batch, seq_len, d_model, heads, ffn, layers, causal.
ENCODER_CONFIG4 = (4, 2048, 1024, 16, 4096, 6, True)
# Config 5b: huge batch of short sequences, fp32 (FFN 4*d, non-causal).
ENCODER_CONFIG5B = (512, 64, 512, 8, 2048, 4, False)


def model_tokens_per_second(dtype_name: str, cfg=ENCODER_CONFIG4, steps: int = 5, warmup: int = 2):
    """Encoder tokens/s with hipGraph replay (config 4 by default)."""
    import torch

    from transformer_opt.submission import TransformerConfig, UserOptimizedTransformer

    dtype = {"fp32": torch.float32, "bf16": torch.bfloat16}[dtype_name]
    config = TransformerConfig(*cfg)
    batch, seq_len, d_model = cfg[0], cfg[1], cfg[2]
    torch.manual_seed(1234)
    model = UserOptimizedTransformer(config).to(device="cuda", dtype=dtype).eval()
    g = torch.Generator(device="cuda")
    g.manual_seed(1234)
    x = torch.randn(batch, seq_len, d_model, generator=g, device="cuda").to(dtype)
    with torch.inference_mode():
        settle(lambda: model(x), SECONDARY_SETTLE_S)
        wall, ms = time_launches(lambda: model(x), steps, warmup)
        replays = model.cuda_graph_replays
    med = statistics.median(ms)
    del model
    torch.cuda.empty_cache()
    return batch * seq_len * 1000.0 / med, med, replays


def _median_call_seconds(fn, min_calls: int, max_calls: int, budget_s: float) -> tuple:
    """One untimed warm-up call, then perf_counter_ns per call (the reference's
    timer, benchmarks/torch_transformer_benchmark.py:501-506) until at least
    ``min_calls`` calls and the budget or ``max_calls`` is reached."""
    fn()
    samples = []
    t_start = time.perf_counter()
    while len(samples) < min_calls or (time.perf_counter() - t_start < budget_s
                                       and len(samples) < max_calls):
        t0 = time.perf_counter_ns()
        fn()
        samples.append((time.perf_counter_ns() - t0) / 1e9)
    return statistics.median(samples), len(samples)


def _cpu_model_tokens_per_second(cfg, batch: int, min_calls: int, budget_s: float) -> dict:
    """The organizer's explicit encoder (oracle restatement of benchmarks/
    torch_transformer_benchmark.py:59-172) on ``batch`` sequences of ``cfg``."""
    import torch

    from oracle.model import BaselineTransformer, TransformerConfig

    config = TransformerConfig(batch, *cfg[1:])
    torch.manual_seed(1234)
    model = BaselineTransformer(config).eval()
    x = torch.randn(batch, config.seq_len, config.d_model, generator=torch.Generator().manual_seed(3))
    with torch.inference_mode():
        med, calls = _median_call_seconds(lambda: model(x), min_calls, 20, budget_s)
    return {"tokens_per_s": round(batch * config.seq_len / med, 1), "ms": round(med * 1e3, 2),
            "calls": calls}


def cpu_baseline(time_budget_s: float = 8.0):
    """The reference's explicit PyTorch path on host cores, bounded samples.

    All three CPU paths the baseline plan names, timed in this process on
    identically generated fp32 inputs, median per call after a warm-up:

    * attention (``value``): the oracle restatement of the explicit attention
      (reference transformer_opt/dispatch.py:69-96) on the config-2 workload
      (causal, S=1024, D=64), one of the 8 batch elements (16 heads) per call,
      as algorithmic causal TFLOP/s;
    * residual + LayerNorm: ``x + u`` then ``F.layer_norm`` (the reference's
      explicit order) on config 3 rows=32768, hidden=1024, as GB/s of the same
      algorithmic bytes the GPU figure uses;
    * the explicit encoder (benchmarks/torch_transformer_benchmark.py:59-172):
      config 1 (B=2, S=128, d=256, 1 layer, the reference's CPU-runnable
      case) and one of the 4 sequences of config 4 (S=2048, d=1024, 6 layers,
      causal), as tokens/s.
    """
    import torch
    import torch.nn.functional as F

    sys.path.insert(0, str(REPO))
    from oracle.attention import kernel_contract_attention

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    g = torch.Generator().manual_seed(7)
    shape = (1, 1024, 16, 64)
    q, k, v = (torch.randn(shape, generator=g) for _ in range(3))
    att_s, att_calls = _median_call_seconds(
        lambda: kernel_contract_attention(q, k, v, None, True), 5, 50, time_budget_s)
    tflops = attention_flops(1, 16, 1024, 64, True) / att_s / 1e12

    rows, hidden = 32768, 1024
    x = torch.randn(rows, hidden, generator=g)
    u = torch.randn(rows, hidden, generator=g)
    w = torch.rand(hidden, generator=g) + 0.5
    b = torch.randn(hidden, generator=g) * 0.1

    def residual_norm():
        r = x + u
        return r, F.layer_norm(r, (hidden,), w, b, 1e-5)

    ln_s, ln_calls = _median_call_seconds(residual_norm, 5, 50, time_budget_s / 2)
    del x, u
    model_1 = _cpu_model_tokens_per_second((2, 128, 256, 4, 1024, 1, False), 2, 5, 2.0)
    model_4 = _cpu_model_tokens_per_second(ENCODER_CONFIG4, 1, 3, 1.0)
    return {
        "value": tflops,
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"explicit PyTorch attention (oracle restatement of reference dispatch.py:69-96), "
                   f"fp32 causal, 1 of 8 batch elements of [8,1024,16,64] per call, median of "
                   f"{att_calls} calls ({att_s * 1e3:.1f} ms each); os.cpu_count()={os.cpu_count()}, "
                   f"cpu={platform.processor() or platform.machine()}"),
        "residual_layernorm": {
            "gbps": round(layer_norm_bytes(rows, hidden) / ln_s / 1e9, 2), "ms": round(ln_s * 1e3, 2),
            "calls": ln_calls,
            "sample": "x + u then F.layer_norm, fp32 [32768, 1024] (config 3 at hidden 1024)"},
        "model_config1": dict(model_1, sample="explicit encoder, fp32, B=2 S=128 d=256 H=4 FFN 1024, 1 layer"),
        "model_config4": dict(model_4, sample="explicit encoder, fp32, 1 of 4 sequences of config 4 "
                                              "(S=2048 d=1024 H=16 FFN 4096, 6 layers, causal)"),
    }


def profile_only(which: str, steps: int, warmup: int, seq_len: int = 1024, hidden: int = 4096,
                 settle_s: float = 0.0) -> int:
    """Launch one kernel `steps` times (after `settle_s` seconds of untimed launches
    and `warmup` more) for a profiler run.

    attention:      fp32 causal [8,S,16,64], S = --seq-len (1024: the headline step)
    attention_bf16: bf16 causal [1,16384,32,128] (config 5a)
    attention_bf16_d64: bf16 causal [4,2048,16,64] (the attention of the config-4 encoder)
    attention_5b:   fp32 non-causal [512,64,8,64] on packed-QKV views (the attention of the
                    config-5b encoder)
    encoder_fp32 / encoder_bf16: config-4 encoder forward (hipGraph replay), for the
                    per-kernel split
    encoder_5b:     config-5b encoder forward (fp32, B=512, S=64, d=512, 4 layers,
                    hipGraph replay), for the per-kernel split
    gelu:           exact GELU, bf16, the config-4 FFN activation [8192, 4096] (GB/s)
    linear_gelu:    fused Linear + exact GELU, bf16, the config-4 FFN input
                    ([8192, 1024] x [4096, 1024]^T + b)
    linear_gelu_pair: the same FFN input as the library GEMM (F.linear) followed by
                    the elementwise GELU kernel in place (what the fused kernel replaces)
    layernorm:      fp32 residual+LN rows=32768, hidden = --hidden (config 3), rotating
                    among input sets that together exceed twice the 256 MB MALL
    layernorm_bf16: bf16 residual+LN rows=8192, hidden=1024 (the config-4 encoder's LN),
                    rotating input sets as above
    copy:           a plain device copy of 256 MiB (the PMC byte-counter calibration:
                    FETCH_SIZE and WRITE_SIZE should each read 262144 KiB per dispatch)
    """
    import torch

    from transformer_opt.kernels import fused_residual_layer_norm, hip_attention

    if which == "attention":
        q, k, v = make_qkv(8, seq_len, 16, 64, torch.float32, seed=1234)
        out = torch.empty_like(q)
        fn = lambda: hip_attention(q, k, v, causal=True, out=out)  # noqa: E731
        work = attention_flops(8, 16, seq_len, 64, True)
    elif which == "attention_bf16":
        q, k, v = make_qkv(1, 16384, 32, 128, torch.bfloat16, seed=5)
        out = torch.empty_like(q)
        fn = lambda: hip_attention(q, k, v, causal=True, out=out)  # noqa: E731
        work = attention_flops(1, 32, 16384, 128, True)
    elif which == "attention_bf16_d64":
        q, k, v = make_qkv(4, 2048, 16, 64, torch.bfloat16, seed=6)
        out = torch.empty_like(q)
        fn = lambda: hip_attention(q, k, v, causal=True, out=out)  # noqa: E731
        work = attention_flops(4, 16, 2048, 64, True)
    elif which == "attention_5b":
        g = torch.Generator(device="cuda").manual_seed(7)
        packed = torch.randn(512, 64, 3, 8, 64, device="cuda", generator=g)
        q, k, v = packed.unbind(dim=2)
        out = torch.empty(512, 64, 8, 64, device="cuda")
        fn = lambda: hip_attention(q, k, v, causal=False, out=out)  # noqa: E731
        work = attention_flops(512, 8, 64, 64, False)
    elif which == "layernorm":
        rows = 32768
        nsets = max(1, -(-2 * MALL_BYTES // (rows * hidden * 4 * 4)))
        sets = [(torch.randn(rows, hidden, device="cuda"), torch.randn(rows, hidden, device="cuda"))
                for _ in range(nsets)]
        w = torch.rand(hidden, device="cuda") + 0.5
        b = torch.randn(hidden, device="cuda") * 0.1
        calls = iter(range(1 << 62))

        def fn():
            x, u = sets[next(calls) % nsets]
            fused_residual_layer_norm(x, u, w, b, 1e-5)

        work = layer_norm_bytes(rows, hidden)
    elif which == "layernorm_bf16":
        rows, width = 8192, 1024
        nsets = max(1, -(-2 * MALL_BYTES // (rows * width * 2 * 4)))
        sets = [(torch.randn(rows, width, device="cuda").to(torch.bfloat16),
                 torch.randn(rows, width, device="cuda").to(torch.bfloat16)) for _ in range(nsets)]
        w = (torch.rand(width, device="cuda") + 0.5).to(torch.bfloat16)
        b = (torch.randn(width, device="cuda") * 0.1).to(torch.bfloat16)
        calls = iter(range(1 << 62))

        def fn():
            x, u = sets[next(calls) % nsets]
            fused_residual_layer_norm(x, u, w, b, 1e-5)

        work = layer_norm_bytes(rows, width, elem=2)
    elif which == "gelu":
        from transformer_opt.kernels import gelu_

        act = torch.randn(8192, 4096, device="cuda").to(torch.bfloat16)
        fn = lambda: gelu_(act)  # noqa: E731
        work = 2.0 * act.numel() * 2  # bytes: read and write once
    elif which in ("linear_gelu", "linear_gelu_pair"):
        from transformer_opt.kernels import gelu_, linear_gelu

        x, w, b = ffn_input_operands()
        if which == "linear_gelu":
            fn = lambda: linear_gelu(x, w, b)  # noqa: E731
        else:
            fn = lambda: gelu_(torch.nn.functional.linear(x, w, b))  # noqa: E731
        work = 2.0 * 8192 * 4096 * 1024
    elif which in ("linear_ln", "linear_ln_pair"):
        from transformer_opt.kernels import fused_residual_layer_norm
        from transformer_opt.kernels.linear_ln import linear_residual_layer_norm, pack_weight

        a, w, b, x, gamma, beta = out_projection_norm_operands()
        if which == "linear_ln":
            wp = pack_weight(w)
            fn = lambda: linear_residual_layer_norm(a, wp, b, x, gamma, beta, 1e-5)  # noqa: E731
        else:
            fn = lambda: fused_residual_layer_norm(  # noqa: E731
                x, torch.nn.functional.linear(a, w, b), gamma, beta, 1e-5)
        work = 2.0 * 8192 * 1024 * 1024
    elif which in ("encoder_fp32", "encoder_bf16"):
        from transformer_opt.submission import TransformerConfig, UserOptimizedTransformer

        dtype = torch.float32 if which == "encoder_fp32" else torch.bfloat16
        torch.manual_seed(1234)
        model = UserOptimizedTransformer(TransformerConfig(4, 2048, 1024, 16, 4096, 6, True))
        model = model.to(device="cuda", dtype=dtype).eval()
        x = torch.randn(4, 2048, 1024, device="cuda").to(dtype)
        fn = lambda: model(x)  # noqa: E731
        work = 4 * 2048  # tokens
    elif which == "encoder_5b":
        from transformer_opt.submission import TransformerConfig, UserOptimizedTransformer

        torch.manual_seed(1234)
        model = UserOptimizedTransformer(TransformerConfig(*ENCODER_CONFIG5B)).to(device="cuda").eval()
        x = torch.randn(ENCODER_CONFIG5B[0], ENCODER_CONFIG5B[1], ENCODER_CONFIG5B[2], device="cuda")
        fn = lambda: model(x)  # noqa: E731
        work = ENCODER_CONFIG5B[0] * ENCODER_CONFIG5B[1]  # tokens
    else:
        src = torch.empty(64 * 1024 * 1024, device="cuda")
        dst = torch.empty_like(src)
        fn = lambda: dst.copy_(src)  # noqa: E731
        work = 2.0 * src.numel() * 4
    with torch.inference_mode():
        # The same clock settling as the headline run, so a profile of the
        # step sees the clocks the bench line is measured at.
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < settle_s:
            for _ in range(10):
                fn()
            torch.cuda.synchronize()
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        begin = torch.cuda.Event(enable_timing=True)
        finish = torch.cuda.Event(enable_timing=True)
        begin.record()
        for _ in range(steps):
            fn()
        finish.record()
        torch.cuda.synchronize()
    ms = begin.elapsed_time(finish) / steps
    if which in ("layernorm", "layernorm_bf16", "copy", "gelu"):
        rate, unit = work / (ms * 1e-3) / 1e9, "GB/s"
    elif which.startswith("encoder"):
        rate, unit = work / (ms * 1e-3), "tokens/s"
    else:
        rate, unit = work / (ms * 1e-3) / 1e12, "TFLOP/s"
    print(json.dumps({"profile_only": which, "steps": steps, "avg_launch_us": round(ms * 1e3, 2),
                      "rate": round(rate, 2), "unit": unit}), flush=True)
    return 0


def load_traffic(key: str):
    path = REPO / "profiles" / "traffic.json"
    if not path.exists():
        return None
    try:
        return json.loads(path.read_text()).get(key)
    except (OSError, ValueError):
        return None


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=200)
    parser.add_argument("--warmup", type=int, default=50)
    parser.add_argument("--quick", action="store_true", help="skip the secondary measurements")
    parser.add_argument("--settle-s", type=float, default=1.0,
                        help="seconds of untimed launches before the warm-up (clock settling)")
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--profile-only", choices=("attention", "layernorm", "layernorm_bf16", "copy", "attention_bf16",
                                                   "attention_bf16_d64", "attention_5b", "encoder_fp32", "encoder_bf16",
                                                   "encoder_5b", "gelu", "linear_gelu", "linear_gelu_pair",
                                                   "linear_ln", "linear_ln_pair"),
                        help="launch only one kernel (warmup + steps) for rocprofv3 runs; prints its timing")
    parser.add_argument("--seq-len", type=int, default=1024,
                        help="sequence length of --profile-only attention (B=8, H=16, D=64, fp32)")
    parser.add_argument("--hidden", type=int, default=4096,
                        help="hidden size of --profile-only layernorm (rows=32768, fp32)")
    args = parser.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one MI355X; --gpus {args.gpus} is not supported "
              "(this build has no multi-GPU path: heads/batch shard without exchange)", file=sys.stderr)
        return 2
    if args.steps <= 0 or args.warmup < 0:
        print("--steps must be positive and --warmup non-negative", file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    from transformer_opt import _native
    from transformer_opt.kernels import hip_attention

    _native.load()
    dev_name = torch.cuda.get_device_name(0)
    log(f"device {dev_name}; library {_native.library_path()}")
    if args.profile_only:
        return profile_only(args.profile_only, args.steps, args.warmup, args.seq_len, args.hidden, args.settle_s)

    # ---- headline: config 2, fp32 causal attention, S=1024 -----------------
    B, S, H, D = 8, 1024, 16, 64
    q, k, v = make_qkv(B, S, H, D, torch.float32, seed=1234)
    out = torch.empty_like(q)

    def step():
        hip_attention(q, k, v, causal=True, out=out)

    # Clock settling: the GPU leaves its idle clock only after some
    # sustained work, so the headline would otherwise time the ramp when the
    # warm-up is short.  Launch the step for a fixed wall time before the W
    # warm-up steps; the JSON line reports it.
    settle_launches = 0
    settle_t0 = time.perf_counter()
    while time.perf_counter() - settle_t0 < args.settle_s:
        for _ in range(20):
            step()
        torch.cuda.synchronize()
        settle_launches += 20
    settle_s = time.perf_counter() - settle_t0
    for _ in range(args.warmup):
        step()
    # The kernel is launched on torch's current stream, so events recorded on
    # that stream bracket exactly the K back-to-back launches: their elapsed
    # time / K is the average launch duration (what rocprofv3 --stats reports).
    stream = torch.cuda.current_stream()
    begin = torch.cuda.Event(enable_timing=True)
    finish = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    begin.record(stream)
    for _ in range(args.steps):
        step()
    finish.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    flops = attention_flops(B, H, S, D, True)
    value = flops * args.steps / wall / 1e12
    avg_launch_ms = begin.elapsed_time(finish) / args.steps
    achieved = flops / (avg_launch_ms * 1e-3) / 1e12
    log(f"attention fp32 causal [8,1024,16,64]: {value:.2f} TFLOP/s wall, "
        f"{achieved:.2f} TFLOP/s per launch ({avg_launch_ms * 1e3:.1f} us)")

    result = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic N(0,1) Q/K/V from a fixed seed, resident in HBM",
        "config": {"workload": "fused attention forward, BASELINE config 2", "layout": "BSHD",
                   "B": B, "S": S, "H": H, "D": D, "causal": True, "scale": D ** -0.5},
        "roofline": {
            "bound": "mfma",
            "achieved": round(achieved, 3),
            "peak": FP32_MFMA_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / FP32_MFMA_PEAK_TFLOPS, 4),
            "traffic": load_traffic("attn_fwd_f32_kernel<64,true,false> B8 S1024 H16"),
            "kernel": "attn_fwd_f32_kernel<64, causal>",
            "launch_us": round(avg_launch_ms * 1e3, 2),
        },
        "clock_settle": {"launches": settle_launches, "seconds": round(settle_s, 3),
                         "note": "untimed launches of the step before the warm-up"},
    }
    del q, k, v, out
    torch.cuda.empty_cache()

    if not args.quick:
        secondary = {}
        sweep = {}
        for s_len in (256, 512, 1024, 2048, 4096):
            entry = {}
            for causal in (True, False):
                tf, ms = attention_tflops(8, s_len, 16, 64, causal, torch.float32)
                entry["causal" if causal else "noncausal"] = {
                    "tflops": round(tf, 2), "ms": round(ms, 4),
                    "frac_fp32_mfma_peak": round(tf / FP32_MFMA_PEAK_TFLOPS, 4)}
            entry["causal_speedup_vs_noncausal_time"] = round(
                entry["noncausal"]["ms"] / entry["causal"]["ms"], 3)
            sweep[str(s_len)] = entry
            log(f"attention fp32 S={s_len}: causal {entry['causal']['tflops']} TF, "
                f"non-causal {entry['noncausal']['tflops']} TF")
        secondary["attention_fp32_B8_H16_D64_sweep"] = sweep
        torch.cuda.empty_cache()
        tf, ms = attention_tflops(1, 16384, 32, 128, True, torch.bfloat16, steps=10, warmup=5)
        secondary["attention_bf16_causal_B1_H32_S16384_D128"] = {
            "tflops": round(tf, 2), "ms": round(ms, 3),
            "frac_bf16_mfma_peak": round(tf / BF16_MFMA_PEAK_TFLOPS, 4)}
        log(f"attention bf16 causal long-sequence: {tf:.1f} TF")
        torch.cuda.empty_cache()
        # The attention of the config-4 bf16 encoder and of the config-5b
        # encoder (non-causal fp32 on packed-QKV views), per launch.
        tf, ms = attention_tflops(4, 2048, 16, 64, True, torch.bfloat16, steps=50, warmup=20)
        secondary["attention_bf16_causal_B4_H16_S2048_D64"] = {
            "tflops": round(tf, 2), "us": round(ms * 1e3, 2),
            "frac_bf16_mfma_peak": round(tf / BF16_MFMA_PEAK_TFLOPS, 4)}
        log(f"attention bf16 causal [4,2048,16,64]: {tf:.1f} TF ({ms * 1e3:.1f} us)")
        # Shorter causal bf16 launches (the 32-key-tile kernels: three or four
        # workgroups per CU).
        short = {}
        for b_, s_, d_ in ((16, 512, 64), (8, 1024, 64), (8, 1024, 128)):
            tf, ms = attention_tflops(b_, s_, 16, d_, True, torch.bfloat16, steps=50, warmup=20)
            short[f"B{b_}_S{s_}_H16_D{d_}"] = {
                "tflops": round(tf, 2), "us": round(ms * 1e3, 2),
                "frac_bf16_mfma_peak": round(tf / BF16_MFMA_PEAK_TFLOPS, 4)}
        secondary["attention_bf16_causal_short_sequences"] = short
        log(f"attention bf16 causal short sequences: {short}")
        us = packed_attention_5b_us()
        tf = attention_flops(512, 8, 64, 64, False) / (us * 1e-6) / 1e12
        secondary["attention_fp32_noncausal_B512_H8_S64_D64_packed"] = {
            "tflops": round(tf, 2), "us": round(us, 2),
            "frac_fp32_mfma_peak": round(tf / FP32_MFMA_PEAK_TFLOPS, 4)}
        log(f"attention fp32 config-5b layer: {tf:.1f} TF ({us:.1f} us)")
        torch.cuda.empty_cache()
        ln = {}
        for hidden in (256, 512, 768, 1024, 4096):
            gbps, ms, nsets = layer_norm_gbps(hidden)
            ln[str(hidden)] = {"gbps": round(gbps, 1), "us": round(ms * 1e3, 2),
                               "frac_hbm_peak": round(gbps / HBM_PEAK_GBPS, 4), "rotating_sets": nsets}
            log(f"residual+LN hidden={hidden}: {gbps:.0f} GB/s")
            torch.cuda.empty_cache()
        secondary["residual_layernorm_fp32_rows32768_gbps"] = ln
        # Narrow shapes: width-32 rows (8 rows per wavefront; 2^22 rows so a
        # set is 268 MB) and small head dims, causal [8, 1024, 16, D].
        gbps, ms, nsets = layer_norm_gbps(32, rows=1 << 22, steps=20)
        secondary["residual_layernorm_fp32_hidden32_rows4194304_gbps"] = {
            "gbps": round(gbps, 1), "us": round(ms * 1e3, 2),
            "frac_hbm_peak": round(gbps / HBM_PEAK_GBPS, 4), "rotating_sets": nsets}
        log(f"residual+LN hidden=32 rows=4194304: {gbps:.0f} GB/s")
        torch.cuda.empty_cache()
        small = {}
        for d_head, dt, name in ((8, torch.float16, "fp16"), (8, torch.float32, "fp32"),
                                 (16, torch.float32, "fp32"), (32, torch.float32, "fp32")):
            tf, ms = attention_tflops(8, 1024, 16, d_head, True, dt)
            small[f"D{d_head}_{name}"] = {"tflops": round(tf, 2), "ms": round(ms, 4)}
            log(f"attention {name} causal [8,1024,16,{d_head}]: {tf:.1f} TF")
        secondary["attention_small_head_dim_causal_B8_S1024_H16"] = small
        torch.cuda.empty_cache()
        ffn = ffn_input_ab()
        secondary["ffn_input_bf16_8192x4096x1024"] = ffn
        log(f"FFN input bf16: {ffn}")
        torch.cuda.empty_cache()
        proj = out_projection_norm_ab()
        secondary["out_projection_residual_ln_bf16_8192x1024x1024"] = proj
        log(f"out projection + residual + LN bf16: {proj}")
        torch.cuda.empty_cache()
        model = {}
        for dtype_name in ("fp32", "bf16"):
            tok, ms, replays = model_tokens_per_second(dtype_name)
            model[dtype_name] = {"tokens_per_s": round(tok, 1), "ms": round(ms, 3), "graph_replays": replays}
            log(f"encoder {dtype_name}: {tok:.0f} tokens/s ({ms:.2f} ms)")
        secondary["encoder_6L_d1024_B4_S2048_causal"] = model
        tok, ms, replays = model_tokens_per_second("fp32", ENCODER_CONFIG5B, steps=10, warmup=3)
        secondary["encoder_5b_4L_d512_B512_S64_fp32"] = {
            "tokens_per_s": round(tok, 1), "ms": round(ms, 3), "graph_replays": replays}
        log(f"encoder config 5b fp32: {tok:.0f} tokens/s ({ms:.2f} ms)")
        result["secondary"] = secondary

    if not args.no_cpu_baseline:
        log("timing the CPU baseline (explicit PyTorch attention, residual+LN, encoder)")
        result["cpu_baseline"] = cpu_baseline()
        result["cpu_baseline"]["value"] = round(result["cpu_baseline"]["value"], 5)
    result["device"] = dev_name
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
