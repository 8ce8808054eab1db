"""hipGraph replay of the encoder against eager execution of a twin model.

The replay contract (reference transformer_opt/submission.py:527-723): a
capture is reused while nothing it baked in has changed, and replaced when
anything has; every call returns a tensor the caller owns; replays from
different caller streams are ordered; warm-up and capture are not counted.

Each check drives a replaying model and an eager twin with identical weights
through the same edits and compares every output BITWISE, with eager work and
synchronisations between replays, so a graph node that misbehaves on a later
replay is caught as well.
"""

from __future__ import annotations

import copy
import pickle

import pytest
import torch
import torch.nn as nn

from oracle.model import TransformerConfig

pytestmark = pytest.mark.gpu

CFG = TransformerConfig(2, 96, 128, 4, 256, 3, True)


def twin(cfg=CFG, dtype=torch.float32, seed=0, **kwargs):
    from transformer_opt.submission import UserOptimizedTransformer

    torch.manual_seed(seed)
    replaying = UserOptimizedTransformer(cfg, **kwargs).to("cuda", dtype).eval()
    eager = UserOptimizedTransformer(cfg, execution_mode="eager").to("cuda", dtype).eval()
    eager.load_state_dict(replaying.state_dict(), strict=True)
    return replaying, eager


def sample(cfg=CFG, dtype=torch.float32, seed=1):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(cfg.batch_size, cfg.seq_len, cfg.d_model, generator=g).to("cuda", dtype)


def _fresh_norm(model):
    norm = nn.LayerNorm(CFG.d_model).to("cuda").eval()
    with torch.no_grad():
        norm.weight.fill_(1.25)
        norm.bias.fill_(-0.0625)
    return norm


def _perturbed_state(model):
    state = {k: v.clone() for k, v in model.state_dict().items()}
    state["layers.2.ffn_out.weight"].mul_(-1)
    return state


# (event, edit applied to both models, must the capture in use be replaced?)
MODEL_EVENTS = [
    ("nothing changes", lambda m, s: None, False),
    ("final LayerNorm bias updated in place", lambda m, s: m.final_norm.bias.add_(0.125), True),
    ("Q projection weight updated in place",
     lambda m, s: m.layers[0].attention.q_proj.weight.add_(0.01), True),
    ("V projection bias updated in place",
     lambda m, s: m.layers[1].attention.v_proj.bias.mul_(0.5), True),
    ("FFN weight overwritten by copy_",
     lambda m, s: m.layers[2].ffn_out.weight.copy_(m.layers[2].ffn_out.weight.flip(0)), True),
    ("state dict loaded", lambda m, s: m.load_state_dict(s, strict=True), True),
    ("LayerNorm eps changed", lambda m, s: setattr(m.layers[1].norm2, "eps", 0.02), True),
    ("attention scale changed",
     lambda m, s: setattr(m.layers[0].attention, "scale", m.layers[0].attention.scale * 2), True),
    ("parameter object replaced",
     lambda m, s: setattr(m.layers[2].ffn_in, "bias",
                          nn.Parameter(torch.full_like(m.layers[2].ffn_in.bias, 0.03))), True),
    ("LayerNorm module replaced", lambda m, s: setattr(m.layers[1], "norm2", _fresh_norm(m)), True),
    ("unrelated buffer registered",
     lambda m, s: m.register_buffer("unused", torch.zeros(1, device="cuda")), False),
]


@pytest.mark.parametrize("event,edit,recapture", MODEL_EVENTS, ids=[e[0] for e in MODEL_EVENTS])
def test_model_events_replace_exactly_the_stale_captures(gpu_ready, event, edit, recapture):
    model, eager = twin()
    state = _perturbed_state(model)
    x = sample()
    with torch.inference_mode():
        assert torch.equal(model(x), eager(x))
        before = model._inference_graph
        assert before is not None and model.cuda_graph_replays == 1
    with torch.no_grad():
        edit(model, state)
        edit(eager, state)
    with torch.inference_mode():
        for step in range(2):
            out = model(x)
            torch.cuda.synchronize()
            assert torch.equal(out, eager(x)), (event, step)
        assert (model._inference_graph is not before) == recapture, event
        assert model.cuda_graph_replays == 3


def test_input_geometry_keys_captures(gpu_ready):
    model, eager = twin(max_cuda_graphs=8)
    x = sample()
    mask = torch.ones(CFG.batch_size, CFG.seq_len, dtype=torch.bool, device="cuda")
    with torch.inference_mode():
        model(x, mask)
        masked = model._inference_graph
        # New values and a new mask pattern: same geometry, same capture.
        for lengths in ((96, 96), (40, 96), (1, 7)):
            x.normal_()
            mask.copy_(torch.arange(CFG.seq_len, device="cuda")[None, :]
                       < torch.tensor(lengths, device="cuda")[:, None])
            out = model(x, mask)
            assert model._inference_graph is masked
            assert torch.equal(out, eager(x, mask)), lengths
            assert torch.count_nonzero(out[~mask]) == 0
        # Mask presence, shape and inference context are part of the geometry.
        model(x)
        assert model._inference_graph is not masked
        shorter = x[:, :50].contiguous()
        assert torch.equal(model(shorter), eager(shorter))
        assert len(model._inference_graphs) == 3
    with torch.no_grad():
        out = model(x)
        assert not out.is_inference()
        assert torch.equal(out, eager(x))
    assert len(model._inference_graphs) == 4
    with torch.inference_mode():
        out = model(x, mask)
        assert out.is_inference() and model._inference_graph is masked


def test_every_returned_tensor_stays_owned_by_the_caller(gpu_ready):
    model, eager = twin()
    inputs = [sample(seed=s) for s in range(4)]
    with torch.inference_mode():
        outputs = [model(x) for x in inputs]
        pointers = {o.data_ptr() for o in outputs}
        assert len(pointers) == len(outputs)
        for x, out in zip(inputs, outputs):
            assert torch.equal(out, eager(x))


def test_replays_from_several_caller_streams_stay_ordered(gpu_ready):
    model, eager = twin()
    inputs = [sample(seed=10 + s) for s in range(3)]
    streams = [torch.cuda.Stream() for _ in inputs]
    with torch.inference_mode():
        model(inputs[0])
        results = []
        for stream, x in zip(streams, inputs):
            stream.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(stream):
                results.append(model(x))
        for stream in streams:
            torch.cuda.current_stream().wait_stream(stream)
        torch.cuda.synchronize()
        for x, out in zip(inputs, results):
            assert torch.equal(out, eager(x))


def test_counters_count_forwards_not_warmups(gpu_ready):
    model, _ = twin()
    x = sample()
    mask = torch.ones(CFG.batch_size, CFG.seq_len, dtype=torch.bool, device="cuda")
    with torch.inference_mode():
        for _ in range(3):
            model(x, mask)
    layers = CFG.num_layers
    assert model.cuda_graph_replays == 3
    assert model.attention_backend_counts == {"hip": 3 * layers, "reference": 0}
    assert model.fused_residual_layer_norm_calls == 3 * 2 * layers
    model.reset_attention_backend_counts()
    assert (model.attention_backend_counts, model.fused_residual_layer_norm_calls,
            model.cuda_graph_replays) == ({"hip": 0, "reference": 0}, 0, 0)


# (why the call stays eager, how the call is made, expected refusal)
def _with_hook(model, x):
    handle = model.layers[0].attention.register_forward_pre_hook(lambda *args: None)
    try:
        return model._can_replay_cuda_graph(x, None)
    finally:
        handle.remove()


ELIGIBILITY = [
    ("autograd on", lambda m, x: torch.enable_grad(), "autograd enabled"),
    ("training mode", lambda m, x: m.train(), "training mode"),
    ("autocast", lambda m, x: torch.autocast("cuda"), "autocast enabled"),
]


@pytest.mark.parametrize("why,context,refusal", ELIGIBILITY, ids=[e[0] for e in ELIGIBILITY])
def test_context_rules_keep_calls_eager(gpu_ready, why, context, refusal):
    model, _ = twin()
    x = sample()
    with torch.inference_mode(refusal != "autograd enabled"):
        ctx = context(model, x)
        if hasattr(ctx, "__enter__"):
            with ctx:
                assert model._replay_refusal(x, None) == refusal
        else:
            assert model._replay_refusal(x, None) == refusal


def test_input_rules_keep_calls_eager(gpu_ready):
    model, eager = twin()
    x = sample()
    mask = torch.ones(CFG.batch_size, CFG.seq_len, dtype=torch.bool, device="cuda")
    with torch.inference_mode():
        assert model._replay_refusal(x, None) is None
        assert model._replay_refusal(x.half(), None) == "input dtype or device differs from the model's"
        assert model._replay_refusal(x.double(), None) == "unsupported dtype"
        assert model._replay_refusal(x.transpose(0, 1), None) == "input not contiguous"
        assert model._replay_refusal(x[..., :64].contiguous(), None).startswith("input is not")
        assert model._replay_refusal(x.cpu(), None) == "input not on a ROCm device"
        assert model._replay_refusal(x, mask.int()).startswith("mask is not")
        assert model._replay_refusal(x, mask[:, ::2].repeat(1, 2)) is None
        assert not _with_hook(model, x)
        # A module hook keeps the call eager and the output unchanged.
        handle = model.layers[1].ffn_in.register_forward_hook(lambda *args: None)
        assert torch.equal(model(x), eager(x))
        handle.remove()
        assert model.cuda_graph_replays == 0
    for kwargs, refusal in (({"execution_mode": "eager"}, "execution_mode='eager'"),
                            ({"attention_backend": "triton"}, "attention backend is forced"),
                            ({"attention_backend": "hip"}, "attention backend is forced")):
        forced, _ = twin(**kwargs)
        with torch.inference_mode():
            assert forced._replay_refusal(x, None) == refusal
            assert torch.equal(forced(x), eager(x))
            assert forced.attention_backend_counts == {"hip": CFG.num_layers, "reference": 0}


def test_least_recently_used_capture_is_evicted(gpu_ready):
    model, eager = twin(max_cuda_graphs=2)
    xs = [sample(TransformerConfig(b, s, 128, 4, 256, 3, True), seed=b)
          for b, s in ((1, 64), (2, 48), (3, 32))]
    with torch.inference_mode():
        model(xs[0])
        a = model._inference_graph
        model(xs[1])
        b = model._inference_graph
        for _ in range(2):
            assert torch.equal(model(xs[0]), eager(xs[0])) and model._inference_graph is a
            assert torch.equal(model(xs[1]), eager(xs[1])) and model._inference_graph is b
        model(xs[2])  # evicts xs[0]'s capture, used least recently
        assert list(model._inference_graphs.values())[0] is b
        assert torch.equal(model(xs[0]), eager(xs[0])) and model._inference_graph is not a
        with torch.no_grad():
            model.layers[0].ffn_in.bias.add_(0.01)
        model(xs[1])
        assert len(model._inference_graphs) == 1 and model._inference_graph is not b
    from transformer_opt.submission import UserOptimizedTransformer

    with pytest.raises(ValueError, match="max_cuda_graphs"):
        UserOptimizedTransformer(CFG, max_cuda_graphs=0)


def test_copies_start_without_captures_and_moves_drop_them(gpu_ready):
    model, eager = twin()
    x = sample()
    with torch.inference_mode():
        model(x)
    assert model._inference_graph is not None and model._packed_qkv_cache
    for clone in (copy.deepcopy(model), pickle.loads(pickle.dumps(model))):
        assert clone._inference_graph is None and clone._packed_qkv_cache == {}
        with torch.inference_mode():
            assert torch.equal(clone(x), eager(x))
            assert clone.cuda_graph_replays == model.cuda_graph_replays + 1
    model.clear_cuda_graph()
    assert model._inference_graph is None and len(model._inference_graphs) == 0
    model.half()
    eager.half()
    assert model._inference_graph is None and model._packed_qkv_cache == {}
    with torch.inference_mode():
        assert torch.equal(model(x.half()), eager(x.half()))


@pytest.mark.parametrize("dtype,cfg,masked", [
    (torch.bfloat16, TransformerConfig(2, 200, 256, 4, 512, 2, False), True),
    (torch.float16, TransformerConfig(3, 130, 256, 2, 512, 2, True), True),
    (torch.float32, TransformerConfig(3, 64, 512, 8, 1024, 2, True), False),
])
def test_replay_is_bitwise_eager_across_dtypes(gpu_ready, dtype, cfg, masked):
    model, eager = twin(cfg, dtype, seed=3)
    with torch.inference_mode():
        for step in range(4):
            x = sample(cfg, dtype, seed=20 + step)
            mask = None
            if masked:
                lengths = torch.tensor([cfg.seq_len - 17 * (b + step) for b in range(cfg.batch_size)])
                mask = (torch.arange(cfg.seq_len)[None, :] < lengths[:, None].clamp_min(1)).cuda()
            out = model(x, mask)
            torch.cuda.synchronize()
            reference = eager(x, mask)
            torch.cuda.synchronize()
            assert torch.equal(out, reference), (dtype, step)
    assert model.cuda_graph_replays == 4


def test_replay_of_a_key_split_attention_is_bitwise_eager(gpu_ready):
    # A causal bf16 encoder whose attention takes the key-split schedule
    # (B=1, S=4096, H=4, head_dim 64): under capture its workspace comes from
    # the graph pool and its counter block is cleared inside the graph, so
    # every replay - with eager split launches on the same stream in
    # between, which reuse the stream's own workspace - equals the eager twin.
    from transformer_opt import _native

    cfg = TransformerConfig(1, 4096, 256, 4, 512, 2, True)
    assert _native.load().ttk_attention_workspace_size(1, 1, 4096, 4, 64, 1) > 0
    model, eager = twin(cfg, torch.bfloat16, seed=4)
    with torch.inference_mode():
        for step in range(3):
            x = sample(cfg, torch.bfloat16, seed=30 + step)
            out = model(x)
            torch.cuda.synchronize()
            reference = eager(x)
            torch.cuda.synchronize()
            assert torch.equal(out, reference), step
    assert model.cuda_graph_replays == 3
    assert model._inference_graph is not None
