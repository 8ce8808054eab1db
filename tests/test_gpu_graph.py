"""hipGraph replay of the encoder (reference tests/test_cuda_graph_inference.py).

Every replayed output is compared BITWISE with an eager forward of an
identical model, with eager work and synchronisations between replays, so a
graph node that misbehaves on a later replay (for example a recorded memset)
is caught.
"""

from __future__ import annotations

import copy

import pytest
import torch

from oracle.model import TransformerConfig

pytestmark = pytest.mark.gpu


def make_model(**kwargs):
    from transformer_opt.submission import UserOptimizedTransformer

    torch.manual_seed(0)
    return UserOptimizedTransformer(TransformerConfig(1, 128, 128, 4, 128, 4, True), **kwargs).eval()


def pair():
    model = make_model().cuda()
    eager = make_model(execution_mode="eager").cuda()
    eager.load_state_dict(model.state_dict(), strict=True)
    return model, eager


def test_replay_uses_new_inputs_and_masks_and_does_not_alias_outputs(gpu_ready):
    model, eager = pair()
    with torch.inference_mode():
        x = torch.randn(1, 128, 128, device="cuda")
        mask = torch.ones(1, 128, device="cuda", dtype=torch.bool)
        first = model(x, mask)
        saved = first.clone()
        entry = model._inference_graph
        assert entry is not None
        for padding in (False, True, False):
            x.normal_()
            if padding:
                mask[:, 80:] = False
            actual = model(x, mask)
            torch.cuda.synchronize()
            assert torch.equal(actual, eager(x, mask))
            assert model._inference_graph is entry
            assert torch.equal(first, saved)
            assert actual.data_ptr() != first.data_ptr()
        assert model.cuda_graph_replays == 4
        assert model.attention_backend_counts == {"hip": 16}
        assert model.fused_residual_layer_norm_calls == 32
        no_mask = model(x)
        assert torch.equal(no_mask, eager(x))
        assert model._inference_graph is not entry


def test_replay_recaptures_after_parameter_update_state_load_and_epsilon_change(gpu_ready):
    model, eager = pair()
    x = torch.randn(1, 128, 128, device="cuda")
    with torch.inference_mode():
        model(x)
        entry = model._inference_graph
        model.final_norm.bias.add_(0.125)
        eager.final_norm.bias.add_(0.125)
        assert torch.equal(model(x), eager(x))
        assert model._inference_graph is not entry
        entry = model._inference_graph
        model.layers[0].attention.q_proj.weight.add_(0.01)
        eager.layers[0].attention.q_proj.weight.add_(0.01)
        assert torch.equal(model(x), eager(x))
        assert model._inference_graph is not entry
        entry = model._inference_graph
        model.load_state_dict(eager.state_dict(), strict=True)
        assert torch.equal(model(x), eager(x))
        assert model._inference_graph is not entry
        entry = model._inference_graph
        model.final_norm.eps = eager.final_norm.eps = 0.02
        assert torch.equal(model(x), eager(x))
        assert model._inference_graph is not entry
        with torch.inference_mode(False):
            cloned = copy.deepcopy(model)
        assert cloned._inference_graph is None
        assert torch.equal(cloned(x), eager(x))
        model.clear_cuda_graph()
        assert model._inference_graph is None
        model(x)
        model.half()
        assert model._inference_graph is None
        assert model._packed_qkv_cache == {}


def test_replay_keeps_separate_caller_streams_ordered(gpu_ready):
    model, eager = pair()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    with torch.inference_mode():
        inputs = [torch.randn(1, 128, 128, device="cuda") for _ in streams]
        model(inputs[0])
        outputs = []
        for stream, x in zip(streams, inputs):
            stream.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(stream):
                outputs.append(model(x))
        for stream in streams:
            torch.cuda.current_stream().wait_stream(stream)
        for x, actual in zip(inputs, outputs):
            assert torch.equal(actual, eager(x))


def test_replay_recaptures_when_inference_context_changes(gpu_ready):
    model, eager = pair()
    x = torch.randn(1, 128, 128, device="cuda")
    with torch.inference_mode():
        model(x)
        first_entry = model._inference_graph
    with torch.no_grad():
        actual = model(x)
        assert torch.equal(actual, eager(x))
        assert not actual.is_inference()
        assert model._inference_graph is not first_entry
        second_entry = model._inference_graph
    with torch.inference_mode():
        actual = model(x)
        assert torch.equal(actual, eager(x))
        assert actual.is_inference()
        assert model._inference_graph is not second_entry


def test_replay_recaptures_after_attention_configuration_change(gpu_ready):
    model, eager = pair()
    x = torch.randn(1, 128, 128, device="cuda")
    with torch.inference_mode():
        model(x)
        entry = model._inference_graph
        model.layers[0].attention.scale *= 2
        eager.layers[0].attention.scale *= 2
        assert torch.equal(model(x), eager(x))
        assert model._inference_graph is not entry


def test_training_gradients_hooks_and_autocast_bypass_capture(gpu_ready):
    model = make_model().cuda()
    x = torch.randn(1, 128, 128, device="cuda")
    assert not model._can_replay_cuda_graph(x, None)  # gradients enabled
    with torch.inference_mode():
        assert model._can_replay_cuda_graph(x, None)
        assert not model._can_replay_cuda_graph(x.half(), None)  # dtype differs from the model's
        assert not model._can_replay_cuda_graph(x.double(), None)
        assert not model._can_replay_cuda_graph(x.transpose(1, 2), None)
        with torch.autocast("cuda"):
            assert not model._can_replay_cuda_graph(x, None)
        calls = []
        handle = model.layers[0].norm1.register_forward_hook(lambda *args: calls.append(1))
        assert not model._can_replay_cuda_graph(x, None)
        handle.remove()
        model.train()
        assert not model._can_replay_cuda_graph(x, None)
        model.eval()


def test_other_shapes_and_dtypes_replay_bitwise(gpu_ready):
    from transformer_opt.submission import UserOptimizedTransformer

    for dtype, cfg in ((torch.bfloat16, TransformerConfig(2, 200, 256, 4, 512, 2, False)),
                       (torch.float32, TransformerConfig(3, 64, 512, 8, 1024, 2, True))):
        torch.manual_seed(1)
        model = UserOptimizedTransformer(cfg).to("cuda", dtype).eval()
        eager = UserOptimizedTransformer(cfg, execution_mode="eager").to("cuda", dtype).eval()
        eager.load_state_dict(model.state_dict())
        with torch.inference_mode():
            for step in range(3):
                x = torch.randn(cfg.batch_size, cfg.seq_len, cfg.d_model, device="cuda").to(dtype)
                out = model(x)
                torch.cuda.synchronize()
                assert torch.equal(out, eager(x)), (dtype, step)
        assert model.cuda_graph_replays == 3


def test_alternating_shapes_replay_without_recapture_and_evict_lru(gpu_ready):
    # Up to max_cuda_graphs captures live side by side, one per input geometry;
    # the least recently used is evicted; a parameter change drops them all.
    model = make_model(max_cuda_graphs=2).cuda()
    eager = make_model(execution_mode="eager").cuda()
    eager.load_state_dict(model.state_dict(), strict=True)
    shapes = [(1, 64, 128), (2, 48, 128), (3, 32, 128)]
    with torch.inference_mode():
        xs = [torch.randn(shape, device="cuda") for shape in shapes]
        model(xs[0])
        first = model._inference_graph
        model(xs[1])
        second = model._inference_graph
        assert second is not first
        for _ in range(2):
            out0 = model(xs[0])
            assert model._inference_graph is first
            out1 = model(xs[1])
            assert model._inference_graph is second
        assert torch.equal(out0, eager(xs[0])) and torch.equal(out1, eager(xs[1]))
        model(xs[2])  # evicts the least recently used capture (shape 0)
        assert len(model._inference_graphs) == 2
        model(xs[0])
        assert model._inference_graph is not first
        assert model.cuda_graph_replays == 8
        with torch.no_grad():
            model.layers[0].ffn_in.bias.add_(0.01)
        model(xs[1])
        assert len(model._inference_graphs) == 1 and model._inference_graph is not second
    with pytest.raises(ValueError, match="max_cuda_graphs"):
        make_model(max_cuda_graphs=0)
