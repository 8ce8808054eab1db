"""ttk_attention_fwd_noalloc: the allocation-free attention entry point.

It runs the same kernels as ttk_attention_fwd_ws, with the key-split
schedule's counters and partial states in the library's static device
scratch instead of a caller workspace.  Called through the C ABI on two
launches in a row - the second smaller - its output must equal the
workspace entry point's on the same inputs (same schedule, same arithmetic:
bitwise), be within the oracle's bound, and allocate nothing.
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

import pytest
import torch

from oracle.attention import kernel_rounding_attention

pytestmark = pytest.mark.gpu

REPO = Path(__file__).resolve().parent.parent


def _launch(entry, q, k, v, out, workspace=None):
    """Causal attention of q/k/v into ``out`` through one C ABI entry point."""
    from transformer_opt import _native
    from transformer_opt.kernels.attention import _DTYPE_CODE

    lib = _native.load()
    B, S, H, D = q.shape
    args = [q.data_ptr(), k.data_ptr(), v.data_ptr(), None, out.data_ptr(), _DTYPE_CODE[q.dtype],
            B, S, H, D, _native.strides3(q.stride()[:3]), _native.strides3(k.stride()[:3]),
            _native.strides3(v.stride()[:3]), None, _native.strides3(out.stride()[:3]),
            D ** -0.5, 1]
    stream = torch.cuda.current_stream().cuda_stream
    if entry == "ws":
        return lib.ttk_attention_fwd_ws(*args, workspace.data_ptr(), workspace.numel(), stream)
    if entry == "plain":
        return lib.ttk_attention_fwd(*args, stream)
    return lib.ttk_attention_fwd_noalloc(*args, stream)


def _inputs(shape, seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    return tuple(torch.randn(shape, generator=g).to(dtype) for _ in range(3))


def test_noalloc_matches_the_workspace_entry_point_on_two_calls(gpu_ready):
    from transformer_opt import _native

    lib = _native.load()
    # Both shapes take the key-split schedule; the second call is smaller and
    # finds the scratch as the first left it (counters back at zero).
    for shape, seed in (((1, 4096, 4, 64), 11), ((1, 2048, 2, 64), 12)):
        need = lib.ttk_attention_workspace_size(1, *shape, 1)
        assert 0 < need <= 32 << 20, need
        q, k, v = _inputs(shape, seed)
        qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
        workspace = torch.zeros(need, dtype=torch.uint8, device="cuda")
        expected = torch.empty_like(qd)
        got = torch.empty_like(qd)
        with torch.inference_mode():
            _native.check(_launch("ws", qd, kd, vd, expected, workspace), "attention_ws")
            torch.cuda.synchronize()
            allocated = torch.cuda.memory_allocated()
            torch.cuda.reset_peak_memory_stats()
            _native.check(_launch("noalloc", qd, kd, vd, got), "attention_noalloc")
            torch.cuda.synchronize()
            assert torch.cuda.memory_allocated() == allocated
            assert torch.cuda.max_memory_allocated() == allocated
        assert torch.equal(got, expected), shape
        reference = kernel_rounding_attention(q, k, v, None, True).float()
        err = (got.float().cpu() - reference).abs()
        assert bool(((err <= 2e-3) | (err <= 2e-2 * reference.abs())).all()), shape


def test_noalloc_without_split_and_beyond_the_scratch_limit(gpu_ready):
    from transformer_opt import _native

    lib = _native.load()
    # A launch with no key-split schedule needs no scratch: it equals
    # ttk_attention_fwd bitwise.
    shape = (2, 300, 3, 64)
    assert lib.ttk_attention_workspace_size(1, *shape, 1) == 0
    q, k, v = (t.cuda() for t in _inputs(shape, 13))
    got, plain = torch.empty_like(q), torch.empty_like(q)
    with torch.inference_mode():
        _native.check(_launch("noalloc", q, k, v, got), "attention_noalloc")
        _native.check(_launch("plain", q, k, v, plain), "attention")
    assert torch.equal(got, plain)
    # A launch whose split state exceeds the static 32 MiB is rejected before
    # anything is launched.
    shape = (1, 4096, 4, 128)
    assert lib.ttk_attention_workspace_size(1, *shape, 1) > 32 << 20
    q, k, v = (t.cuda() for t in _inputs(shape, 14))
    out = torch.empty_like(q)
    with torch.inference_mode():
        status = _launch("noalloc", q, k, v, out)
    assert status == _native.TTK_EUNSUPPORTED
    assert "static maximum" in _native.last_error()


def test_noalloc_on_shapes_whose_split_state_grows(gpu_ready):
    # The reverse order of the test above: each call needs more split slots
    # and more partial state than the previous one, so it finds the previous
    # call's partial states in the scratch.  The counter block leads the
    # scratch at a fixed size, so the states never land on counters.  No
    # device memory is allocated: torch's allocator and the device's free
    # bytes are unchanged once the scratch and the kernels are loaded.
    from transformer_opt import _native

    lib = _native.load()
    shapes = [((1, 2048, 2, 64), 21), ((1, 3072, 4, 64), 22), ((1, 4096, 4, 64), 23)]
    for shape, seed in shapes:
        need = lib.ttk_attention_workspace_size(1, *shape, 1)
        assert 0 < need <= 32 << 20, need
        q, k, v = (t.cuda() for t in _inputs(shape, seed))
        workspace = torch.zeros(need, dtype=torch.uint8, device="cuda")
        expected, got = torch.empty_like(q), torch.empty_like(q)
        with torch.inference_mode():
            _native.check(_launch("ws", q, k, v, expected, workspace), "attention_ws")
            _native.check(_launch("noalloc", q, k, v, got), "attention_noalloc")  # warm
            torch.cuda.synchronize()
            allocated = torch.cuda.memory_allocated()
            free_before = torch.cuda.mem_get_info()[0]
            _native.check(_launch("noalloc", q, k, v, got), "attention_noalloc")
            torch.cuda.synchronize()
            assert torch.cuda.mem_get_info()[0] == free_before
            assert torch.cuda.memory_allocated() == allocated
        assert torch.equal(got, expected), shape


def _capture_child() -> int:
    """Run in a fresh process: the first ttk_attention_fwd_noalloc call of the
    process (so the scratch address is looked up there) happens inside a
    hipGraph capture; every replay must equal the eager workspace launch."""
    from transformer_opt import _native

    shape = (1, 4096, 4, 64)
    lib = _native.load()
    need = lib.ttk_attention_workspace_size(1, *shape, 1)
    assert need > 0
    q, k, v = (t.cuda() for t in _inputs(shape, 31))
    out = torch.empty_like(q)
    expected = torch.empty_like(q)
    workspace = torch.zeros(need, dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.inference_mode():
        with torch.cuda.graph(graph):
            status = _launch("noalloc", q, k, v, out)
        _native.check(status, "attention_noalloc under capture")
        _native.check(_launch("ws", q, k, v, expected, workspace), "attention_ws")
        for replay in range(3):
            out.zero_()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, expected), f"replay {replay}"
            # Eager work on the stream between replays: a split launch of
            # another shape through the same scratch.
            other = tuple(t.cuda() for t in _inputs((1, 2048, 2, 64), 32 + replay))
            tmp = torch.empty_like(other[0])
            _native.check(_launch("noalloc", *other, tmp), "attention_noalloc eager")
            torch.cuda.synchronize()
    print("noalloc capture child: OK", flush=True)
    return 0


def test_noalloc_first_call_inside_a_graph_capture(gpu_ready):
    # A fresh process, so this really is the first call of the library's
    # allocation-free entry point (the scratch lookup runs under capture).
    env = dict(os.environ)
    env["PYTHONPATH"] = os.pathsep.join(
        [str(REPO), str(REPO / "triton-transformer-kernels_amd"), env.get("PYTHONPATH", "")])
    proc = subprocess.run([sys.executable, str(Path(__file__).resolve()), "--capture-child"],
                          cwd=str(REPO), env=env, capture_output=True, text=True, timeout=300)
    assert proc.returncode == 0, proc.stdout[-3000:] + proc.stderr[-3000:]
    assert "noalloc capture child: OK" in proc.stdout


if __name__ == "__main__":
    if sys.argv[1:] == ["--capture-child"]:
        raise SystemExit(_capture_child())
