"""The C ABI library: it loads, exports every declared symbol, and rejects bad
arguments before touching the device (so these run without a GPU)."""

from __future__ import annotations

import ctypes
import re
import subprocess
import sys
import threading
from pathlib import Path

import pytest

from transformer_opt import _native

REPO = Path(__file__).resolve().parent.parent
HEADER = REPO / "include" / "ttk_hip.h"


def declared_functions() -> list:
    text = HEADER.read_text()
    return re.findall(r"^\s*(?:const\s+)?[a-z0-9_]+\*?\s+\*?(ttk_[a-z0-9_]+)\s*\(", text, re.MULTILINE)


def test_header_declares_the_exported_symbols():
    assert set(declared_functions()) == set(_native.EXPORTED_SYMBOLS)


def test_library_loads_and_exports_every_declared_symbol():
    lib = _native.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
    nm = subprocess.run(["nm", "-D", "--defined-only", str(_native.library_path())],
                        capture_output=True, text=True, check=True).stdout
    for name in declared_functions():
        assert re.search(rf"\bT {name}$", nm, re.MULTILINE), name


def test_abi_version_matches_header():
    version = int(re.search(r"#define TTK_ABI_VERSION (\d+)", HEADER.read_text()).group(1))
    assert _native.load().ttk_abi_version() == version == _native.ABI_VERSION


def _attention(lib, **over):
    s3 = (ctypes.c_int64 * 3)(16 * 64, 64, 64 * 0 + 64)
    args = dict(q=16, k=32, v=48, mask=None, out=64, dtype=0, B=1, S=16, H=1, D=64,
                qs=s3, ks=s3, vs=s3, ms=None, os=s3, scale=0.125, causal=0, stream=None)
    args.update(over)
    return lib.ttk_attention_fwd(args["q"], args["k"], args["v"], args["mask"], args["out"], args["dtype"],
                                 args["B"], args["S"], args["H"], args["D"], args["qs"], args["ks"],
                                 args["vs"], args["ms"], args["os"], args["scale"], args["causal"],
                                 args["stream"])


def test_attention_argument_errors_are_reported_without_launching():
    lib = _native.load()
    assert _attention(lib, D=48) == _native.TTK_EUNSUPPORTED
    assert "head_dim=48" in _native.last_error()
    assert _attention(lib, S=0) == _native.TTK_EINVAL
    assert "must be positive" in _native.last_error()
    assert _attention(lib, dtype=7) == _native.TTK_EUNSUPPORTED
    assert _attention(lib, qs=None) == _native.TTK_EINVAL
    assert _attention(lib, q=None) == _native.TTK_EINVAL
    assert _attention(lib, q=17) == _native.TTK_EUNSUPPORTED
    assert "16-byte aligned" in _native.last_error()
    bad = (ctypes.c_int64 * 3)(16 * 64, 63, 64)
    assert _attention(lib, ks=bad) == _native.TTK_EUNSUPPORTED
    assert "stride" in _native.last_error()
    assert _attention(lib, mask=16, ms=None) == _native.TTK_EINVAL
    # An empty batch is a valid no-op (nothing is launched).
    assert _attention(lib, B=0) == _native.TTK_OK
    assert _native.last_error() == ""


def test_layernorm_argument_errors_are_reported_without_launching():
    lib = _native.load()
    f = lib.ttk_residual_layernorm_fwd
    assert f(16, 16, 16, None, None, 16, 16, 0, 4, 0, 1e-5, 0, 0, None) == _native.TTK_EINVAL
    assert f(16, 16, 16, None, None, 16, 16, 0, 4, 70000, 1e-5, 0, 0, None) == _native.TTK_EUNSUPPORTED
    assert "65536" in _native.last_error()
    assert f(16, 16, 16, None, None, 16, 16, 0, 4, 128, 1e-5, 1, 0, None) == _native.TTK_EINVAL
    assert "requires valid_token_mask" in _native.last_error()
    assert f(None, 16, 16, None, None, 16, 16, 0, 4, 128, 1e-5, 0, 0, None) == _native.TTK_EINVAL
    assert f(16, 16, 16, None, None, 16, 16, 9, 4, 128, 1e-5, 0, 0, None) == _native.TTK_EUNSUPPORTED
    assert f(16, 16, 16, None, None, 16, 16, 0, 0, 128, 1e-5, 0, 0, None) == _native.TTK_OK


def test_launch_grid_limits_are_unsupported_not_launch_failures():
    # HIP refuses grids above 2^32 - 1 work-items (16777215 workgroups of 256):
    # sizes the kernels cannot launch come back as TTK_EUNSUPPORTED before any
    # HIP call, not as a failed launch.
    lib = _native.load()
    limit = 16777215
    # attention: one workgroup per (batch, head, 128-query tile)
    assert _attention(lib, B=limit + 1, H=1, S=16) == _native.TTK_EUNSUPPORTED
    assert "launch limit" in _native.last_error()
    assert _attention(lib, B=1 << 17, H=128, S=16) == _native.TTK_EUNSUPPORTED  # 2^24 groups
    assert _attention(lib, B=1 << 10, H=1 << 7, S=129 * 128) == _native.TTK_EUNSUPPORTED
    assert _attention(lib, B=1 << 40, H=1 << 40, S=16) == _native.TTK_EUNSUPPORTED  # no overflow
    f = lib.ttk_residual_layernorm_fwd
    # (x, u, w, b, valid, r_out, y_out, dtype, rows, N, eps, zr, zn, stream)
    # width 7 (fp32) takes the one-workgroup-per-row path
    assert f(16, 16, 16, None, None, 16, 16, 0, limit + 1, 7, 1e-5, 0, 0, None) == _native.TTK_EUNSUPPORTED
    assert "launch limit" in _native.last_error()
    # width 128 fp32: eight rows per wavefront, 32 rows per workgroup
    assert f(16, 16, 16, None, None, 16, 16, 0, 32 * limit + 1, 128, 1e-5, 0, 0, None) == \
        _native.TTK_EUNSUPPORTED
    assert f(16, 16, 16, None, None, 16, 16, 0, 1 << 62, 128, 1e-5, 0, 0, None) == _native.TTK_EUNSUPPORTED


def test_last_error_is_thread_local():
    lib = _native.load()
    assert _attention(lib, D=48) == _native.TTK_EUNSUPPORTED
    seen = {}

    def other():
        seen["msg"] = _native.last_error()

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert seen["msg"] == ""
    assert "head_dim" in _native.last_error()


def test_check_maps_status_to_reference_exception_types():
    lib = _native.load()
    _attention(lib, D=48)
    with pytest.raises(ValueError, match="head_dim"):
        _native.check(_native.TTK_EUNSUPPORTED, "HIP attention")
    with pytest.raises(RuntimeError):
        _native.check(_native.TTK_ELAUNCH, "HIP attention")
    _native.check(_native.TTK_OK, "noop")


def test_missing_library_fails_loudly_in_a_fresh_process(tmp_path):
    code = (
        "import sys; sys.path.insert(0, %r); sys.path.insert(0, %r)\n"
        "import torch\n"
        "from transformer_opt import _native, attention_forward\n"
        "try:\n    _native.load()\nexcept RuntimeError as e:\n    print('LOAD', 'not found' in str(e))\n"
        "q = torch.zeros(1, 4, 1, 8)\n"
        "try:\n    attention_forward(q, q, q, backend='hip')\nexcept RuntimeError as e:\n    print('FWD', 'unavailable' in str(e))\n"
    ) % (str(REPO), str(REPO / "triton-transformer-kernels_amd"))
    env = {"TTK_HIP_LIBRARY": str(tmp_path / "missing.so"), "PATH": "/usr/bin:/bin",
           "HIP_VISIBLE_DEVICES": "", "CUDA_VISIBLE_DEVICES": ""}
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env, timeout=300)
    assert "LOAD True" in out.stdout, out.stderr
    assert "FWD True" in out.stdout, out.stderr


def test_gelu_argument_errors_are_reported_without_launching():
    lib = _native.load()
    f = lib.ttk_gelu_fwd
    # (x, y, dtype, n, stream)
    assert f(16, 16, 7, 8, None) == _native.TTK_EUNSUPPORTED
    assert "dtype" in _native.last_error()
    assert f(16, 16, _native.TTK_BF16, -1, None) == _native.TTK_EINVAL
    # One element per work-item on an unaligned buffer: n stops at 2^32 - 256.
    assert f(16, 16, _native.TTK_BF16, 4294967040 + 1, None) == _native.TTK_EUNSUPPORTED
    assert "launch limit" in _native.last_error()
    assert f(None, 16, _native.TTK_BF16, 8, None) == _native.TTK_EINVAL
    # y one element past x: overlapping but not in place.
    assert f(1024, 1026, _native.TTK_BF16, 8, None) == _native.TTK_EINVAL
    assert "overlap" in _native.last_error()
    assert f(1024 + 16, 1024, _native.TTK_F32, 8, None) == _native.TTK_EINVAL  # 32 bytes, 16 apart
    assert f(16, 16, _native.TTK_F32, 0, None) == _native.TTK_OK


def _linear(lib, **over):
    args = dict(x=1024, w=2048, b=None, y=4096, dtype=_native.TTK_BF16, M=64, N=256, K=256,
                ldx=256, ldw=256, ldy=256, act=_native.TTK_ACT_GELU, stream=None)
    args.update(over)
    return lib.ttk_linear_fwd(args["x"], args["w"], args["b"], args["y"], args["dtype"], args["M"],
                              args["N"], args["K"], args["ldx"], args["ldw"], args["ldy"], args["act"],
                              args["stream"])


def test_linear_argument_errors_are_reported_without_launching():
    # Pointers here are fake: every call below is rejected before any HIP call.
    lib = _native.load()
    assert _linear(lib, dtype=_native.TTK_F32) == _native.TTK_EUNSUPPORTED
    assert "not bf16 or fp16" in _native.last_error()
    assert _linear(lib, act=7) == _native.TTK_EINVAL
    assert _linear(lib, N=0) == _native.TTK_EINVAL
    assert _linear(lib, K=200, ldx=200, ldw=200) == _native.TTK_EUNSUPPORTED
    assert "multiple of 128" in _native.last_error()
    assert _linear(lib, K=128, ldx=128, ldw=128) == _native.TTK_EUNSUPPORTED
    assert _linear(lib, N=250, ldy=256) == _native.TTK_EUNSUPPORTED
    assert "multiple of 32" in _native.last_error()
    assert _linear(lib, x=1032) == _native.TTK_EUNSUPPORTED
    assert "16-byte aligned" in _native.last_error()
    assert _linear(lib, ldy=100) == _native.TTK_EUNSUPPORTED
    assert _linear(lib, b=2050) == _native.TTK_EUNSUPPORTED
    assert "4-byte aligned" in _native.last_error()
    assert _linear(lib, M=1 << 22, N=1024, ldy=1024) == _native.TTK_EUNSUPPORTED
    assert "2^31" in _native.last_error()
    assert _linear(lib, y=1024 + 512) == _native.TTK_EINVAL  # y inside x
    assert "overlaps" in _native.last_error()
    assert _linear(lib, x=None) == _native.TTK_EINVAL
    assert _linear(lib, M=0) == _native.TTK_OK  # nothing to launch


def _linear_ln(lib, **over):
    # 64 rows, K = 128: a at 1 MiB, packed W at 2 MiB, x / r / y 128 KiB apart.
    args = dict(a=1 << 20, wp=2 << 20, b=None, x=3 << 20, g=4 << 20, beta=None, r=5 << 20,
                y=6 << 20, ws=7 << 20, ws_bytes=65536 + 1024, dtype=_native.TTK_BF16, M=64, N=1024, K=128,
                lda=128, ldx=1024, ldr=1024, ldy=1024, eps=1e-5, polls=-1, stream=None)
    args.update(over)
    return lib.ttk_linear_residual_ln_fwd(
        args["a"], args["wp"], args["b"], args["x"], args["g"], args["beta"], args["r"], args["y"],
        args["ws"], args["ws_bytes"], args["dtype"], args["M"], args["N"], args["K"], args["lda"],
        args["ldx"], args["ldr"], args["ldy"], args["eps"], args["polls"], args["stream"])


def test_linear_residual_ln_argument_errors_are_reported_without_launching():
    lib = _native.load()
    size = lib.ttk_linear_residual_ln_workspace_size
    # A fixed counter block (the same bytes for every M) + 1 KB of statistics per 64 rows.
    block = _native.LINEAR_LN_WS_COUNTER_BYTES
    assert block == 65536
    assert size(0) == 0 and size(1) == block + 1024 and size(64 * 64) == block + 64 * 1024
    assert size(64 * 65) == block + 65 * 1024
    assert _linear_ln(lib, dtype=_native.TTK_F32) == _native.TTK_EUNSUPPORTED
    assert "not bf16 or fp16" in _native.last_error()
    assert _linear_ln(lib, N=512, ldx=512, ldr=512, ldy=512) == _native.TTK_EUNSUPPORTED
    assert "1024" in _native.last_error()
    assert _linear_ln(lib, K=192, lda=192) == _native.TTK_EUNSUPPORTED
    assert "multiple of 128" in _native.last_error()
    assert _linear_ln(lib, M=-1) == _native.TTK_EINVAL
    assert _linear_ln(lib, ws=None) == _native.TTK_EINVAL
    assert _linear_ln(lib, ws_bytes=4) == _native.TTK_EINVAL
    assert "workspace" in _native.last_error()
    assert _linear_ln(lib, g=(4 << 20) + 8) == _native.TTK_EUNSUPPORTED
    assert "16-byte aligned" in _native.last_error()
    assert _linear_ln(lib, b=(8 << 20) + 1) == _native.TTK_EUNSUPPORTED
    assert _linear_ln(lib, lda=100) == _native.TTK_EUNSUPPORTED
    assert _linear_ln(lib, M=1 << 20, ws_bytes=1 << 26) == _native.TTK_EUNSUPPORTED
    assert "2^31" in _native.last_error()
    assert _linear_ln(lib, y=(5 << 20) + 1024) == _native.TTK_EINVAL  # y inside r
    assert "overlap" in _native.last_error()
    assert _linear_ln(lib, r=3 << 20) == _native.TTK_EINVAL  # r on x
    assert _linear_ln(lib, y=7 << 20) == _native.TTK_EINVAL  # y on the workspace
    assert _linear_ln(lib, M=0) == _native.TTK_OK  # nothing to launch
    pack = lib.ttk_linear_pack_weight
    # (w, w_packed, dtype, N, K, ldw, stream)
    assert pack(1 << 20, 2 << 20, _native.TTK_F32, 64, 64, 64, None) == _native.TTK_EUNSUPPORTED
    assert pack(1 << 20, 2 << 20, _native.TTK_BF16, 40, 64, 64, None) == _native.TTK_EUNSUPPORTED
    assert pack(1 << 20, 2 << 20, _native.TTK_BF16, 64, 64, 60, None) == _native.TTK_EUNSUPPORTED
    assert pack(1 << 20, (1 << 20) + 4096, _native.TTK_BF16, 64, 64, 64, None) == _native.TTK_EINVAL
    assert pack(None, 2 << 20, _native.TTK_BF16, 64, 64, 64, None) == _native.TTK_EINVAL
