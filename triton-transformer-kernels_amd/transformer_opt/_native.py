"""ctypes binding of libttk_hip.so (the C ABI declared in include/ttk_hip.h).

The library is built in-tree by ``triton-transformer-kernels_amd/build.py``
into ``triton-transformer-kernels_amd/lib/libttk_hip.so``.  Nothing here
builds it: a missing library is a hard error, never a fallback.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path
from typing import Optional

LIB_PATH = Path(__file__).resolve().parent.parent / "lib" / "libttk_hip.so"
ENV_LIB = "TTK_HIP_LIBRARY"

TTK_OK = 0
TTK_EINVAL = 1
TTK_EUNSUPPORTED = 2
TTK_ELAUNCH = 3

TTK_F32 = 0
TTK_BF16 = 1
TTK_F16 = 2

TTK_ACT_NONE = 0
TTK_ACT_GELU = 1

# Exported symbols (kept in the same order as include/ttk_hip.h).
EXPORTED_SYMBOLS = (
    "ttk_abi_version",
    "ttk_last_error",
    "ttk_attention_fwd",
    "ttk_attention_workspace_size",
    "ttk_attention_fwd_ws",
    "ttk_attention_fwd_noalloc",
    "ttk_residual_layernorm_fwd",
    "ttk_gelu_fwd",
    "ttk_linear_fwd",
    "ttk_linear_residual_ln_workspace_size",
    "ttk_linear_pack_weight",
    "ttk_linear_residual_ln_fwd",
)
ABI_VERSION = 9
# TTK_ATTENTION_WS_COUNTER_BYTES: the zero-initialised counter block that
# leads every attention workspace, the same for every launch shape.
ATTENTION_WS_COUNTER_BYTES = 16384
# TTK_LINEAR_LN_WS_COUNTER_BYTES: the counter block that leads every
# linear + residual + LayerNorm workspace, the same for every M.
LINEAR_LN_WS_COUNTER_BYTES = 65536

_lock = threading.Lock()
_lib: Optional[ctypes.CDLL] = None
_load_error: Optional[BaseException] = None

_i64 = ctypes.c_int64
_i64p = ctypes.POINTER(ctypes.c_int64)
_vp = ctypes.c_void_p


def library_path() -> Path:
    override = os.environ.get(ENV_LIB)
    return Path(override) if override else LIB_PATH


def _configure(lib: ctypes.CDLL) -> None:
    lib.ttk_abi_version.restype = ctypes.c_int
    lib.ttk_abi_version.argtypes = []
    lib.ttk_last_error.restype = ctypes.c_char_p
    lib.ttk_last_error.argtypes = []
    lib.ttk_attention_fwd.restype = ctypes.c_int
    lib.ttk_attention_fwd.argtypes = [
        _vp, _vp, _vp, _vp, _vp, ctypes.c_int,
        _i64, _i64, _i64, _i64,
        _i64p, _i64p, _i64p, _i64p, _i64p,
        ctypes.c_float, ctypes.c_int, _vp,
    ]
    lib.ttk_attention_workspace_size.restype = ctypes.c_size_t
    lib.ttk_attention_workspace_size.argtypes = [ctypes.c_int, _i64, _i64, _i64, _i64, ctypes.c_int]
    lib.ttk_attention_fwd_ws.restype = ctypes.c_int
    lib.ttk_attention_fwd_ws.argtypes = [
        _vp, _vp, _vp, _vp, _vp, ctypes.c_int,
        _i64, _i64, _i64, _i64,
        _i64p, _i64p, _i64p, _i64p, _i64p,
        ctypes.c_float, ctypes.c_int, _vp, ctypes.c_size_t, _vp,
    ]
    lib.ttk_attention_fwd_noalloc.restype = ctypes.c_int
    lib.ttk_attention_fwd_noalloc.argtypes = lib.ttk_attention_fwd.argtypes
    lib.ttk_residual_layernorm_fwd.restype = ctypes.c_int
    lib.ttk_residual_layernorm_fwd.argtypes = [
        _vp, _vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_int,
        _i64, _i64, ctypes.c_float, ctypes.c_int, ctypes.c_int, _vp,
    ]
    lib.ttk_gelu_fwd.restype = ctypes.c_int
    lib.ttk_gelu_fwd.argtypes = [_vp, _vp, ctypes.c_int, _i64, _vp]
    lib.ttk_linear_fwd.restype = ctypes.c_int
    lib.ttk_linear_fwd.argtypes = [_vp, _vp, _vp, _vp, ctypes.c_int, _i64, _i64, _i64, _i64, _i64,
                                   _i64, ctypes.c_int, _vp]
    lib.ttk_linear_residual_ln_workspace_size.restype = _i64
    lib.ttk_linear_residual_ln_workspace_size.argtypes = [_i64]
    lib.ttk_linear_pack_weight.restype = ctypes.c_int
    lib.ttk_linear_pack_weight.argtypes = [_vp, _vp, ctypes.c_int, _i64, _i64, _i64, _vp]
    lib.ttk_linear_residual_ln_fwd.restype = ctypes.c_int
    lib.ttk_linear_residual_ln_fwd.argtypes = [
        _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, ctypes.c_int,
        _i64, _i64, _i64, _i64, _i64, _i64, _i64, ctypes.c_float, ctypes.c_int, _vp,
    ]


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raise RuntimeError if it is absent."""
    global _lib, _load_error
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = library_path()
        if not path.exists():
            _load_error = FileNotFoundError(str(path))
            raise RuntimeError(
                f"HIP kernel library not found at {path}; build it with "
                "`python triton-transformer-kernels_amd/build.py` (or __graft_entry__.build())"
            )
        try:
            lib = ctypes.CDLL(str(path))
        except OSError as exc:
            _load_error = exc
            raise RuntimeError(f"failed to load HIP kernel library {path}: {exc}") from exc
        _configure(lib)
        version = lib.ttk_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"{path} has ABI version {version}, expected {ABI_VERSION}")
        _lib = lib
        return lib


def available() -> bool:
    try:
        load()
        return True
    except RuntimeError:
        return False


def last_error() -> str:
    return load().ttk_last_error().decode("utf-8", "replace")


def check(status: int, what: str) -> None:
    """Translate a ttk_status into the reference's exception types."""
    if status == TTK_OK:
        return
    message = last_error() or f"status {status}"
    if status in (TTK_EINVAL, TTK_EUNSUPPORTED):
        raise ValueError(f"{what}: {message}")
    raise RuntimeError(f"{what}: {message}")


def strides3(values) -> ctypes.Array:
    arr = (ctypes.c_int64 * 3)(*values)
    return arr


def strides2(values) -> ctypes.Array:
    return (ctypes.c_int64 * 2)(*values)
