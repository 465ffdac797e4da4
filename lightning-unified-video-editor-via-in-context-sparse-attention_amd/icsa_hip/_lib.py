"""ctypes binding of ``libicsa.so`` (declarations: include/icsa.h).

The library is loaded from this package's directory.  There is no fallback: when the
library is missing, :func:`lib` raises, and every GPU entry point of the package fails
loudly instead of computing anything another way.
"""
from __future__ import annotations

import ctypes
import os
import threading

# ICSA_LIB_PATH selects another build of the same library (e.g. a tuning variant)
_LIB_PATH = os.environ.get("ICSA_LIB_PATH") or os.path.join(
    os.path.dirname(os.path.abspath(__file__)), "libicsa.so")
_lock = threading.Lock()
_lib = None

BF16 = 0
F32 = 1

OK = 0
EINVAL = -1
EUNSUPPORTED = -2
EWORKSPACE = -3
EHIP = -4

# bytes of the static scratch of icsa_editing_sparse_attention_noalloc
NOALLOC_SCRATCH_BYTES = 256 << 20

# stage boundaries of icsa_editing_sparse_attention_ev
STAGES = ["start", "pool", "compressed", "select", "sparse", "flash"]

# workspace slots of icsa_editing_sparse_attention (enum icsa_ws_slot)
WS_SLOTS = ["QSUM", "KSUM", "VSUM", "VT", "QB", "KB", "VB", "LOGITS", "OUTC", "SHARP", "SRCSCORE",
            "SEL", "ORDER", "KVMAP", "KC32", "KC", "VCT", "L3", "VC", "COLP", "L3S", "RSTAT"]

# every symbol include/icsa.h declares
EXPORTS = [
    "icsa_editing_sizes", "icsa_editing_workspace_size", "icsa_editing_workspace_layout",
    "icsa_editing_sparse_attention", "icsa_editing_sparse_attention_ev",
    "icsa_editing_sparse_attention_noalloc",
    "icsa_sparse_piecewise_workspace_size",
    "icsa_sparse_piecewise_attn", "icsa_flash_attn_workspace_size", "icsa_flash_attn",
    "icsa_pool", "icsa_gather_kv", "icsa_wan_qk_workspace_size", "icsa_wan_qk_prologue",
    "icsa_editing_sparse_attention_presummed", "icsa_wan_ln_modulate", "icsa_last_error",
    "icsa_version", "icsa_sparse_piecewise_attn_fwd", "icsa_sparse_piecewise_attn_bwd_workspace_size",
    "icsa_sparse_piecewise_attn_bwd", "icsa_sparse_piecewise_attn_hosttopk",
]

_p = ctypes.c_void_p
_i = ctypes.c_int
_l = ctypes.c_int64
_d = ctypes.c_double
_f = ctypes.c_float

_SIGNATURES = {
    "icsa_editing_sizes": (_i, [_i, _i, _i, _i, _i, _d, _d, _d, _p]),
    "icsa_editing_workspace_size": (_l, [_i, _i, _i, _i, _i, _d, _d, _d, _i, _i, _i]),
    "icsa_editing_workspace_layout": (_l, [_i, _i, _i, _i, _i, _d, _d, _d, _i, _i, _i, _p]),
    "icsa_editing_sparse_attention": (_i, [
        _p, _i, _l, _l, _l,
        _p, _i, _l, _l, _l,
        _p, _i, _l, _l, _l,
        _i, _i, _i, _i, _i, _d, _d, _d,
        _p, _i, _l, _l, _l, _l, _f,
        _p, _i, _l, _l, _l,
        _p, _p, _p,
        _p, _l, _p]),
    "icsa_editing_sparse_attention_ev": (_i, [
        _p, _i, _l, _l, _l,
        _p, _i, _l, _l, _l,
        _p, _i, _l, _l, _l,
        _i, _i, _i, _i, _i, _d, _d, _d,
        _p, _i, _l, _l, _l, _l, _f,
        _p, _i, _l, _l, _l,
        _p, _p, _p,
        _p, _l, _p, _p]),
    "icsa_editing_sparse_attention_noalloc": (_i, [
        _p, _i, _l, _l, _l,
        _p, _i, _l, _l, _l,
        _p, _i, _l, _l, _l,
        _i, _i, _i, _i, _i, _d, _d, _d,
        _p, _i, _l, _l, _l, _l, _f,
        _p, _i, _l, _l, _l,
        _p, _p, _p,
        _p]),
    "icsa_sparse_piecewise_workspace_size": (_l, [_i, _i, _i, _i, _i, _d]),
    "icsa_sparse_piecewise_attn": (_i, [
        _p, _l, _l, _l,
        _p, _l, _l, _l,
        _p, _l, _l, _l,
        _i, _i, _i, _i, _i, _d,
        _p, _p,
        _p, _l, _l, _l,
        _p, _l, _p]),
    "icsa_sparse_piecewise_attn_hosttopk": (_i, [
        _p, _l, _l, _l,
        _p, _l, _l, _l,
        _p, _l, _l, _l,
        _i, _i, _i, _i, _i, _d, _i,
        _p, _p,
        _p, _l, _l, _l,
        _p, _l, _p]),
    "icsa_sparse_piecewise_attn_fwd": (_i, [
        _p, _l, _l, _l,
        _p, _l, _l, _l,
        _p, _l, _l, _l,
        _i, _i, _i, _i, _i, _d,
        _p, _p,
        _p, _l, _l, _l, _p,
        _p, _l, _p]),
    "icsa_sparse_piecewise_attn_bwd_workspace_size": (_l, [_i, _i, _i, _i, _i]),
    "icsa_sparse_piecewise_attn_bwd": (_i, [
        _p, _l, _l, _l,
        _p, _l, _l, _l,
        _p, _l, _l, _l,
        _p, _l, _l, _l,
        _p, _l, _l, _l,
        _p, _p,
        _i, _i, _i, _i, _i, _i,
        _p, _i, _l, _l, _l,
        _p, _i, _l, _l, _l,
        _p, _i, _l, _l, _l,
        _p, _l, _p]),
    "icsa_flash_attn_workspace_size": (_l, [_i, _i, _i, _i]),
    "icsa_flash_attn": (_i, [
        _p, _l, _l, _l,
        _p, _l, _l, _l,
        _p, _l, _l, _l,
        _i, _i, _i, _i, _i,
        _p, _i, _l, _l, _l,
        _p, _l, _p]),
    "icsa_pool": (_i, [
        _p, _i, _l, _l, _l,
        _p, _i, _l, _l, _l,
        _p, _i, _l, _l, _l,
        _i, _i, _i, _i, _p, _p, _p, _p, _p]),
    "icsa_gather_kv": (_i, [
        _p, _i, _l, _l, _l,
        _p, _i, _l, _l, _l,
        _i, _i, _i, _i, _i, _p, _i, _p, _p, _p]),
    "icsa_wan_qk_workspace_size": (_l, [_i, _i]),
    "icsa_wan_qk_prologue": (_i, [
        _p, _p, _i, _l, _l,
        _p, _p, _f,
        _p, _p, _i,
        _p, _i,
        _p, _i, _l, _l,
        _i, _i, _i, _i,
        _p, _p, _l, _l, _l,
        _p, _p, _p,
        _p, _l, _p]),
    "icsa_editing_sparse_attention_presummed": (_i, [
        _p, _i, _l, _l, _l,
        _p, _i, _l, _l, _l,
        _p, _i, _l, _l, _l,
        _i, _i, _i, _i, _i, _d, _d, _d,
        _p, _i, _l, _l, _l, _l, _f,
        _p, _i, _l, _l, _l,
        _p, _p, _p,
        _p, _l, _p, _p,
        _p, _p]),
    "icsa_wan_ln_modulate": (_i, [
        _p, _i, _l, _l,
        _p, _l, _l, _p, _l,
        _p, _l, _l,
        _p, _p,
        _p, _p, _l, _f,
        _i, _i, _i, _p, _l, _l, _p]),
    "icsa_last_error": (ctypes.c_char_p, []),
    "icsa_version": (_i, []),
}


def lib_path() -> str:
    return _LIB_PATH


def lib():
    """The loaded library (raises ``OSError`` when it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(_LIB_PATH):
                raise OSError(
                    f"libicsa.so not found at {_LIB_PATH}; build it with "
                    "`python -m icsa_hip.build` (hipcc, gfx950)")
            handle = ctypes.CDLL(_LIB_PATH)
            for name, (res, args) in _SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            _lib = handle
    return _lib


class IcsaError(RuntimeError):
    """A non-zero status returned by libicsa (message from icsa_last_error)."""

    def __init__(self, fn: str, code: int):
        msg = lib().icsa_last_error().decode("utf-8", "replace")
        super().__init__(f"{fn} failed with status {code}: {msg}")
        self.code = code


def check(fn: str, code: int) -> None:
    if code != OK:
        raise IcsaError(fn, code)
