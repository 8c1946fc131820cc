"""ctypes loader for ``libzmlx_amd.so`` (the C ABI declared in
``include/zmlx_amd.h``).

The library is located at ``$ZMOE_LIB`` or ``zmlx_amd/_lib/libzmlx_amd.so``
(built by ``python -m zmlx_amd.build``).  There is no fallback: every op of
this package raises :class:`NativeLibraryMissing` when the library is absent.
"""

from __future__ import annotations

import ctypes
import os
import re
import threading
from pathlib import Path

ZMOE_OK = 0
ZMOE_EINVAL_SHAPE = -1
ZMOE_EINVAL_DTYPE = -2
ZMOE_EUNSUPPORTED = -3
ZMOE_EHIP = -4

DT_BF16 = 0
DT_F32 = 2

Q_AFFINE = 0
Q_MXFP4 = 1

COMBINE_NATIVE = 0
COMBINE_FP32 = 1
COMBINE_FP32_NO_FMA = 2
COMBINE_EXACT = 3
COMBINE_FLOAT = 4
COMBINE_NO_FMA = 5

ROUTER_SOFTMAX_PROBS = 0
ROUTER_TOPK_LOGITS = 1
ROUTER_SIGMOID_GROUPED = 2

LAYER_FORCE_MULTI = 1
LAYER_TRACE = 2

_PKG = Path(__file__).resolve().parent
HEADER = _PKG.parent / "include" / "zmlx_amd.h"
DEFAULT_LIB = _PKG / "_lib" / "libzmlx_amd.so"


class NativeLibraryMissing(RuntimeError):
    """The HIP library is not built / not loadable."""


class ZmoeError(RuntimeError):
    """A HIP-level failure reported by the library."""


c_void_p = ctypes.c_void_p
c_int = ctypes.c_int
c_i64 = ctypes.c_int64
c_float = ctypes.c_float
c_size_t = ctypes.c_size_t


class LayerDesc(ctypes.Structure):
    """Mirror of ``zmoe_layer_desc`` (include/zmlx_amd.h)."""

    _fields_ = [
        ("hidden", c_int),
        ("n_experts", c_int),
        ("top_k", c_int),
        ("inter", c_int),
        ("group_size", c_int),
        ("bits", c_int),
        ("quant_mode", c_int),
        ("router_kind", c_int),
        ("norm_topk_prob", c_int),
        ("n_group", c_int),
        ("topk_group", c_int),
        ("routed_scaling_factor", c_float),
        ("combine_mode", c_int),
        ("router_w", c_void_p),
        ("router_bias", c_void_p),
        ("gate_w", c_void_p), ("gate_s", c_void_p), ("gate_b", c_void_p),
        ("up_w", c_void_p), ("up_s", c_void_p), ("up_b", c_void_p),
        ("down_w", c_void_p), ("down_s", c_void_p), ("down_b", c_void_p),
        ("shared_inter", c_int),
        ("sh_gate_w", c_void_p), ("sh_gate_s", c_void_p), ("sh_gate_b", c_void_p),
        ("sh_up_w", c_void_p), ("sh_up_s", c_void_p), ("sh_up_b", c_void_p),
        ("sh_down_w", c_void_p), ("sh_down_s", c_void_p), ("sh_down_b", c_void_p),
        ("flags", c_int),
        ("error_flag_host", c_void_p),
        ("spin_limit", c_int),
    ]


_SIGNATURES = {
    "zmoe_version": (ctypes.c_char_p, []),
    "zmoe_last_error": (ctypes.c_char_p, []),
    "zmoe_host_flags_alloc": (c_void_p, [c_int]),
    "zmoe_host_flags_free": (None, [c_void_p]),
    "zmoe_gather_qmm_swiglu": (
        c_int,
        [c_void_p, c_void_p, c_i64, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
         c_void_p, c_void_p, c_i64, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_void_p],
    ),
    "zmoe_gather_qmm": (
        c_int,
        [c_void_p, c_void_p, c_i64, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_i64,
         c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_void_p],
    ),
    "zmoe_grouped_gather_qmm_workspace_size": (c_size_t, [c_i64, c_int, c_int, c_int, c_int]),
    "zmoe_grouped_gather_qmm": (
        c_int,
        [c_void_p, c_void_p, c_i64, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
         c_i64, c_int, c_int, c_int, c_int, c_int, c_int, c_void_p, c_size_t, c_void_p],
    ),
    "zmoe_dense_logits": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_void_p]),
    "zmoe_router_softmax_topk": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_void_p]),
    "zmoe_topk_gating_softmax": (
        c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_int, c_void_p, c_void_p]),
    "zmoe_deepseek_router_topk_sigmoid": (
        c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_float, c_void_p, c_void_p]),
    "zmoe_moe_combine": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p]),
    "zmoe_weighted_accumulate": (
        c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_i64, c_int, c_int, c_int, c_int, c_void_p]),
    "zmoe_swiglu2": (c_int, [c_void_p, c_void_p, c_void_p, c_i64, c_int, c_void_p]),
    "zmoe_swiglu2_backward": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_i64, c_int, c_void_p, c_void_p]),
    "zmoe_moe_dispatch": (c_int, [c_void_p, c_void_p, c_i64, c_int, c_int, c_int, c_void_p]),
    "zmoe_moe_layer_workspace_size": (c_size_t, [ctypes.POINTER(LayerDesc), c_int]),
    "zmoe_moe_layer_trace_info": (
        c_size_t, [ctypes.POINTER(LayerDesc), c_int, ctypes.POINTER(c_int), ctypes.POINTER(c_int)]),
    "zmoe_moe_layer": (
        c_int, [c_void_p, ctypes.POINTER(LayerDesc), c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p,
                c_size_t]),
    "zmoe_moe_layer_noalloc": (
        c_int, [c_void_p, ctypes.POINTER(LayerDesc), c_void_p, c_int, c_void_p, c_void_p, c_void_p]),
    "zmoe_moe_layer_noalloc_max_bytes": (c_size_t, []),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def library_path() -> Path:
    env = os.environ.get("ZMOE_LIB")
    return Path(env) if env else DEFAULT_LIB


def lib() -> ctypes.CDLL:
    """Load (once) and return the library; raises NativeLibraryMissing."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            path = library_path()
            if not path.exists():
                raise NativeLibraryMissing(
                    f"zmlx_amd HIP library not found at {path}; build it with `python -m zmlx_amd.build`"
                )
            try:
                handle = ctypes.CDLL(str(path))
            except OSError as e:  # pragma: no cover - depends on the host
                raise NativeLibraryMissing(f"cannot load {path}: {e}") from e
            for name, (res, args) in _SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            _lib = handle
    return _lib


def header_functions() -> list[str]:
    """Names of every function the public header declares."""
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(zmoe_[a-z_0-9]+)\s*\(", text, re.M)))


def check(rc: int, op: str) -> None:
    """Raise the reference's exception type for a non-zero status."""
    if rc == ZMOE_OK:
        return
    msg = lib().zmoe_last_error().decode() or f"{op} failed with status {rc}"
    if rc in (ZMOE_EINVAL_SHAPE, ZMOE_EINVAL_DTYPE, ZMOE_EUNSUPPORTED):
        raise ValueError(msg)
    raise ZmoeError(msg)


def version() -> str:
    return lib().zmoe_version().decode()
