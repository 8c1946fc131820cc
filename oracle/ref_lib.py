"""ctypes wrapper of the C++ restatement (oracle/moe_ref.cpp).

TEST INFRASTRUCTURE ONLY (CPU baseline timing and oracle cross-checks)."""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "_build" / "libmoe_ref.so"
_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        _lib = ctypes.CDLL(str(LIB))
        _lib.oref_num_threads.restype = ctypes.c_int
        _lib.oref_set_threads.argtypes = [ctypes.c_int]
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def bf16_bits(a) -> np.ndarray:
    from oracle.moe_oracle import bf16_to_bits

    return np.ascontiguousarray(bf16_to_bits(np.asarray(a, np.float32)))


def moe_layer_qwen(x, wr, gate, up, down, *, k: int, group_size: int = 64, norm: bool = True, threads: int = 0):
    """x [B,H] float32 (bf16 values); wr [E,H]; gate/up/down (w u32, s, b)
    with bf16-valued float32 scales/biases.  Returns (out float32 [B,H],
    idx int32 [B,k])."""
    L = lib()
    if threads:
        L.oref_set_threads(int(threads))
    x16 = bf16_bits(x)
    B, H = x16.shape
    E = int(np.asarray(wr).shape[0])
    I = int(gate[0].shape[1])
    out = np.zeros((B, H), np.uint16)
    idx = np.zeros((B, k), np.int32)
    args = [_p(x16), B, H, E, k, I, group_size, int(norm), _p(bf16_bits(wr))]
    keep = []
    for w, s, b in (gate, up, down):
        w = np.ascontiguousarray(w, np.uint32)
        s16, b16 = bf16_bits(s), bf16_bits(b)
        keep += [w, s16, b16]
        args += [_p(w), _p(s16), _p(b16)]
    args += [_p(out), _p(idx)]
    L.oref_moe_layer_qwen(*args)
    from oracle.moe_oracle import bf16_from_bits

    return bf16_from_bits(out), idx


def moe_layer_qwen_bits(x16, wr16, gate, up, down, *, k: int, group_size: int = 64, norm: bool = True):
    """Same as moe_layer_qwen but every bf16 array is passed as raw uint16
    bits (no conversion cost) -- used by the CPU baseline timing."""
    L = lib()
    x16 = np.ascontiguousarray(x16, np.uint16)
    B, H = x16.shape
    E = int(wr16.shape[0])
    I = int(gate[0].shape[1])
    out = np.zeros((B, H), np.uint16)
    idx = np.zeros((B, k), np.int32)
    args = [_p(x16), B, H, E, k, I, group_size, int(norm), _p(np.ascontiguousarray(wr16, np.uint16))]
    for w, s, b in (gate, up, down):
        args += [_p(w), _p(s), _p(b)]
    args += [_p(out), _p(idx)]
    L.oref_moe_layer_qwen(*args)
    return out, idx
