"""MLX-format weight quantisers in torch (run on the GPU for large banks).

These build the packed layouts the kernels consume -- they play the role of
``mx.quantize`` for synthetic or converted weights and are not on the decode
path.  Layouts (MLX): uint32 words with element i of a word at bits 4*i;
affine: bf16 scales/biases per ``group_size``; mxfp4: e8m0 byte per 32.
"""

from __future__ import annotations

import torch

E2M1_MAGNITUDES = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0)


def _pack_nibbles(q: torch.Tensor) -> torch.Tensor:
    """int tensor [..., K] of 4-bit codes -> uint32 [..., K/8]."""
    q = q.to(torch.int64).reshape(*q.shape[:-1], q.shape[-1] // 8, 8)
    shifts = torch.arange(8, device=q.device, dtype=torch.int64) * 4
    packed = (q << shifts).sum(-1)  # disjoint bit fields: sum == or
    packed = packed - (packed >= 2**31).to(torch.int64) * 2**32  # two's-complement into int32 range
    return packed.to(torch.int32).view(torch.uint32)


def quantize_affine(w: torch.Tensor, group_size: int = 64, bits: int = 4):
    """Min/max affine quantisation -> (w_packed uint32, scales bf16, biases bf16).

    scale = bf16((max-min)/15), bias = bf16(min), q = clip(round((w-bias)/scale)).
    The same rule as the CPU oracle's fixture quantiser."""
    if bits != 4:
        raise ValueError("quantize_affine: only bits=4 is supported")
    w = w.to(torch.float32)
    K = w.shape[-1]
    if K % group_size:
        raise ValueError("quantize_affine: last dimension must be a multiple of group_size")
    g = w.reshape(*w.shape[:-1], K // group_size, group_size)
    wmin = g.amin(-1)
    wmax = g.amax(-1)
    scale = torch.clamp((wmax - wmin) / 15.0, min=1e-8).to(torch.bfloat16)
    bias = wmin.to(torch.bfloat16)
    q = torch.round((g - bias.float()[..., None]) / scale.float()[..., None]).clamp_(0, 15)
    q = q.reshape(*w.shape[:-1], K)
    return _pack_nibbles(q), scale, bias


def quantize_mxfp4(w: torch.Tensor):
    """OCP-MX mxfp4: shared e8m0 exponent per 32 (block max into e2m1 range),
    nearest e2m1 code per element -> (w_packed uint32, scales uint8)."""
    w = w.to(torch.float32)
    K = w.shape[-1]
    g = w.reshape(*w.shape[:-1], K // 32, 32)
    amax = g.abs().amax(-1).clamp_min(2.0**-126)
    ex = torch.floor(torch.log2(amax)).to(torch.int32) - 2
    e = (ex + 127).clamp(1, 254)
    s = torch.pow(torch.tensor(2.0, device=w.device), (e - 127).to(torch.float32))
    v = g / s[..., None]
    mags = torch.tensor(E2M1_MAGNITUDES, device=w.device)
    idx = (v.abs()[..., None] - mags).abs().argmin(-1)
    code = idx | (torch.signbit(v).to(torch.int64) << 3)
    return _pack_nibbles(code.reshape(*w.shape[:-1], K)), e.to(torch.uint8)


def dequantize(w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor | None, *, group_size: int = 64,
               mode: str = "affine") -> torch.Tensor:
    """Reference dequantisation to float32 (host-side utility, torch ops)."""
    wi = w.view(torch.int32).to(torch.int64) & 0xFFFFFFFF
    shifts = torch.arange(8, device=w.device, dtype=torch.int64) * 4
    q = ((wi[..., None] >> shifts) & 0xF).reshape(*w.shape[:-1], w.shape[-1] * 8)
    if mode == "affine":
        s = scales.float().repeat_interleave(group_size, -1)
        b = biases.float().repeat_interleave(group_size, -1)
        return q.float() * s + b
    lut = torch.tensor(E2M1_MAGNITUDES + tuple(-m for m in E2M1_MAGNITUDES), device=w.device)
    e = scales.to(torch.int32)
    s = torch.pow(torch.tensor(2.0, device=w.device), (e - 127).float()).repeat_interleave(32, -1)
    return lut[q] * s
