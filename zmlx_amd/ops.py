"""torch-facing MoE ops with the reference's names, arguments and errors.

Each op validates on the host, then enqueues hand-written HIP kernels of
``libzmlx_amd.so`` on the current torch stream of the tensors' device.  There
is no torch or CPU fallback: a missing library raises
:class:`zmlx_amd._native.NativeLibraryMissing`, a CPU tensor raises
``ValueError``.

Reference surface (Hmbown/ZMLX):
  gather_qmm_swiglu                ``src/zmlx/kernels/fused_moe.py:39-106``
                                    / ``mx.gather_qmm_swiglu`` (gather_qmm_swiglu.patch:695-800)
  gather_qmm                       MLX ``mx.gather_qmm`` as used at ``moe_mlp.py:572``
  topk_gating_softmax              ``src/zmlx/kernels/moe.py:1239-1396``
  router_argpartition_logits_topk  ``moe.py:1448-1490``
  deepseek_router_topk_sigmoid     ``moe.py:1745-1817``
  moe_combine{,_no_fma,_exact,_fp32,_fp32_no_fma}   ``moe.py:830-1127``
  moe_dispatch                     ``moe.py:776-827``
  gather_qmm_combine_quantized     ``moe.py:2043-2174``
  qwen_gating                      the Qwen branch of ``_gating`` (``moe_mlp.py:255-266``)

Index outputs are ``torch.int32`` (same bits as the reference's uint32 for
every valid expert index; torch cannot index with uint32 tensors).
"""

from __future__ import annotations

import math
from typing import Any

import torch

from . import _native as N

__all__ = [
    "gather_qmm_swiglu",
    "gather_qmm",
    "gather_qmm_grouped",
    "dense_logits",
    "qwen_gating",
    "topk_gating_softmax",
    "top2_gating_softmax",
    "router_argpartition_logits_topk",
    "deepseek_router_topk_sigmoid",
    "moe_dispatch",
    "swiglu2",
    "moe_combine",
    "moe_combine_no_fma",
    "moe_combine_exact",
    "moe_combine_fp32",
    "moe_combine_fp32_no_fma",
    "weighted_accumulate",
    "gather_qmm_combine_quantized",
    "has_gather_qmm_swiglu",
]


# ----------------------------------------------------------------------------
# plumbing
# ----------------------------------------------------------------------------


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _require_gpu(op: str, *ts: torch.Tensor | None) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if not isinstance(t, torch.Tensor):
            raise ValueError(f"{op}: expected torch tensors")
        if t.device.type != "cuda":
            raise ValueError(f"{op}: tensors must be on a ROCm GPU device (got {t.device})")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"{op}: all tensors must be on the same device")
    if dev is None:
        raise ValueError(f"{op}: no tensor arguments")
    return dev


def _c(t: torch.Tensor | None) -> torch.Tensor | None:
    return None if t is None else t.contiguous()


def _u16(t: torch.Tensor, op: str, name: str) -> torch.Tensor:
    if t.dtype != torch.bfloat16:
        raise ValueError(f"{op}: {name} must be bfloat16 (got {t.dtype})")
    return t.contiguous()


def has_gather_qmm_swiglu() -> bool:
    """True when the HIP library is loadable (fused_moe.py:25-31 analogue)."""
    try:
        N.lib()
        return True
    except N.NativeLibraryMissing:
        return False


def _mode_id(mode: str) -> int:
    if mode == "affine":
        return N.Q_AFFINE
    if mode == "mxfp4":
        return N.Q_MXFP4
    raise ValueError(f"[gather_qmm] Unsupported quantization mode {mode!r}.")


def _default_indices(batch_shape: tuple[int, ...], device) -> torch.Tensor:
    n = int(math.prod(batch_shape)) if batch_shape else 1
    return torch.arange(n, device=device, dtype=torch.int32).reshape(batch_shape)


def _prep_gather(op, x, w, lhs_indices, rhs_indices, transpose):
    if not transpose:
        raise ValueError(f"[{op}] Only transpose=True is supported.")
    if x.ndim < 2:
        raise ValueError(
            f"[{op}] Non-quantized input must have at least two dimensions but got input with shape {tuple(x.shape)}."
        )
    if w.ndim < 3:
        raise ValueError(f"[{op}] weights must have shape (E, N, K_packed).")
    if w.dtype not in (torch.uint32, torch.int32):
        raise ValueError(f"[{op}] packed weights must be uint32 (got {w.dtype}).")
    x_batch = tuple(x.shape[:-2])
    w_batch = tuple(w.shape[:-2])
    lhs = _default_indices(x_batch, x.device) if lhs_indices is None else lhs_indices
    rhs = _default_indices(w_batch, x.device) if rhs_indices is None else rhs_indices
    for name, t in (("lhs_indices", lhs), ("rhs_indices", rhs)):
        if t.dtype.is_floating_point or t.dtype == torch.bool:
            raise ValueError(f"[{op}] Got {name} with invalid dtype. Indices must be integral.")
    lhs, rhs = torch.broadcast_tensors(lhs.to(x.device), rhs.to(x.device))
    out_batch = tuple(lhs.shape)
    lhs = lhs.reshape(-1).to(torch.int32).contiguous()
    rhs = rhs.reshape(-1).to(torch.int32).contiguous()
    nx = int(math.prod(x_batch)) if x_batch else 1
    ne = int(math.prod(w_batch))
    return lhs, rhs, out_batch, nx, ne


# ----------------------------------------------------------------------------
# gather + quantized matmul
# ----------------------------------------------------------------------------


def gather_qmm_swiglu(
    x: torch.Tensor,
    gate_w: torch.Tensor,
    gate_scales: torch.Tensor,
    gate_biases: torch.Tensor | None,
    up_w: torch.Tensor,
    up_scales: torch.Tensor,
    up_biases: torch.Tensor | None,
    *,
    lhs_indices: torch.Tensor | None = None,
    rhs_indices: torch.Tensor | None = None,
    transpose: bool = True,
    group_size: int = 64,
    bits: int = 4,
    mode: str = "affine",
) -> torch.Tensor:
    """Fused gather + quantized matmul + SwiGLU: ``silu(gather_qmm(x, gate)) *
    gather_qmm(x, up)`` with the unpatched MLX rounding points.

    x ``(..., M, K)`` bf16; gate/up weights ``(E, N, K/8)`` uint32; output
    ``broadcast(lhs, rhs).shape + (M, N)`` bf16."""
    op = "gather_qmm_swiglu"
    dev = _require_gpu(op, x, gate_w, gate_scales, up_w, up_scales, gate_biases, up_biases)
    qm = _mode_id(mode)
    if qm == N.Q_AFFINE and (gate_biases is None or up_biases is None):
        raise ValueError(f"[{op}] affine mode requires biases.")
    if gate_w.shape != up_w.shape or gate_scales.shape != up_scales.shape:
        raise ValueError(f"[{op}] gate and up weights must have matching shapes.")
    lhs, rhs, out_batch, nx, ne = _prep_gather(op, x, gate_w, lhs_indices, rhs_indices, transpose)
    xc = _u16(x, op, "x")
    M, K = int(x.shape[-2]), int(x.shape[-1])
    Nn = int(gate_w.shape[-2])
    if int(gate_w.shape[-1]) * (32 // bits) != K:
        raise ValueError(f"[{op}] weight inner dimension {int(gate_w.shape[-1]) * (32 // bits)} does not match x ({K}).")
    out = torch.empty(out_batch + (M, Nn), dtype=torch.bfloat16, device=dev)
    gs, us = _c(gate_scales), _c(up_scales)
    gb, ub = _c(gate_biases), _c(up_biases)
    if qm == N.Q_AFFINE:
        gs, us, gb, ub = (_u16(t, op, "scales/biases") for t in (gs, us, gb, ub))
    rc = N.lib().zmoe_gather_qmm_swiglu(
        _stream(dev), _ptr(xc), nx, _ptr(gate_w.contiguous()), _ptr(gs), _ptr(gb), _ptr(up_w.contiguous()),
        _ptr(us), _ptr(ub), _ptr(lhs), _ptr(rhs), lhs.numel(), M, Nn, K, ne, group_size, bits, qm, _ptr(out),
    )
    N.check(rc, op)
    return out


def gather_qmm(
    x: torch.Tensor,
    w: torch.Tensor,
    scales: torch.Tensor,
    biases: torch.Tensor | None = None,
    lhs_indices: torch.Tensor | None = None,
    rhs_indices: torch.Tensor | None = None,
    transpose: bool = True,
    group_size: int = 64,
    bits: int = 4,
    mode: str = "affine",
) -> torch.Tensor:
    """Gather + quantized matmul (``mx.gather_qmm`` with ``transpose=True``),
    output bf16 ``broadcast(lhs, rhs).shape + (M, N)``."""
    op = "gather_qmm"
    dev = _require_gpu(op, x, w, scales, biases)
    qm = _mode_id(mode)
    lhs, rhs, out_batch, nx, ne = _prep_gather(op, x, w, lhs_indices, rhs_indices, transpose)
    xc = _u16(x, op, "x")
    M, K = int(x.shape[-2]), int(x.shape[-1])
    Nn = int(w.shape[-2])
    if int(w.shape[-1]) * (32 // bits) != K:
        raise ValueError(f"[{op}] weight inner dimension {int(w.shape[-1]) * (32 // bits)} does not match x ({K}).")
    out = torch.empty(out_batch + (M, Nn), dtype=torch.bfloat16, device=dev)
    s, b = _c(scales), _c(biases)
    if qm == N.Q_AFFINE:
        if b is None:
            raise ValueError(f"[{op}] affine mode requires biases.")
        s, b = _u16(s, op, "scales"), _u16(b, op, "biases")
    rc = N.lib().zmoe_gather_qmm(
        _stream(dev), _ptr(xc), nx, _ptr(w.contiguous()), _ptr(s), _ptr(b), _ptr(lhs), _ptr(rhs), lhs.numel(),
        M, Nn, K, ne, group_size, bits, qm, _ptr(out),
    )
    N.check(rc, op)
    return out


def gather_qmm_grouped(
    x: torch.Tensor,
    w: torch.Tensor,
    scales: torch.Tensor,
    biases: torch.Tensor | None,
    lhs_indices: torch.Tensor,
    rhs_indices: torch.Tensor,
    *,
    up: tuple | None = None,
    group_size: int = 64,
    bits: int = 4,
    mode: str = "affine",
) -> torch.Tensor:
    """Grouped (expert-sorted) gather + quantized matmul on MFMA for many
    single-row pairs: ``out[p] = x[lhs[p]] @ deq(w[rhs[p]]).T`` -- or, with
    ``up=(up_w, up_scales, up_biases)``, the SwiGLU of the two -- in pair
    order.  x ``(x_batch, K)`` bf16; returns ``(P, N)`` bf16.  The batched
    counterpart of :func:`gather_qmm` / :func:`gather_qmm_swiglu`
    (``mx.gather_qmm(..., sorted_indices=True)`` in mlx_lm's prefill)."""
    op = "gather_qmm"
    uw, us, ub = up if up is not None else (None, None, None)
    dev = _require_gpu(op, x, w, scales, biases, lhs_indices, rhs_indices, uw, us, ub)
    qm = _mode_id(mode)
    if x.dim() != 2:
        raise ValueError(f"[{op}] grouped path expects x of shape (x_batch, K).")
    if w.dim() != 3:
        raise ValueError(f"[{op}] weights must have shape (E, N, K_packed).")
    E, Nn = int(w.shape[0]), int(w.shape[1])
    K = int(x.shape[-1])
    if int(w.shape[-1]) * (32 // bits) != K:
        raise ValueError(f"[{op}] weight inner dimension {int(w.shape[-1]) * (32 // bits)} does not match x ({K}).")
    if up is not None and (uw.shape != w.shape or us.shape != scales.shape):
        raise ValueError(f"[{op}] gate and up weights must have matching shapes.")
    lhs = lhs_indices.reshape(-1).to(torch.int32).contiguous()
    rhs = rhs_indices.reshape(-1).to(torch.int32).contiguous()
    if lhs.numel() != rhs.numel():
        raise ValueError(f"[{op}] lhs_indices and rhs_indices must have the same number of elements.")
    P = int(rhs.numel())
    xc = _u16(x, op, "x").contiguous()
    s, b = _c(scales), _c(biases)
    us_, ub_ = _c(us), _c(ub)
    if qm == N.Q_AFFINE:
        if b is None or (up is not None and ub is None):
            raise ValueError(f"[{op}] affine mode requires biases.")
        s, b = _u16(s, op, "scales"), _u16(b, op, "biases")
        if up is not None:
            us_, ub_ = _u16(us_, op, "scales"), _u16(ub_, op, "biases")
    L = N.lib()
    ws_bytes = int(L.zmoe_grouped_gather_qmm_workspace_size(P, int(x.shape[0]), E, K, group_size))
    ws = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device=dev)
    out = torch.empty((P, Nn), dtype=torch.bfloat16, device=dev)
    rc = L.zmoe_grouped_gather_qmm(
        _stream(dev), _ptr(xc), int(x.shape[0]), _ptr(w.contiguous()), _ptr(s), _ptr(b),
        _ptr(None if uw is None else uw.contiguous()), _ptr(us_), _ptr(ub_), _ptr(lhs), _ptr(rhs), P, Nn, K, E,
        group_size, bits, qm, _ptr(ws), ws.numel(), _ptr(out),
    )
    N.check(rc, op)
    return out


def dense_logits(x: torch.Tensor, weight: torch.Tensor, *, out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """Router projection ``x @ weight.T`` (bf16 weights, f32 accumulation)."""
    op = "dense_logits"
    dev = _require_gpu(op, x, weight)
    xc = _u16(x, op, "x").reshape(-1, x.shape[-1])
    wc = _u16(weight, op, "weight")
    B, H = xc.shape
    E = int(wc.shape[0])
    if int(wc.shape[1]) != H:
        raise ValueError(f"{op}: weight must have shape (E, {H})")
    dt = N.DT_F32 if out_dtype == torch.float32 else N.DT_BF16
    out = torch.empty((B, E), dtype=out_dtype, device=dev)
    N.check(N.lib().zmoe_dense_logits(_stream(dev), _ptr(xc), _ptr(wc), B, E, H, dt, _ptr(out)), op)
    return out.reshape(*x.shape[:-1], E)


# ----------------------------------------------------------------------------
# routers
# ----------------------------------------------------------------------------


def _rows(x: torch.Tensor) -> tuple[torch.Tensor, int, int]:
    D = int(x.shape[-1])
    xc = x.contiguous().reshape(-1, D)
    return xc, int(xc.shape[0]), D


def qwen_gating(logits: torch.Tensor, k: int, norm_topk_prob: bool = True) -> tuple[torch.Tensor, torch.Tensor]:
    """Qwen3 gating: precise softmax of bf16 logits -> bf16 probabilities ->
    top-k -> gather -> optional ``/sum`` in bf16.  Returns ``(indices int32,
    weights bf16)`` like ``_gating`` (moe_mlp.py:255-266)."""
    op = "qwen_gating"
    dev = _require_gpu(op, logits)
    xc, B, E = _rows(_u16(logits, op, "logits"))
    w = torch.empty((B, k), dtype=torch.bfloat16, device=dev)
    idx = torch.empty((B, k), dtype=torch.int32, device=dev)
    N.check(N.lib().zmoe_router_softmax_topk(_stream(dev), _ptr(xc), B, E, int(k), int(bool(norm_topk_prob)),
                                             _ptr(w), _ptr(idx)), op)
    shp = tuple(logits.shape[:-1]) + (k,)
    return idx.reshape(shp), w.reshape(shp)


def topk_gating_softmax(
    x: torch.Tensor,
    k: int = 2,
    *,
    threadgroup: int = 256,
    compute_dtype: Any | None = None,
    expert_bias: torch.Tensor | None = None,
    norm_topk_prob: bool | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Top-k gating with softmax (moe.py:1239-1396).  Returns ``(weights
    float32, indices int32)``; ``threadgroup``/``compute_dtype`` are accepted
    for signature compatibility (compute is always float32)."""
    op = "topk_gating_softmax"
    K = int(k)
    if K <= 0:
        raise ValueError("topk_gating_softmax: k must be > 0")
    D = int(x.shape[-1])
    if K > D:
        raise ValueError(f"topk_gating_softmax: k={K} exceeds last dimension D={D}")
    dev = _require_gpu(op, x, expert_bias)
    norm = True if norm_topk_prob is None else bool(norm_topk_prob)
    if x.dtype == torch.bfloat16:
        dt = N.DT_BF16
        xs = x
    else:
        dt = N.DT_F32
        xs = x.to(torch.float32)
    xc, B, D = _rows(xs)
    bias = None
    if expert_bias is not None:
        if int(expert_bias.numel()) != D:
            raise ValueError(f"topk_gating_softmax: expert_bias must have {D} elements")
        bias = expert_bias.reshape(D).to(torch.float32).contiguous()
    w = torch.empty((B, K), dtype=torch.float32, device=dev)
    idx = torch.empty((B, K), dtype=torch.int32, device=dev)
    N.check(N.lib().zmoe_topk_gating_softmax(_stream(dev), _ptr(xc), dt, B, D, K, _ptr(bias), int(norm),
                                             _ptr(w), _ptr(idx)), op)
    shp = tuple(x.shape[:-1]) + (K,)
    return w.reshape(shp), idx.reshape(shp)


def top2_gating_softmax(x: torch.Tensor, *, threadgroup: int = 256, compute_dtype: Any | None = None):
    """Top-2 gating (moe.py:398-431): top-2 logits then softmax over them."""
    return topk_gating_softmax(x, 2, threadgroup=threadgroup, compute_dtype=compute_dtype)


def router_argpartition_logits_topk(logits: torch.Tensor, *, k: int, compute_dtype: Any | None = None):
    """Top-k on the logits then softmax over the selected logits
    (moe.py:1448-1490).  Returns ``(weights float32, indices int32)``."""
    if logits.ndim < 1:
        raise ValueError("router_argpartition_logits_topk: logits must have rank >= 1")
    K = int(k)
    D = int(logits.shape[-1])
    if K <= 0:
        raise ValueError("router_argpartition_logits_topk: k must be > 0")
    if K > D:
        raise ValueError(f"router_argpartition_logits_topk: k={K} exceeds D={D}")
    return topk_gating_softmax(logits, K, norm_topk_prob=True)


def deepseek_router_topk_sigmoid(
    logits: torch.Tensor,
    bias: torch.Tensor,
    *,
    k: int = 8,
    n_group: int = 1,
    topk_group: int = 1,
    threadgroup: int = 256,
    compute_dtype: Any | None = None,
    routed_scaling_factor: float = 1.0,
) -> tuple[torch.Tensor, torch.Tensor]:
    """DeepSeek/Kimi sigmoid router with selection bias and group selection
    (moe.py:1745-1817).  Returns ``(weights float32, indices int32)`` in
    selection order (score desc, index asc).  Unlike the reference, every
    expert count up to 1024 runs on the fused kernel (no MLX fallback)."""
    op = "deepseek_router_topk_sigmoid"
    if logits.ndim < 1:
        raise ValueError("deepseek_router_topk_sigmoid: logits must have rank >= 1")
    dev = _require_gpu(op, logits, bias)
    D = int(logits.shape[-1])
    if bias.ndim != 1:
        if int(bias.numel()) == D:
            bias = bias.reshape(D)
        else:
            raise ValueError(f"deepseek_router_topk_sigmoid: bias must have shape ({D},)")
    if int(bias.shape[0]) != D:
        raise ValueError(f"deepseek_router_topk_sigmoid: bias must have shape ({D},)")
    K = int(k)
    if K <= 0:
        raise ValueError("deepseek_router_topk_sigmoid: k must be > 0")
    if K > D:
        raise ValueError(f"deepseek_router_topk_sigmoid: k={K} exceeds D={D}")
    xc, B, D = _rows(logits.to(torch.float32))
    bc = bias.to(torch.float32).contiguous()
    w = torch.empty((B, K), dtype=torch.float32, device=dev)
    idx = torch.empty((B, K), dtype=torch.int32, device=dev)
    N.check(N.lib().zmoe_deepseek_router_topk_sigmoid(_stream(dev), _ptr(xc), _ptr(bc), B, D, K, int(n_group),
                                                      int(topk_group), float(routed_scaling_factor), _ptr(w),
                                                      _ptr(idx)), op)
    shp = tuple(logits.shape[:-1]) + (K,)
    return w.reshape(shp), idx.reshape(shp)


# ----------------------------------------------------------------------------
# dispatch / combine
# ----------------------------------------------------------------------------


def moe_dispatch(x: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
    """Copy each token to its K expert slots: ``(..., D) -> (..., K, D)``
    (moe.py:776-827; the indices give K only)."""
    op = "moe_dispatch"
    dev = _require_gpu(op, x)
    K = int(indices.shape[-1])
    D = int(x.shape[-1])
    xc = x.contiguous()
    B = int(xc.numel() // max(1, D))
    out = torch.empty((*x.shape[:-1], K, D), dtype=x.dtype, device=dev)
    N.check(N.lib().zmoe_moe_dispatch(_stream(dev), _ptr(xc), B, D, K, xc.element_size(), _ptr(out)), op)
    return out


def _swiglu2_dtype(t: torch.Tensor, op: str) -> int:
    if t.dtype == torch.bfloat16:
        return N.DT_BF16
    if t.dtype == torch.float32:
        return N.DT_F32
    raise ValueError(f"{op}: gate and up must be bfloat16 or float32 (got {t.dtype})")


class _SwiGLU2(torch.autograd.Function):
    @staticmethod
    def forward(ctx, gate, up):
        op = "swiglu2"
        dev = _require_gpu(op, gate, up)
        g, u = gate.contiguous(), up.contiguous()
        out = torch.empty_like(g)
        N.check(N.lib().zmoe_swiglu2(_stream(dev), _ptr(g), _ptr(u), g.numel(), _swiglu2_dtype(g, op), _ptr(out)),
                op)
        ctx.save_for_backward(g, u)
        return out

    @staticmethod
    def backward(ctx, cotan):
        op = "swiglu2"
        g, u = ctx.saved_tensors
        c = cotan.to(g.dtype).contiguous()
        dg, du = torch.empty_like(g), torch.empty_like(u)
        N.check(N.lib().zmoe_swiglu2_backward(_stream(g.device), _ptr(g), _ptr(u), _ptr(c), g.numel(),
                                              _swiglu2_dtype(g, op), _ptr(dg), _ptr(du)), op)
        return dg, du


def swiglu2(gate: torch.Tensor, up: torch.Tensor, *, compute_dtype: Any | None = None) -> torch.Tensor:
    """``SiLU(gate) * up`` with two separate inputs, differentiable
    (transformer.py:917-935).  bf16 or f32; ``compute_dtype`` is accepted and
    ignored, as the reference deprecates it."""
    if gate.shape != up.shape:
        raise ValueError("swiglu2: gate and up must have the same shape")
    if gate.dtype != up.dtype:
        raise ValueError("swiglu2: gate and up must have the same dtype")
    return _SwiGLU2.apply(gate, up)


def _combine(expert_outputs, weights, mode: int, op: str) -> torch.Tensor:
    dev = _require_gpu(op, expert_outputs, weights)
    K = int(weights.shape[-1])
    D = int(expert_outputs.shape[-1])
    y = _u16(expert_outputs, op, "expert_outputs").reshape(-1, K, D)
    B = int(y.shape[0])
    if mode in (N.COMBINE_FP32, N.COMBINE_FP32_NO_FMA):
        w = weights.to(torch.float32).contiguous().reshape(B, K)
        wdt = N.DT_F32
        out = torch.empty((B, D), dtype=torch.float32, device=dev)
    else:
        if weights.dtype == torch.float32 and mode not in (N.COMBINE_NATIVE, N.COMBINE_EXACT):
            w, wdt = weights.contiguous().reshape(B, K), N.DT_F32
        else:
            w, wdt = weights.to(torch.bfloat16).contiguous().reshape(B, K), N.DT_BF16
        out = torch.empty((B, D), dtype=torch.bfloat16, device=dev)
    N.check(N.lib().zmoe_moe_combine(_stream(dev), _ptr(y), _ptr(w), wdt, B, K, D, mode, _ptr(out)), op)
    return out.reshape(*weights.shape[:-1], D)


def moe_combine(expert_outputs: torch.Tensor, weights: torch.Tensor, *, native: bool = False) -> torch.Tensor:
    """Σ_k w·y with f32 FMA accumulation, bf16 out (moe.py:830-883).  With
    ``native=True``: MLX ``(y*w[...,None]).sum(-2)`` rounding (bf16 products)."""
    return _combine(expert_outputs, weights, N.COMBINE_NATIVE if native else N.COMBINE_FLOAT, "moe_combine")


def moe_combine_no_fma(expert_outputs: torch.Tensor, weights: torch.Tensor) -> torch.Tensor:
    """f32 multiply then f32 add, no contraction, bf16 out (moe.py:886-950)."""
    return _combine(expert_outputs, weights, N.COMBINE_NO_FMA, "moe_combine_no_fma")


def moe_combine_exact(expert_outputs: torch.Tensor, weights: torch.Tensor) -> torch.Tensor:
    """bf16 rounding after every multiply and add (moe.py:953-1006)."""
    return _combine(expert_outputs, weights, N.COMBINE_EXACT, "moe_combine_exact")


def moe_combine_fp32(expert_outputs: torch.Tensor, weights: torch.Tensor) -> torch.Tensor:
    """f32 FMA accumulation, float32 out (moe.py:1009-1066)."""
    return _combine(expert_outputs, weights, N.COMBINE_FP32, "moe_combine_fp32")


def moe_combine_fp32_no_fma(expert_outputs: torch.Tensor, weights: torch.Tensor) -> torch.Tensor:
    """f32 no-FMA accumulation, float32 out (moe.py:1069-1127)."""
    return _combine(expert_outputs, weights, N.COMBINE_FP32_NO_FMA, "moe_combine_fp32_no_fma")


def weighted_accumulate(acc: torch.Tensor, proj: torch.Tensor, gate: torch.Tensor, *, no_fma: bool = False,
                        out: torch.Tensor | None = None) -> torch.Tensor:
    """``out = acc + gate[:, None] * proj`` (moe.py:1820-1921); acc bf16 or f32."""
    op = "weighted_accumulate"
    dev = _require_gpu(op, acc, proj, gate)
    B, D = int(proj.shape[0]), int(proj.shape[-1])
    p = _u16(proj, op, "proj").reshape(B, D)
    a = acc.contiguous()
    if a.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"{op}: acc must be bfloat16 or float32")
    g = gate.to(torch.float32).contiguous().reshape(B)
    o = torch.empty_like(a) if out is None else out
    dt = N.DT_F32 if a.dtype == torch.float32 else N.DT_BF16
    N.check(N.lib().zmoe_weighted_accumulate(_stream(dev), _ptr(a), _ptr(p), _ptr(g), 1, B, D, dt, int(no_fma),
                                             _ptr(o)), op)
    return o


def _should_use_streaming(batch_size: int, streaming: bool | None) -> bool:
    """Streaming accumulation for B <= 16 unless forced (moe.py:1924-1932)."""
    if streaming is not None:
        return streaming
    return batch_size <= 16


def gather_qmm_combine_quantized(
    act: torch.Tensor,
    weights: torch.Tensor,
    scales: torch.Tensor,
    biases: torch.Tensor | None,
    gate: torch.Tensor,
    indices: torch.Tensor,
    *,
    group_size: int = 64,
    bits: int = 4,
    streaming: bool | None = None,
    no_fma: bool = False,
    output_dtype: torch.dtype | None = None,
    vectorized_k: bool = False,
    mode: str = "affine",
) -> torch.Tensor:
    """Down projection + combine (moe.py:2043-2174):
    ``out = sum_k gate[:, k] * gather_qmm(act[:, k], W[indices[:, k]])``.

    Streaming (default for B <= 16) accumulates per expert into the output
    dtype exactly like the reference's K loop; otherwise all K projections are
    computed in one launch and combined in k order."""
    if act.ndim != 3:
        raise ValueError("gather_qmm_combine_quantized: act must have shape (B, K, D_in)")
    B, K, D_in = (int(s) for s in act.shape)
    D_out = int(weights.shape[1])
    out_dtype = act.dtype if output_dtype is None else output_dtype
    idx = indices.reshape(B, K).to(torch.int32)
    if vectorized_k or not _should_use_streaming(B, streaming):
        proj = gather_qmm(
            act.reshape(B * K, 1, D_in), weights, scales, biases,
            lhs_indices=torch.arange(B * K, device=act.device, dtype=torch.int32).reshape(B, K),
            rhs_indices=idx, group_size=group_size, bits=bits, mode=mode,
        ).reshape(B, K, D_out)
        if out_dtype == torch.float32:
            return (moe_combine_fp32_no_fma if no_fma else moe_combine_fp32)(proj, gate.to(torch.float32))
        g = gate.to(proj.dtype)
        return (moe_combine_no_fma if no_fma else moe_combine)(proj, g)
    output = torch.zeros((B, D_out), dtype=out_dtype, device=act.device)
    lhs = torch.arange(B, device=act.device, dtype=torch.int32)
    for k in range(K):
        proj_k = gather_qmm(act[:, k, :].unsqueeze(1), weights, scales, biases, lhs_indices=lhs,
                            rhs_indices=idx[:, k], group_size=group_size, bits=bits, mode=mode).squeeze(1)
        output = weighted_accumulate(output, proj_k, gate[:, k], no_fma=no_fma)
    return output
