"""numpy restatement of MLX's unpatched quantized-MoE block (parity oracle).

TEST INFRASTRUCTURE ONLY -- imported by ``tests/``, ``__graft_entry__.smoke``
and ``bench.py``'s CPU-baseline leg, never by the ``zmlx_amd`` package.

Every function restates one step of the path that ZMLX's ``patch(model)``
replaces, at the rounding points of the *unpatched* MLX evaluation (the parity
target of the reference's own tests):

* dequantisation          -- ``src/zmlx/kernels/quant.py:736-745`` (nibble
                              order, ``q*scale+bias``) and OCP MX v1.0 for mxfp4
* gather_qmm (GEMV)       -- ``tests/test_gather_qmm_swiglu.py:49-73`` (two-pass
                              reference), MLX ``mx.gather_qmm`` (third party)
* SwiGLU                  -- ``nn.silu(g) * u`` (same test file :73)
* routers                 -- ``src/zmlx/kernels/moe.py:1239-1396`` (softmax
                              top-k), ``:1448-1490`` (argpartition logits),
                              ``:1682-1742`` (DeepSeek grouped sigmoid) and the
                              Qwen gating branch ``patch/patterns/moe_mlp.py:255-266``
* combines                -- ``moe.py:830-1127`` and the native
                              ``(y*w[...,None]).sum(-2)`` of ``moe_mlp.py:1043``

Values are carried as float32 arrays holding bf16-representable numbers
wherever MLX holds a bf16 array; ``bf16_round`` is the only rounding primitive
(round-to-nearest-even, as MLX's and torch's float->bf16 casts).
Points where MLX's own choice is not visible from the reference (reduction
order of a bf16 ``sum``, argpartition tie order) are stated in each docstring
and only pinned by tolerance / tie-set rules in the tests.

Pinning (tests/test_oracle_pins.py, tests/test_golden.py): every function is
checked against closed forms, exhaustive format tables, the reference's known
answers, brute force or an independent C++ restatement.  Parity unpinned
(nothing without MLX can fix them): ``quantize_affine`` versus MLX's
``mx.quantize`` rounding, MLX qmv's accumulation order, the native combine's
bf16 ``sum`` order, ``mx.argpartition`` order inside tie sets, and mxfp4
versus MLX (the OCP MX closed form is pinned).
"""

from __future__ import annotations

import numpy as np

# ----------------------------------------------------------------------------
# bf16 helpers
# ----------------------------------------------------------------------------


def bf16_round(x) -> np.ndarray:
    """Round float32 values to the nearest bf16 (ties to even); NaN stays NaN."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = x.view(np.uint32).astype(np.uint64)
    lsb = (u >> np.uint64(16)) & np.uint64(1)
    r = ((u + np.uint64(0x7FFF) + lsb) >> np.uint64(16)) << np.uint64(16)
    out = r.astype(np.uint32).view(np.float32)
    return np.where(np.isnan(x), np.float32(np.nan), out).astype(np.float32)


def bf16_to_bits(x) -> np.ndarray:
    """float32 (already bf16-representable or not) -> uint16 bf16 bits (RNE)."""
    return (bf16_round(x).view(np.uint32) >> np.uint32(16)).astype(np.uint16)


def bf16_from_bits(b) -> np.ndarray:
    """uint16 bf16 bits -> float32 values."""
    b = np.asarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << np.uint32(16)).view(np.float32)


def bf16_ulp_diff(a, b) -> np.ndarray:
    """Distance in bf16 ulps between two bf16-valued float32 arrays."""

    def ordered(v):
        bits = bf16_to_bits(v).astype(np.int32)
        return np.where(bits & 0x8000, 0x8000 - bits, bits)

    return np.abs(ordered(a) - ordered(b))


# ----------------------------------------------------------------------------
# Dequantisation
# ----------------------------------------------------------------------------


def unpack_uint(w: np.ndarray, bits: int) -> np.ndarray:
    """Unpack MLX packed uint32 words: element i of a word sits at bits
    ``bits*i`` (low bits first) -- ``quant.py:736-745``."""
    epw = 32 // bits
    mask = np.uint32((1 << bits) - 1)
    shifts = (np.arange(epw, dtype=np.uint32) * np.uint32(bits)).astype(np.uint32)
    q = (np.asarray(w, dtype=np.uint32)[..., None] >> shifts) & mask
    return q.reshape(*w.shape[:-1], w.shape[-1] * epw)


def dequant_affine(w, scales, biases, group_size: int = 64, bits: int = 4) -> np.ndarray:
    """Affine dequant ``w_hat = scale*q + bias`` per group (``quant.py:741-745``).

    ``scales``/``biases`` are bf16-valued float32 ``[..., N, K/group_size]``.
    ``scale*q`` is exact in float32 (<= 8+8 significant bits), so this equals
    the single-rounding ``fma(q, scale, bias)`` the GPU evaluates.
    """
    q = unpack_uint(w, bits).astype(np.float32)
    s = np.repeat(np.asarray(scales, np.float32), group_size, axis=-1)
    b = np.repeat(np.asarray(biases, np.float32), group_size, axis=-1)
    return (q * s + b).astype(np.float32)


# OCP Microscaling v1.0 E2M1: sign bit 3, magnitudes {0,.5,1,1.5,2,3,4,6}.
E2M1_VALUES = np.array(
    [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0],
    dtype=np.float32,
)


def e8m0_to_float(e) -> np.ndarray:
    """OCP MX E8M0 scale: 2**(e-127); 0xFF is NaN."""
    e = np.asarray(e, dtype=np.int32)
    v = np.ldexp(np.float32(1.0), e - 127).astype(np.float32)
    return np.where(e == 255, np.float32(np.nan), v).astype(np.float32)


def dequant_mxfp4(w, scales_e8m0) -> np.ndarray:
    """mxfp4 dequant: ``e2m1[q] * 2**(e-127)``, group 32, no bias
    (MLX ``mode="mxfp4"``; the layer config uses it for GLM experts)."""
    q = unpack_uint(w, 4)
    s = np.repeat(e8m0_to_float(scales_e8m0), 32, axis=-1)
    return (E2M1_VALUES[q] * s).astype(np.float32)


def dequant(w, scales, biases, *, group_size=64, bits=4, mode="affine") -> np.ndarray:
    if mode == "affine":
        return dequant_affine(w, scales, biases, group_size, bits)
    if mode == "mxfp4":
        return dequant_mxfp4(w, scales)
    raise ValueError(f"unknown quantization mode {mode!r}")


# ----------------------------------------------------------------------------
# Quantisers (fixture generators only; not part of the checked path)
# ----------------------------------------------------------------------------


def quantize_affine(w_fp: np.ndarray, group_size: int = 64, bits: int = 4):
    """Min/max affine quantiser producing MLX-format (w_u32, scales, biases).

    Scale/bias are rounded to bf16 before the codes are chosen, so dequant of
    the codes is exactly representable by the stored parameters.  Its choice
    of scale/bias is this build's own (MLX's ``mx.quantize`` rounding is not
    needed: the kernels are checked on whatever codes are given)."""
    w = np.asarray(w_fp, dtype=np.float32)
    N, K = w.shape[-2], w.shape[-1]
    g = w.reshape(*w.shape[:-1], K // group_size, group_size)
    wmin = g.min(-1)
    wmax = g.max(-1)
    nb = (1 << bits) - 1
    scale = bf16_round(np.maximum((wmax - wmin) / nb, 1e-8))
    bias = bf16_round(wmin)
    q = np.clip(np.rint((g - bias[..., None]) / scale[..., None]), 0, nb).astype(np.uint32)
    q = q.reshape(*w.shape[:-1], K)
    epw = 32 // bits
    qw = q.reshape(*w.shape[:-1], K // epw, epw)
    shifts = (np.arange(epw, dtype=np.uint32) * np.uint32(bits)).astype(np.uint32)
    packed = np.bitwise_or.reduce(qw << shifts, axis=-1).astype(np.uint32)
    return packed, scale.astype(np.float32), bias.astype(np.float32)


def quantize_mxfp4(w_fp: np.ndarray):
    """OCP-MX style mxfp4 quantiser: shared exponent per 32 so the block max
    maps into the e2m1 range, then nearest e2m1 code per element."""
    w = np.asarray(w_fp, dtype=np.float32)
    K = w.shape[-1]
    g = w.reshape(*w.shape[:-1], K // 32, 32)
    amax = np.abs(g).max(-1)
    # shared exponent: floor(log2(amax)) - 2 (emax of e2m1)
    with np.errstate(divide="ignore"):
        ex = np.floor(np.log2(np.maximum(amax, 2.0**-126))).astype(np.int32) - 2
    e = np.clip(ex + 127, 1, 254).astype(np.uint8)
    s = e8m0_to_float(e)[..., None]
    v = g / s
    mags = E2M1_VALUES[:8]
    idx = np.abs(np.abs(v)[..., None] - mags).argmin(-1).astype(np.uint32)
    code = idx | (np.signbit(v).astype(np.uint32) << np.uint32(3))
    code = code.reshape(*w.shape[:-1], K)
    qw = code.reshape(*w.shape[:-1], K // 8, 8)
    shifts = (np.arange(8, dtype=np.uint32) * np.uint32(4)).astype(np.uint32)
    packed = np.bitwise_or.reduce(qw << shifts, axis=-1).astype(np.uint32)
    return packed, e


# ----------------------------------------------------------------------------
# GEMV stages
# ----------------------------------------------------------------------------


def qmv(x, w_deq) -> np.ndarray:
    """One quantized matrix-vector product as MLX's ``gather_qmm`` returns it:
    float accumulation, single rounding of the result to bf16.

    Accumulated here in float64 (the exact value to ~1e-16); the GPU's fp32
    accumulation is checked against it to within one bf16 ulp."""
    y = np.asarray(w_deq, np.float64) @ np.asarray(x, np.float64)
    return _f64_to_bf16(y)


def _f64_to_bf16(y64) -> np.ndarray:
    """Round float64 to bf16 with a single rounding (via exact float32 split)."""
    y64 = np.asarray(y64, np.float64)
    f = y64.astype(np.float32)  # RNE to float32 (may double-round, fixed below)
    # Correct possible double rounding: if the float32 value sits exactly on a
    # bf16 midpoint but the float64 value does not, nudge toward the float64.
    u = np.ascontiguousarray(f).view(np.uint32)
    mid = (u & np.uint32(0xFFFF)) == np.uint32(0x8000)
    if np.any(mid):
        resid = y64 - f.astype(np.float64)
        nudged = np.where(
            mid & (resid > 0),
            np.nextafter(f, np.float32(np.inf)),
            np.where(mid & (resid < 0), np.nextafter(f, np.float32(-np.inf)), f),
        ).astype(np.float32)
        f = nudged
    return bf16_round(f)


def gather_qmm(x, w, scales, biases, lhs_indices, rhs_indices, *, group_size=64, bits=4, mode="affine"):
    """``mx.gather_qmm(x, w, scales, biases, lhs_indices, rhs_indices,
    transpose=True)`` for x ``[Bx, M, K]``, w ``[E, N, K/epw]`` and 1-D index
    arrays of equal length P.  Returns bf16-valued float32 ``[P, M, N]``."""
    x = np.asarray(x, np.float32)
    lhs = np.asarray(lhs_indices).reshape(-1)
    rhs = np.asarray(rhs_indices).reshape(-1)
    out = []
    cache: dict[int, np.ndarray] = {}
    for li, ri in zip(lhs, rhs):
        ri = int(ri)
        if ri not in cache:
            cache[ri] = dequant(
                w[ri], scales[ri], None if biases is None else biases[ri],
                group_size=group_size, bits=bits, mode=mode,
            )
        wd = cache[ri]
        out.append(np.stack([qmv(xm, wd) for xm in x[int(li)]]))
    return np.stack(out).astype(np.float32)


def sigmoid_bf16(g) -> np.ndarray:
    """MLX ``mx.sigmoid`` on a bf16 array: evaluated in higher precision and
    rounded once to bf16."""
    g64 = np.asarray(g, np.float64)
    return _f64_to_bf16(1.0 / (1.0 + np.exp(-g64)))


def swiglu(g, u) -> np.ndarray:
    """``nn.silu(g) * u`` on bf16 arrays: silu = bf16(g*bf16(sigmoid(g))),
    out = bf16(silu*u) (``test_gather_qmm_swiglu.py:73``)."""
    sig = sigmoid_bf16(g)
    silu = bf16_round(np.asarray(g, np.float32) * sig)  # exact product of two bf16 in f32
    return bf16_round(silu * np.asarray(u, np.float32))


def swiglu2_f32(g, u) -> np.ndarray:
    """``transformer.swiglu2`` on float32 arrays (transformer.py:882-890,
    917-935): ``g * kk_sigmoid(g) * u`` evaluated in float32."""
    g = np.asarray(g, np.float32)
    return ((g * sigmoid_abs_f32(g)).astype(np.float32) * np.asarray(u, np.float32)).astype(np.float32)


def swiglu2_backward(g, u, cotan):
    """Backward of ``swiglu2`` (transformer.py:899-914) in float64:
    s = sigmoid(g), dgate = c*u*(s + g*s*(1 - s)), dup = c*g*s."""
    g = np.asarray(g, np.float64)
    u = np.asarray(u, np.float64)
    c = np.asarray(cotan, np.float64)
    s = 1.0 / (1.0 + np.exp(-g))
    sw = g * s
    return c * u * (s + sw * (1.0 - s)), c * sw


def moe_dispatch(x, k: int) -> np.ndarray:
    """``moe.moe_dispatch`` (moe.py:776-827): ``out[..., j, :] = x[..., :]``
    for every slot j < k."""
    x = np.asarray(x)
    return np.repeat(x[..., None, :], int(k), axis=-2)


def gather_qmm_swiglu(x, gw, gs, gb, uw, us, ub, lhs_indices, rhs_indices, *, group_size=64, bits=4, mode="affine"):
    """Unfused reference of ``mx.gather_qmm_swiglu`` (patch:695-800):
    ``silu(gather_qmm(gate)) * gather_qmm(up)``."""
    g = gather_qmm(x, gw, gs, gb, lhs_indices, rhs_indices, group_size=group_size, bits=bits, mode=mode)
    u = gather_qmm(x, uw, us, ub, lhs_indices, rhs_indices, group_size=group_size, bits=bits, mode=mode)
    return swiglu(g, u)


def dense_logits(x, w_router) -> np.ndarray:
    """Router ``nn.Linear`` (bf16 weights, no bias): bf16(x @ W.T)."""
    y = np.asarray(x, np.float64) @ np.asarray(w_router, np.float64).T
    return _f64_to_bf16(y)


# ----------------------------------------------------------------------------
# Routers
# ----------------------------------------------------------------------------


def softmax_precise_bf16(logits) -> np.ndarray:
    """``mx.softmax(bf16_logits, precise=True)``: float accumulation, bf16 out
    (``moe_mlp.py:261``)."""
    l64 = np.asarray(logits, np.float64)
    e = np.exp(l64 - l64.max(-1, keepdims=True))
    return _f64_to_bf16(e / e.sum(-1, keepdims=True))


def topk_desc(values, k: int) -> np.ndarray:
    """Top-k indices by value descending; equal values -> lower index first.
    This build's canonical order for MLX's (unspecified) argpartition order."""
    v = np.asarray(values)
    order = np.lexsort((np.broadcast_to(np.arange(v.shape[-1]), v.shape), -v.astype(np.float64)), axis=-1)
    return order[..., :k].astype(np.int64)


def topk_is_valid(sel, values, k: int) -> np.ndarray:
    """Per row: True when ``sel`` holds k distinct indices none of which is
    beaten by an unselected value (the set of valid answers under ties)."""
    v = np.asarray(values, np.float64)
    sel = np.asarray(sel, np.int64)
    rows = v.reshape(-1, v.shape[-1])
    srows = sel.reshape(-1, sel.shape[-1])
    ok = np.zeros(rows.shape[0], dtype=bool)
    for r in range(rows.shape[0]):
        s = srows[r]
        if len(set(s.tolist())) != k or s.min() < 0 or s.max() >= rows.shape[1]:
            continue
        mask = np.ones(rows.shape[1], bool)
        mask[s] = False
        ok[r] = (not mask.any()) or rows[r][s].min() >= rows[r][mask].max()
    return ok.reshape(v.shape[:-1])


def qwen_gating(logits, k: int, norm_topk_prob: bool = True, idx=None):
    """Qwen3 MoE gating (``moe_mlp.py:255-266``): precise softmax -> bf16
    probs -> top-k -> gather -> optional ``/sum`` (bf16 arithmetic).

    ``idx`` lets a caller pin the selection (e.g. the GPU's choice inside a
    tie set); otherwise the canonical order of ``topk_desc``.
    Returns (idx int64 [B,k], weights bf16-valued float32 [B,k], probs)."""
    p = softmax_precise_bf16(logits)
    if idx is None:
        idx = topk_desc(p, k)
    scores = np.take_along_axis(p, np.asarray(idx, np.int64), -1)
    if norm_topk_prob:
        s = _f64_to_bf16(scores.astype(np.float64).sum(-1, keepdims=True))
        scores = _f64_to_bf16(scores.astype(np.float64) / s.astype(np.float64))
    return np.asarray(idx, np.int64), scores.astype(np.float32), p


def topk_gating_softmax(x, k: int, expert_bias=None, norm_topk_prob=None, idx=None):
    """``moe.topk_gating_softmax`` (moe.py:1239-1396), compute dtype float32.

    * no bias, renormalised (default): top-k of the *logits*, softmax over the
      k selected values (moe.py:1287-1315); exact for the renormalised case.
    * bias and/or ``norm_topk_prob=False``: full softmax, ``+bias`` after the
      softmax, top-k, optional ``/(sum+1e-20)`` (moe.py:1326-1377).
    Returns (weights float32 [..,k], indices int64 [..,k])."""
    xf = np.asarray(x, np.float32).astype(np.float64)
    norm = True if norm_topk_prob is None else bool(norm_topk_prob)
    if expert_bias is None and norm:
        if idx is None:
            idx = topk_desc(xf, k)
        v = np.take_along_axis(xf, np.asarray(idx, np.int64), -1)
        e = np.exp(v - v.max(-1, keepdims=True))
        return (e / e.sum(-1, keepdims=True)).astype(np.float32), np.asarray(idx, np.int64)
    e = np.exp(xf - xf.max(-1, keepdims=True))
    gates = e / e.sum(-1, keepdims=True)
    if expert_bias is not None:
        gates = gates + np.asarray(expert_bias, np.float32).astype(np.float64)
    if idx is None:
        idx = topk_desc(gates, k)
    scores = np.take_along_axis(gates, np.asarray(idx, np.int64), -1)
    if norm:
        scores = scores / (scores.sum(-1, keepdims=True) + 1e-20)
    return scores.astype(np.float32), np.asarray(idx, np.int64)


def router_argpartition_logits_topk(logits, k: int, idx=None):
    """``moe.router_argpartition_logits_topk`` (moe.py:1448-1490): top-k on the
    logits, softmax over the selected logits in selection order."""
    return topk_gating_softmax(logits, k, None, True, idx=idx)


def sigmoid_abs_f32(x) -> np.ndarray:
    """``kk_sigmoid`` (msl.py:20-24) in float32: y=1/(1+exp(|x|)); x<0 ? y : 1-y."""
    x = np.asarray(x, np.float32)
    y = (np.float32(1.0) / (np.float32(1.0) + np.exp(np.abs(x)).astype(np.float32))).astype(np.float32)
    return np.where(x < 0, y, (np.float32(1.0) - y)).astype(np.float32)


def deepseek_router_topk_sigmoid(logits, bias, k: int = 8, n_group: int = 1, topk_group: int = 1,
                                 routed_scaling_factor: float = 1.0):
    """DeepSeek/Kimi grouped sigmoid router (moe.py:1682-1742 and the kernel
    :1501-1679; scaling from ``deepseek_router.py:118-119``).

    score = sigmoid(l) + bias; group score = top1+top2 within each group;
    keep ``topk_group`` groups (ties -> lower group), dropped groups' scores
    become 0.0; top-k with ties -> lower expert index; weights are the selected
    sigmoids normalised by their float32 sum, times the routed scaling factor.
    Returns (weights float32 [B,k], indices int64 [B,k]) in selection order."""
    L = np.asarray(logits, np.float32).reshape(-1, np.asarray(logits).shape[-1])
    D = L.shape[-1]
    if D % n_group != 0:
        raise ValueError("deepseek_router_topk_sigmoid: n_group must divide D")
    if topk_group <= 0 or topk_group > n_group:
        raise ValueError("deepseek_router_topk_sigmoid: invalid topk_group")
    aff = sigmoid_abs_f32(L)
    scores = (aff + np.asarray(bias, np.float32)).astype(np.float32)
    if n_group > 1 and topk_group < n_group:
        gsz = D // n_group
        grouped = scores.reshape(-1, n_group, gsz)
        srt = -np.sort(-grouped, axis=-1)
        gscore = (srt[..., 0] + srt[..., 1]).astype(np.float32)
        keep_g = topk_desc(gscore, topk_group)
        keep = np.zeros_like(gscore, dtype=bool)
        np.put_along_axis(keep, keep_g, True, axis=-1)
        grouped = np.where(keep[..., None], grouped, np.float32(0.0))
        scores = grouped.reshape(-1, D).astype(np.float32)
    idx = topk_desc(scores, k)
    sel = np.take_along_axis(aff, idx, -1).astype(np.float32)
    ssum = np.zeros(sel.shape[0], np.float32)
    for j in range(k):  # float32 sum in selection order
        ssum = (ssum + sel[:, j]).astype(np.float32)
    w = (sel / ssum[:, None]).astype(np.float32)
    if routed_scaling_factor != 1.0:
        w = (w * np.float32(routed_scaling_factor)).astype(np.float32)
    shape = np.asarray(logits).shape[:-1] + (k,)
    return w.reshape(shape), idx.reshape(shape)


# ----------------------------------------------------------------------------
# Combines
# ----------------------------------------------------------------------------

COMBINE_MODES = ("native", "fp32", "fp32_no_fma", "exact", "float", "no_fma")


def _fma32(a, b, c):
    """float32 fused multiply-add with a single rounding (a*b exact in f64)."""
    return (np.asarray(a, np.float64) * np.asarray(b, np.float64) + np.asarray(c, np.float64)).astype(np.float32)


def moe_combine(y, w, mode: str = "native") -> np.ndarray:
    """Weighted expert sum over axis -2, k ascending.

    y: bf16-valued float32 ``[B, K, D]``; w: ``[B, K]`` (bf16-valued for
    ``native``/``exact``/``float``/``no_fma``, float32 for the fp32 modes).

    * ``native``      MLX ``(y*w[...,None]).sum(-2)`` on bf16 operands
                      (moe_mlp.py:1043): products rounded to bf16, summed with
                      float accumulation, result rounded to bf16.  MLX's bf16
                      reduction order is not visible: pinned by tolerance.
    * ``fp32``        ``moe_combine_fp32`` (moe.py:1009-1066): f32 FMA chain,
                      float32 out.
    * ``fp32_no_fma`` ``moe_combine_fp32_no_fma`` (moe.py:1069-1127):
                      p=fl(w*v); acc=fl(acc+p); float32 out.  Bit-exact target.
    * ``exact``       ``moe_combine_exact`` (moe.py:953-1006): bf16 rounding
                      after every multiply and add.
    * ``float``       ``moe_combine`` (moe.py:830-883): f32 FMA chain, bf16 out.
    * ``no_fma``      ``moe_combine_no_fma`` (moe.py:886-950): f32 no-FMA
                      chain, bf16 out.
    """
    y = np.asarray(y, np.float32)
    w = np.asarray(w, np.float32)
    B, K, D = y.shape
    if mode == "native":
        p = bf16_round(y * w[..., None])
        return _f64_to_bf16(p.astype(np.float64).sum(-2))
    acc = np.zeros((B, D), np.float32)
    for k in range(K):
        wk = w[:, k : k + 1]
        vk = y[:, k, :]
        if mode in ("fp32", "float"):
            acc = _fma32(wk, vk, acc)
        elif mode in ("fp32_no_fma", "no_fma"):
            acc = (acc + (wk * vk).astype(np.float32)).astype(np.float32)
        elif mode == "exact":
            acc = bf16_round(acc + bf16_round(wk * vk))
        else:
            raise ValueError(f"unknown combine mode {mode!r}")
    if mode in ("float", "no_fma"):
        return bf16_round(acc)
    return acc


def weighted_accumulate(acc, proj, gate, *, no_fma=False, fp32_out=False) -> np.ndarray:
    """Streaming combine step ``out = acc + gate[row]*proj`` (moe.py:1820-1921)."""
    acc = np.asarray(acc, np.float32)
    proj = np.asarray(proj, np.float32)
    g = np.asarray(gate, np.float32)[:, None]
    out = (acc + (g * proj).astype(np.float32)).astype(np.float32) if no_fma else _fma32(g, proj, acc)
    return out if fp32_out else bf16_round(out)


# ----------------------------------------------------------------------------
# Whole MoE block
# ----------------------------------------------------------------------------


def moe_experts(x, idx, gate, up, down, *, group_size=64, bits=4, mode="affine"):
    """Routed experts for tokens x ``[B, H]`` and routing idx ``[B, K]``:
    gate/up gather_qmm -> SwiGLU -> down gather_qmm.  Each of gate/up/down is
    a tuple (w, scales, biases).  Returns bf16-valued ``[B, K, H]``."""
    x = np.asarray(x, np.float32)
    B, K = np.asarray(idx).shape
    lhs = np.repeat(np.arange(B), K)
    rhs = np.asarray(idx).reshape(-1)
    xx = x[:, None, :]
    act = gather_qmm_swiglu(xx, *gate, *up, lhs, rhs, group_size=group_size, bits=bits, mode=mode)
    y = gather_qmm(act, *down, np.arange(B * K), rhs, group_size=group_size, bits=bits, mode=mode)
    return y.reshape(B, K, -1)


def shared_expert(x, gate, up, down, *, group_size=64, bits=4, mode="affine"):
    """Dense SwiGLU shared expert (GLM/DeepSeek ``shared_experts``), bf16."""
    x = np.asarray(x, np.float32)
    B = x.shape[0]
    z = np.zeros(B, np.int64)
    one = lambda t: tuple(None if a is None else np.asarray(a)[None] for a in t)  # noqa: E731
    act = gather_qmm_swiglu(x[:, None, :], *one(gate), *one(up), np.arange(B), z,
                            group_size=group_size, bits=bits, mode=mode)
    y = gather_qmm(act, *one(down), np.arange(B), z, group_size=group_size, bits=bits, mode=mode)
    return y[:, 0, :]
