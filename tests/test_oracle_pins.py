"""CPU pins of the oracle (oracle/moe_oracle.py) -- no GPU, no MLX.

Each check compares the oracle with something it does not compute itself:
the number formats' definitions (OCP MX v1.0 e2m1/e8m0, bf16 round-to-
nearest-even via torch and via exact integer arithmetic), exhaustive tables,
known answers from the reference's own tests
(tests/test_fused_ops.py:247-267, tests/test_deepseek_router_topk_sigmoid.py:
77-180), mathematical identities and brute force on tiny inputs.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import moe_oracle as O

# ----------------------------------------------------------------------------
# bf16 rounding
# ----------------------------------------------------------------------------


def _bf16_exact(v: float) -> float:
    """Round a float64 to bf16 (8 significant bits, ties to even) with exact
    integer arithmetic: frexp gives v = m*2^e, m in [0.5, 1); m*256 is exact."""
    if v == 0.0 or not math.isfinite(v):
        return v
    m, e = math.frexp(v)
    r = round(m * 256.0)  # Python's round: exact value, ties to even
    return math.ldexp(r, e - 8)


def test_bf16_round_matches_torch():
    import torch

    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(100_000).astype(np.float32) * np.float32(10.0) ** rng.integers(-30, 30, 100_000),
        np.array([0.0, -0.0, 1.0, -1.0, 1.00390625, 1.001953125, 3.0e38, -3.0e38, 1e-40, np.inf, -np.inf], np.float32),
    ]).astype(np.float32)
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    got = O.bf16_round(x)
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_f64_to_bf16_single_rounding():
    """Double rounding (f64 -> f32 -> bf16) would be wrong exactly at bf16
    midpoints displaced by less than a float32 ulp; the oracle corrects them."""
    rng = np.random.default_rng(1)
    base = O.bf16_round(rng.standard_normal(20_000).astype(np.float32)).astype(np.float64)
    ulp = np.ldexp(1.0, np.frexp(np.abs(base))[1] - 8)
    tiny = ulp * 2.0**-30
    vals = np.concatenate([
        base + ulp / 2 + tiny, base + ulp / 2 - tiny, base + ulp / 2, base - ulp / 2,
        rng.standard_normal(20_000) * 100.0,
    ])
    got = O._f64_to_bf16(vals).astype(np.float64)
    ref = np.array([_bf16_exact(float(v)) for v in vals])
    np.testing.assert_array_equal(got, ref)


def test_bf16_ulp_diff():
    a = np.array([1.0, 1.0, -1.0, 0.0], np.float32)
    b = np.array([1.0078125, 1.0, -1.0078125, -0.0], np.float32)
    np.testing.assert_array_equal(O.bf16_ulp_diff(a, b), [1, 0, 1, 0])


# ----------------------------------------------------------------------------
# Dequantisation
# ----------------------------------------------------------------------------


def test_nibble_order():
    """quant.py:736-745: element i of a uint32 word sits at bits 4i."""
    w = np.array([[0x76543210, 0xFEDCBA98]], np.uint32)
    np.testing.assert_array_equal(O.unpack_uint(w, 4)[0], np.arange(16))


def test_affine_dequant_exhaustive_closed_form():
    """Every q in 0..15 at every nibble position, 512 random bf16 (scale,
    bias) pairs: the dequantised value is the float64 q*scale+bias rounded
    once to float32, bit for bit."""
    rng = np.random.default_rng(2)
    n = 512
    s = O.bf16_round(rng.standard_normal(n).astype(np.float32) * np.float32(0.01))
    b = O.bf16_round(rng.standard_normal(n).astype(np.float32) * np.float32(0.05))
    # row r: 64 elements = 8 words; word j holds q = (j*8 + i) % 16 at nibble i
    q = (np.arange(64) % 16).astype(np.uint32)
    words = np.zeros(8, np.uint32)
    for i in range(64):
        words[i // 8] |= np.uint32(q[i]) << np.uint32(4 * (i % 8))
    w = np.tile(words, (n, 1))
    got = O.dequant_affine(w, s[:, None], b[:, None], group_size=64)
    ref = (q[None, :].astype(np.float64) * s[:, None].astype(np.float64) + b[:, None].astype(np.float64)).astype(np.float32)
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("gs", [32, 64, 128])
def test_affine_groups(gs):
    """Group g of a row uses scales[:, g] / biases[:, g]."""
    K = 256
    w = np.full((2, K // 8), 0x11111111, np.uint32)  # every q = 1
    s = np.arange(2 * K // gs, dtype=np.float32).reshape(2, K // gs) + 1
    b = np.zeros_like(s)
    got = O.dequant_affine(w, s, b, group_size=gs)
    np.testing.assert_array_equal(got, np.repeat(s, gs, axis=-1))


def _e2m1_from_bits(c: int) -> float:
    """OCP MX v1.0 E2M1: sign bit 3, exponent bits 2..1 (bias 1), mantissa bit 0;
    exponent 0 is subnormal (0.5 * mantissa)."""
    sign = -1.0 if c & 8 else 1.0
    e, m = (c >> 1) & 3, c & 1
    mag = 0.5 * m if e == 0 else (1.0 + 0.5 * m) * 2.0 ** (e - 1)
    return sign * mag


def test_mxfp4_exhaustive_table():
    """All 16 codes x 256 e8m0 exponents against the format definition
    (2^(e-127), e = 0xFF is NaN)."""
    codes = np.arange(16, dtype=np.uint32)
    words = np.zeros(2, np.uint32)
    for i, c in enumerate(codes):
        words[i // 8] |= c << np.uint32(4 * (i % 8))
    w = np.zeros((256, 4), np.uint32)
    w[:, :2] = words  # elements 16..31 are code 0
    e = np.arange(256, dtype=np.uint8)[:, None]
    with np.errstate(over="ignore"):  # 6 * 2^127 is inf on both sides
        got = O.dequant_mxfp4(w, e)
    for ei in range(256):
        for c in range(16):
            v = got[ei, c]
            if ei == 255:
                assert np.isnan(v)
            else:
                with np.errstate(over="ignore"):
                    ref = np.float32(_e2m1_from_bits(c) * 2.0 ** (ei - 127))
                assert v == ref and np.signbit(v) == np.signbit(ref), (ei, c, v, ref)


def test_quantize_affine_roundtrip():
    """Fixture generator: q in 0..15 and reconstruction within half a step
    plus the bf16 rounding of scale and bias (MLX's exact choice unpinned)."""
    rng = np.random.default_rng(3)
    w = O.bf16_round(rng.standard_normal((64, 256)).astype(np.float32) * np.float32(0.02))
    q, s, b = O.quantize_affine(w, group_size=64)
    assert q.dtype == np.uint32 and q.shape == (64, 32)
    assert O.unpack_uint(q, 4).max() <= 15
    deq = O.dequant_affine(q, s, b, 64)
    step = np.repeat(np.abs(s), 64, axis=-1)
    assert (np.abs(deq - w) <= 0.5 * step + 2.0**-8 * np.abs(w).max()).all()


def test_quantize_mxfp4_exact_values():
    """Values on the e2m1 grid (block max 6 * 2^k) come back exactly."""
    rng = np.random.default_rng(4)
    mags = np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6], np.float32)
    v = mags[rng.integers(0, 8, (16, 128))] * np.where(rng.random((16, 128)) < 0.5, -1, 1).astype(np.float32)
    v[:, ::32] = 6.0  # every block reaches the top code
    scale = np.float32(2.0) ** rng.integers(-10, 4, (16, 4)).astype(np.float32)
    w = v * np.repeat(scale, 32, axis=-1)
    q, e = O.quantize_mxfp4(w)
    np.testing.assert_array_equal(O.dequant_mxfp4(q, e), w)


# ----------------------------------------------------------------------------
# GEMV / SwiGLU
# ----------------------------------------------------------------------------


def test_qmv_single_rounding_of_exact_dot():
    rng = np.random.default_rng(5)
    wq = rng.integers(0, 2**32, (16, 32), dtype=np.uint64).astype(np.uint32)
    s = O.bf16_round(rng.random((16, 4)).astype(np.float32) * np.float32(0.01))
    b = O.bf16_round(-rng.random((16, 4)).astype(np.float32) * np.float32(0.05))
    x = O.bf16_round(rng.standard_normal(256).astype(np.float32))
    wd = O.dequant_affine(wq, s, b, 64)
    got = O.qmv(x, wd)
    exact = [math.fsum(float(a) * float(c) for a, c in zip(wd[n], x)) for n in range(16)]
    np.testing.assert_array_equal(got, np.array([_bf16_exact(v) for v in exact], np.float32))


def test_gather_qmm_indices():
    """lhs picks the x batch, rhs the expert (mx.gather_qmm semantics)."""
    rng = np.random.default_rng(6)
    E, N, K = 3, 8, 256
    w = rng.integers(0, 2**32, (E, N, K // 8), dtype=np.uint64).astype(np.uint32)
    s = O.bf16_round(rng.random((E, N, K // 64)).astype(np.float32) * np.float32(0.01))
    b = np.zeros_like(s)
    x = O.bf16_round(rng.standard_normal((2, 1, K)).astype(np.float32))
    out = O.gather_qmm(x, w, s, b, [1, 0, 1], [2, 2, 0])
    for p, (li, ri) in enumerate([(1, 2), (0, 2), (1, 0)]):
        np.testing.assert_array_equal(out[p, 0], O.qmv(x[li, 0], O.dequant_affine(w[ri], s[ri], b[ri])))


def test_swiglu_points():
    g = np.array([0.0, 1.0, -1.0, 20.0, -20.0, 2.5], np.float32)
    u = np.array([3.0, 1.0, 1.0, 1.0, 1.0, -2.0], np.float32)
    got = O.swiglu(g, u).astype(np.float64)
    assert got[0] == 0.0
    assert got[3] == 20.0  # sigmoid(20) rounds to 1 in bf16
    assert abs(got[4]) < 1e-7
    exact = g / (1 + np.exp(-g.astype(np.float64))) * u
    np.testing.assert_allclose(got, exact, rtol=2**-7, atol=1e-7)
    np.testing.assert_array_equal(O.sigmoid_bf16(np.array([0.0], np.float32)), [0.5])


def test_sigmoid_abs_symmetry():
    """kk_sigmoid (msl.py:20-24): sigma(-x) = 1 - sigma(x) in the abs form."""
    x = np.linspace(-30, 30, 2001).astype(np.float32)
    s = O.sigmoid_abs_f32(x)
    np.testing.assert_allclose(s.astype(np.float64), 1 / (1 + np.exp(-x.astype(np.float64))), atol=6e-8)
    np.testing.assert_array_equal(s[x == 0], [0.5])


# ----------------------------------------------------------------------------
# Routers
# ----------------------------------------------------------------------------


def test_topk_desc_brute_force():
    """Value descending, equal values -> lower index (against Python sorted)."""
    rng = np.random.default_rng(7)
    for _ in range(300):
        n = int(rng.integers(2, 40))
        k = int(rng.integers(1, n + 1))
        v = rng.integers(0, 5, n).astype(np.float32)  # many ties
        ref = sorted(range(n), key=lambda i: (-float(v[i]), i))[:k]
        assert O.topk_desc(v, k).tolist() == ref


def test_topk_is_valid_tie_sets():
    v = np.array([1.0, 3.0, 2.0, 2.0, 0.0], np.float32)
    assert O.topk_is_valid(np.array([1, 2]), v, 2)
    assert O.topk_is_valid(np.array([1, 3]), v, 2)      # the other tie member
    assert not O.topk_is_valid(np.array([1, 0]), v, 2)  # beaten by index 2
    assert not O.topk_is_valid(np.array([1, 1]), v, 2)  # duplicate


def test_top2_known_answers():
    """tests/test_fused_ops.py:247-267."""
    x = np.array([[0.1, 0.2, 0.3, 0.4, 0.5, 0.6, 0.7, 0.8], [0.9, 0.8, 0.7, 0.6, 0.5, 0.4, 0.3, 0.2]], np.float32)
    w, idx = O.topk_gating_softmax(x, 2)
    assert set(idx[0].tolist()) == {7, 6} and set(idx[1].tolist()) == {0, 1}
    np.testing.assert_allclose(w.sum(-1), 1.0, rtol=1e-6)


def test_topk_gating_renorm_identity():
    """Softmax over the k selected logits equals the renormalised full
    softmax probabilities (moe.py:1287-1315 vs :1326-1377 without bias)."""
    rng = np.random.default_rng(8)
    x = rng.standard_normal((32, 64)).astype(np.float32)
    w_fast, i_fast = O.topk_gating_softmax(x, 6, None, True)
    p = np.exp(x.astype(np.float64) - x.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    sel = np.take_along_axis(p, i_fast, -1)
    np.testing.assert_allclose(w_fast, sel / sel.sum(-1, keepdims=True), rtol=1e-6)
    # bias path: bias added after the softmax, then selection
    bias = np.zeros(64, np.float32)
    bias[[5, 9]] = 1.0
    w_b, i_b = O.topk_gating_softmax(x, 2, bias, True)
    assert all(set(r) == {5, 9} for r in i_b.tolist())
    sel = np.take_along_axis(p + bias, i_b, -1)
    np.testing.assert_allclose(w_b, sel / sel.sum(-1, keepdims=True), rtol=1e-6)


def test_qwen_gating_against_float64():
    """Precise softmax -> bf16 probs; top-k; renormalised by the bf16 sum."""
    rng = np.random.default_rng(9)
    logits = O.bf16_round(rng.standard_normal((16, 128)).astype(np.float32))
    idx, w, p = O.qwen_gating(logits, 8, True)
    ex = np.exp(logits.astype(np.float64) - logits.max(-1, keepdims=True))
    np.testing.assert_array_equal(p, np.vectorize(_bf16_exact)(ex / ex.sum(-1, keepdims=True)).astype(np.float32))
    assert O.topk_is_valid(idx, p, 8).all()
    sel = np.take_along_axis(p, idx, -1).astype(np.float64)
    tot = np.vectorize(_bf16_exact)(sel.sum(-1, keepdims=True))
    np.testing.assert_array_equal(w, np.vectorize(_bf16_exact)(sel / tot).astype(np.float32))
    idx_nn, w_nn, _ = O.qwen_gating(logits, 8, False)
    np.testing.assert_array_equal(w_nn, np.take_along_axis(p, idx_nn, -1))


@pytest.mark.parametrize("D", [256, 384])
def test_deepseek_ties_lower_index(D):
    """test_deepseek_router_topk_sigmoid.py:109-124: zero logits and bias ->
    experts 0..7, weights exactly 1/8."""
    w, idx = O.deepseek_router_topk_sigmoid(np.zeros((1, D), np.float32), np.zeros(D, np.float32), k=8)
    assert idx[0].tolist() == list(range(8))
    np.testing.assert_array_equal(w[0], np.full(8, 0.125, np.float32))


@pytest.mark.parametrize("D", [256, 384])
def test_deepseek_bias_boost(D):
    """test_deepseek_router_topk_sigmoid.py:77-104: bias 10 on 8 experts picks
    exactly them, ordered by score; weights sigmoid(l)/sum in float64."""
    boost = [0, 7, 13, 64, 127, 128, D - 2, D - 1]
    logits = np.stack([np.linspace(-2.0, 2.0, D, dtype=np.float32) + np.float32(0.1 * i) for i in range(3)])
    bias = np.zeros(D, np.float32)
    bias[boost] = 10.0
    w, idx = O.deepseek_router_topk_sigmoid(logits, bias, k=8)
    for r in range(3):
        assert idx[r].tolist() == sorted(boost, reverse=True)  # logits increase with the index
        sig = 1 / (1 + np.exp(-logits[r, idx[r]].astype(np.float64)))
        np.testing.assert_allclose(w[r], sig / sig.sum(), rtol=1e-6, atol=1e-7)


def test_deepseek_group_select():
    """test_deepseek_router_topk_sigmoid.py:127-180 (D 256, 8 groups, keep 4).
    Closed form: group scores g0..g2 = 21, g3 = 11, g7 = 10, others 1, so g7
    (bias 9 at expert 224) is dropped and the 8th pick is the lowest-index
    0.5 in a kept group: {0,1,2,32,33,64,65,96}, weights 1/8."""
    bias = np.zeros(256, np.float32)
    bias[[0, 1, 32, 33, 64, 65, 96]] = 10.0
    bias[224] = 9.0
    w, idx = O.deepseek_router_topk_sigmoid(np.zeros((1, 256), np.float32), bias, k=8, n_group=8, topk_group=4)
    assert sorted(idx[0].tolist()) == [0, 1, 2, 32, 33, 64, 65, 96]
    np.testing.assert_array_equal(w[0], np.full(8, 0.125, np.float32))
    w2, _ = O.deepseek_router_topk_sigmoid(np.zeros((1, 256), np.float32), bias, k=8, n_group=8, topk_group=4,
                                           routed_scaling_factor=2.5)
    np.testing.assert_array_equal(w2[0], np.full(8, 0.3125, np.float32))


def test_deepseek_argument_errors():
    with pytest.raises(ValueError):
        O.deepseek_router_topk_sigmoid(np.zeros((1, 10), np.float32), np.zeros(10, np.float32), k=2, n_group=3)
    with pytest.raises(ValueError):
        O.deepseek_router_topk_sigmoid(np.zeros((1, 8), np.float32), np.zeros(8, np.float32), k=2, n_group=2,
                                       topk_group=3)


# ----------------------------------------------------------------------------
# Combines
# ----------------------------------------------------------------------------


def test_combine_one_hot_and_identity():
    rng = np.random.default_rng(10)
    y = O.bf16_round(rng.standard_normal((3, 4, 64)).astype(np.float32))
    w = np.zeros((3, 4), np.float32)
    w[np.arange(3), [0, 2, 3]] = 1.0
    for mode in O.COMBINE_MODES:
        out = O.moe_combine(y, w, mode)
        np.testing.assert_array_equal(out, y[np.arange(3), [0, 2, 3]], err_msg=mode)


def test_combine_no_fma_is_two_roundings():
    """fp32_no_fma: p = fl32(w*v), acc = fl32(acc + p), k ascending
    (moe.py:1069-1127) -- numpy float32 ops round each step; the FMA chain
    (fp32) differs from it somewhere on a random sample."""
    rng = np.random.default_rng(11)
    y = O.bf16_round(rng.standard_normal((64, 4, 512)).astype(np.float32))
    w = rng.random((64, 4)).astype(np.float32)
    acc = np.zeros((64, 512), np.float32)
    for k in range(4):
        acc = acc + w[:, k : k + 1] * y[:, k, :]  # float32 in, float32 out
    np.testing.assert_array_equal(O.moe_combine(y, w, "fp32_no_fma"), acc)
    fma = O.moe_combine(y, w, "fp32")
    assert (fma != acc).any()
    np.testing.assert_allclose(fma, acc, rtol=1e-5, atol=1e-6)
    np.testing.assert_array_equal(O.moe_combine(y, w, "no_fma"), O.bf16_round(acc))


def test_combine_native_against_float64():
    rng = np.random.default_rng(12)
    y = O.bf16_round(rng.standard_normal((8, 8, 256)).astype(np.float32))
    w = O.bf16_round(rng.random((8, 8)).astype(np.float32) / 8)
    got = O.moe_combine(y, w, "native").astype(np.float64)
    prods = y.astype(np.float64) * w[..., None].astype(np.float64)
    exact = prods.sum(-2)
    # bf16 unit roundoff u = 2^-8: products (rel. error <= u each), a float64
    # sum, one bf16 rounding of the result
    u = 2.0**-8
    bound = u * np.abs(prods).sum(-2) + u * (np.abs(exact) + u * np.abs(prods).sum(-2))
    assert (np.abs(got - exact) <= bound + 1e-30).all()


def test_weighted_accumulate_zero_gate():
    rng = np.random.default_rng(13)
    acc = O.bf16_round(rng.standard_normal((4, 64)).astype(np.float32))
    proj = rng.standard_normal((4, 64)).astype(np.float32)
    for no_fma in (False, True):
        np.testing.assert_array_equal(O.weighted_accumulate(acc, proj, np.zeros(4, np.float32), no_fma=no_fma), acc)


# ----------------------------------------------------------------------------
# Whole block: special cases that reduce to textbook routines
# ----------------------------------------------------------------------------


def _tiny_banks(rng, E=4, H=256, I=256):
    from tests.moe_case import make_bank

    return {n: make_bank(rng, E, *shape) for n, shape in (("gate", (I, H)), ("up", (I, H)), ("down", (H, I)))}


def test_layer_zero_input_is_zero():
    """x = 0 -> g = u = 0 -> silu = 0 -> y = 0 (for any routing)."""
    rng = np.random.default_rng(14)
    banks = _tiny_banks(rng)
    x = np.zeros((2, 256), np.float32)
    y = O.moe_experts(x, np.array([[0, 1], [2, 3]]), banks["gate"].as_tuple(), banks["up"].as_tuple(),
                      banks["down"].as_tuple())
    assert not y.any()


def test_layer_top1_unit_gate_is_gather_gemv():
    """K = 1 with weight 1 is the plain gather GEMV chain
    (test_gather_qmm_combine.py:149-174)."""
    rng = np.random.default_rng(15)
    banks = _tiny_banks(rng)
    x = O.bf16_round(rng.standard_normal((3, 256)).astype(np.float32))
    idx = np.array([[2], [0], [2]])
    y = O.moe_experts(x, idx, banks["gate"].as_tuple(), banks["up"].as_tuple(), banks["down"].as_tuple())
    out = O.moe_combine(y, np.ones((3, 1), np.float32), "native")
    for b in range(3):
        e = int(idx[b, 0])
        g = O.qmv(x[b], banks["gate"].deq(e))
        u = O.qmv(x[b], banks["up"].deq(e))
        np.testing.assert_array_equal(out[b], O.qmv(O.swiglu(g, u), banks["down"].deq(e)))


def test_swiglu2_f32_closed_form():
    """swiglu2 (f32) against the reference test's float64 formula
    (test_fused_ops.py:69-83, rtol 1e-4) and tighter: f32 evaluation."""
    rng = np.random.default_rng(5)
    g = rng.standard_normal((4, 257)).astype(np.float32) * 4
    u = rng.standard_normal((4, 257)).astype(np.float32)
    ref = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    np.testing.assert_allclose(O.swiglu2_f32(g, u), ref, rtol=1e-6, atol=1e-7)
    # special points: SiLU(0) = 0, large |g| saturates to g or 0
    np.testing.assert_allclose(O.swiglu2_f32(np.float32([0.0, 30.0, -30.0]), np.float32([5.0, 2.0, 2.0])),
                               [0.0, 60.0, -60.0 / (1 + np.exp(30.0))], rtol=1e-6, atol=0)


def test_swiglu2_backward_finite_differences():
    """The backward formula against central differences of the float64
    forward: a dropped term or sign fails by far more than the tolerance."""
    rng = np.random.default_rng(6)
    g = rng.standard_normal(64) * 3
    u = rng.standard_normal(64)
    c = rng.standard_normal(64)
    f = lambda gg, uu: gg / (1 + np.exp(-gg)) * uu  # noqa: E731
    h = 1e-6
    dg_fd = c * (f(g + h, u) - f(g - h, u)) / (2 * h)
    du_fd = c * (f(g, u + h) - f(g, u - h)) / (2 * h)
    dg, du = O.swiglu2_backward(g, u, c)
    np.testing.assert_allclose(dg, dg_fd, rtol=1e-6, atol=1e-8)
    np.testing.assert_allclose(du, du_fd, rtol=1e-6, atol=1e-8)


def test_moe_dispatch_by_loop():
    """moe_dispatch against the reference kernel's index formula
    out[(b*K + k)*D + d] = x[b*D + d] (moe.py:785-795), written as loops."""
    x = np.arange(3 * 5, dtype=np.int32).reshape(3, 5)
    K = 4
    got = O.moe_dispatch(x, K).reshape(-1)
    want = np.empty(3 * K * 5, np.int32)
    for b in range(3):
        for k in range(K):
            for d in range(5):
                want[(b * K + k) * 5 + d] = x.reshape(-1)[b * 5 + d]
    np.testing.assert_array_equal(got, want)
