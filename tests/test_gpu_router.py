"""GPU parity: router projection and top-k gating kernels vs the oracle.

Reference pins: tests/test_kernels_catalog.py:139-210 (topk_gating_softmax
normalised / full-softmax / bias vs softmax->argpartition->renorm; argpartition
logits), tests/test_fused_ops.py:247-267 (top-2 known answers),
tests/test_deepseek_router_topk_sigmoid.py:77-180 (bias boosts, zero logits
-> [0..7] with weights exactly 1/8, group selection).
Index sets must be valid top-k sets of the oracle's values (exact up to ties).
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import moe_oracle as O
from tests.moe_case import bf16_randn, from_dev, to_bf16

pytestmark = pytest.mark.gpu


def _t(a, dev, dtype=None):
    import torch

    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return t if dtype is None else t.to(dtype)


def test_dense_logits(dev):
    import torch

    import zmlx_amd as Z

    rng = np.random.default_rng(0)
    for B, E, H in [(1, 128, 2048), (5, 32, 2048), (3, 256, 7168), (16, 64, 2048), (6, 42, 1032), (2, 7, 4608), (40, 64, 2048), (33, 20, 1032)]:
        x = bf16_randn(rng, (B, H))
        w = bf16_randn(rng, (E, H), 0.02)
        got = Z.dense_logits(to_bf16(x, dev), to_bf16(w, dev))
        got32 = Z.dense_logits(to_bf16(x, dev), to_bf16(w, dev), out_dtype=torch.float32)
        torch.cuda.synchronize()
        ref = O.dense_logits(x, w)
        ulp = O.bf16_ulp_diff(from_dev(got), ref)
        assert ulp.max() <= 1 and (ulp == 0).mean() >= 0.99
        exact = x.astype(np.float64) @ w.astype(np.float64).T
        np.testing.assert_allclose(from_dev(got32), exact, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("B,E,k,norm", [(64, 128, 8, True), (16, 128, 8, False), (32, 64, 4, True), (8, 512, 16, True)])
def test_qwen_gating(dev, B, E, k, norm):
    import torch

    import zmlx_amd as Z

    rng = np.random.default_rng(E + k)
    logits = bf16_randn(rng, (B, E), 0.9)
    idx, w = Z.qwen_gating(to_bf16(logits, dev), k, norm)
    torch.cuda.synchronize()
    idx = from_dev(idx).astype(np.int64)
    p = O.softmax_precise_bf16(logits)
    assert O.topk_is_valid(idx, p, k).all()
    # order: probability descending, lower index first on ties
    sel_p = np.take_along_axis(p, idx, -1)
    assert (np.diff(sel_p, axis=-1) <= 0).all()
    _, w_ref, _ = O.qwen_gating(logits, k, norm, idx=idx)
    # exact except where the fp32 softmax lands within noise of a bf16 midpoint
    ulp = O.bf16_ulp_diff(from_dev(w), w_ref)
    assert ulp.max() <= 1 and (ulp == 0).mean() >= 0.99


def test_topk_gating_softmax_variants(dev):
    import torch

    import zmlx_amd as Z

    rng = np.random.default_rng(1)
    # normalised fast path (test_kernels_catalog.py:139-155), D=32 and D=48
    for B, D, k in [(4, 32, 4), (3, 48, 6), (7, 128, 8)]:
        x = bf16_randn(rng, (B, D))
        w, idx = Z.topk_gating_softmax(to_bf16(x, dev), k=k, norm_topk_prob=True)
        torch.cuda.synchronize()
        idx = from_dev(idx).astype(np.int64)
        assert O.topk_is_valid(idx, x, k).all()
        w_ref, _ = O.topk_gating_softmax(x, k, None, True, idx=idx)
        np.testing.assert_allclose(from_dev(w), w_ref, rtol=2e-6, atol=1e-7)
        np.testing.assert_allclose(from_dev(w).sum(-1), 1.0, rtol=1e-5)
    # full softmax, no renorm (:158-173)
    x = bf16_randn(rng, (3, 48))
    w, idx = Z.topk_gating_softmax(to_bf16(x, dev), k=6, norm_topk_prob=False)
    torch.cuda.synchronize()
    idx = from_dev(idx).astype(np.int64)
    full = np.exp(x - x.max(-1, keepdims=True))
    full /= full.sum(-1, keepdims=True)
    assert O.topk_is_valid(idx, full, 6).all()
    w_ref, _ = O.topk_gating_softmax(x, 6, None, False, idx=idx)
    np.testing.assert_allclose(from_dev(w), w_ref, rtol=2e-6, atol=1e-8)
    # with expert bias (:176-196)
    x = bf16_randn(rng, (2, 40))
    bias = (rng.standard_normal(40).astype(np.float32) * 0.01).astype(np.float32)
    w, idx = Z.topk_gating_softmax(to_bf16(x, dev), k=4, expert_bias=_t(bias, dev), norm_topk_prob=True)
    torch.cuda.synchronize()
    idx = from_dev(idx).astype(np.int64)
    w_ref, _ = O.topk_gating_softmax(x, 4, bias, True, idx=idx)
    np.testing.assert_allclose(from_dev(w), w_ref, rtol=2e-6, atol=1e-7)


def test_top2_known_answer(dev):
    """test_fused_ops.py:247-267."""
    import torch

    import zmlx_amd as Z

    x = np.array([[0.1, 0.2, 0.3, 0.4, 0.5, 0.6, 0.7, 0.8],
                  [0.9, 0.8, 0.7, 0.6, 0.5, 0.4, 0.3, 0.2]], np.float32)
    w, idx = Z.top2_gating_softmax(_t(x, dev))
    torch.cuda.synchronize()
    idx = from_dev(idx)
    assert set(idx[0].tolist()) == {7, 6}
    assert set(idx[1].tolist()) == {0, 1}
    np.testing.assert_allclose(from_dev(w).sum(-1), 1.0, rtol=1e-5)


def test_router_argpartition_logits_topk(dev):
    """test_kernels_catalog.py:199-210: weights to 1e-6 of softmax over the
    selected logits."""
    import torch

    import zmlx_amd as Z

    rng = np.random.default_rng(2)
    x = rng.standard_normal((5, 64)).astype(np.float32)
    w, idx = Z.router_argpartition_logits_topk(_t(x, dev), k=8)
    torch.cuda.synchronize()
    idx = from_dev(idx).astype(np.int64)
    assert O.topk_is_valid(idx, x, 8).all()
    sel = np.take_along_axis(x, idx, -1).astype(np.float64)
    ref = np.exp(sel - sel.max(-1, keepdims=True))
    ref /= ref.sum(-1, keepdims=True)
    np.testing.assert_allclose(from_dev(w), ref, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("D", [256, 384])
def test_deepseek_bias_boost(dev, D):
    """test_deepseek_router_topk_sigmoid.py:77-104."""
    import torch

    import zmlx_amd as Z

    B = 3
    row = np.linspace(-2.0, 2.0, D, dtype=np.float32)
    logits = np.stack([row + np.float32(0.1 * i) for i in range(B)]).astype(np.float32)
    boost = [0, 7, 13, 64, 127, 128, D - 2, D - 1]
    bias = np.zeros(D, np.float32)
    bias[boost] = 10.0
    w, idx = Z.deepseek_router_topk_sigmoid(_t(logits, dev), _t(bias, dev), k=8)
    torch.cuda.synchronize()
    w_ref, i_ref = O.deepseek_router_topk_sigmoid(logits, bias, 8)
    np.testing.assert_array_equal(from_dev(idx), i_ref)
    for r in range(B):
        assert set(from_dev(idx)[r].tolist()) == set(boost)
    np.testing.assert_allclose(from_dev(w), w_ref, rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("D", [256, 384])
def test_deepseek_zero_logits_tiebreak(dev, D):
    """test_deepseek_router_topk_sigmoid.py:109-124: exactly [0..7], 1/8."""
    import torch

    import zmlx_amd as Z

    w, idx = Z.deepseek_router_topk_sigmoid(_t(np.zeros((1, D), np.float32), dev), _t(np.zeros(D, np.float32), dev))
    torch.cuda.synchronize()
    assert from_dev(idx)[0].tolist() == list(range(8))
    np.testing.assert_array_equal(from_dev(w)[0], np.full(8, 0.125, np.float32))


def test_deepseek_group_selection(dev):
    """test_deepseek_router_topk_sigmoid.py:128-180: group 7 is dropped, the
    8th pick is the lowest-index 0.5 of a kept group (expert 2)."""
    import torch

    import zmlx_amd as Z

    D = 256
    bias = np.zeros(D, np.float32)
    bias[[0, 1, 32, 33, 64, 65, 96]] = 10.0
    bias[224] = 9.0
    w, idx = Z.deepseek_router_topk_sigmoid(_t(np.zeros((1, D), np.float32), dev), _t(bias, dev), k=8,
                                            n_group=8, topk_group=4)
    torch.cuda.synchronize()
    assert sorted(from_dev(idx)[0].tolist()) == [0, 1, 2, 32, 33, 64, 65, 96]
    np.testing.assert_allclose(from_dev(w)[0], np.full(8, 0.125, np.float32), rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("D,k,ng,tg,scale", [(256, 8, 8, 4, 2.5), (64, 4, 1, 1, 1.8), (384, 8, 8, 4, 1.0), (160, 6, 8, 3, 1.0)])
def test_deepseek_random_vs_oracle(dev, D, k, ng, tg, scale):
    import torch

    import zmlx_amd as Z

    rng = np.random.default_rng(D + k)
    logits = O.bf16_round(rng.standard_normal((33, D)).astype(np.float32))
    bias = (rng.standard_normal(D) * 0.1).astype(np.float32)
    w, idx = Z.deepseek_router_topk_sigmoid(_t(logits, dev), _t(bias, dev), k=k, n_group=ng, topk_group=tg,
                                            routed_scaling_factor=scale)
    torch.cuda.synchronize()
    w_ref, i_ref = O.deepseek_router_topk_sigmoid(logits, bias, k, ng, tg, scale)
    np.testing.assert_array_equal(from_dev(idx), i_ref)
    np.testing.assert_allclose(from_dev(w), w_ref, rtol=1e-6, atol=1e-7)
