"""GPU parity at full layer shapes, all experts present:

- Qwen3-30B-A3B: hidden 2048, 128 experts, top-8 softmax router with
  renormalised weights, expert intermediate 768, affine 4-bit group 64;
  decode batches 1, 4 and 16 (the bench's workload);
- Qwen3-30B-A3B prefill: 512 Zipf-skewed tokens (config 4);
- DeepSeek-V3: hidden 7168, 256 routed experts in 8 groups (top-4 groups,
  top-8 experts, sigmoid + correction bias, routed scaling 2.5), one shared
  expert, expert intermediate 2048; decode batches 1 and 64 (the second runs
  the grouped path).

Every expert's weights are generated and quantised on the GPU.  The oracle
checks every token's routing against the full router, and the layer output of
a few tokens through the experts those tokens selected (their packed tensors
read back), which keeps the float64 oracle to seconds."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import moe_oracle as O
from tests.moe_case import Bank, bf16_randn, from_dev, to_bf16

pytestmark = pytest.mark.gpu

H, E, I, K, NG, TG, SCALE = 7168, 256, 2048, 8, 8, 4, 2.5
QH, QE, QI, QK = 2048, 128, 768, 8


def _gpu_bank(gen, dev, E_, N, Kd, chunk=16):
    """Packed affine g64 weights [E_, N, Kd] from N(0, 0.02) bf16, built on
    the GPU chunk by chunk."""
    import torch

    from zmlx_amd.quant import quantize_affine

    w = torch.empty((E_, N, Kd // 8), dtype=torch.uint32, device=dev)
    s = torch.empty((E_, N, Kd // 64), dtype=torch.bfloat16, device=dev)
    b = torch.empty_like(s)
    for e0 in range(0, E_, chunk):
        e1 = min(E_, e0 + chunk)
        x = (torch.randn((e1 - e0, N, Kd), generator=gen, device=dev) * 0.02).to(torch.bfloat16)
        q, sc, bi = quantize_affine(x, 64)
        w[e0:e1], s[e0:e1], b[e0:e1] = q, sc, bi
    return w, s, b


def _host_bank(w, s, b, experts) -> Bank:
    import torch

    sel = list(int(e) for e in experts)
    wn = w.view(torch.int32)[sel].cpu().numpy().view(np.uint32)
    return Bank(wn, s[sel].float().cpu().numpy(), b[sel].float().cpu().numpy(), "affine", 64)


@pytest.fixture(scope="module")
def deepseek_layer(dev):
    import torch

    from zmlx_amd.layer import QuantizedMoELayer, QuantProj

    rng = np.random.default_rng(7168)
    gen = torch.Generator(device=dev)
    gen.manual_seed(2048)
    mats = {n: _gpu_bank(gen, dev, E, *shape) for n, shape in (("gate", (I, H)), ("up", (I, H)), ("down", (H, I)))}
    sh = {n: _gpu_bank(gen, dev, 1, *shape) for n, shape in (("gate", (I, H)), ("up", (I, H)), ("down", (H, I)))}
    wr = bf16_randn(rng, (E, H), 0.02)
    bias = (rng.standard_normal(E) * 0.05).astype(np.float32)
    layer = QuantizedMoELayer.for_family(
        "deepseek", to_bf16(wr, dev), *(QuantProj(*mats[n]) for n in ("gate", "up", "down")), top_k=K,
        router_bias=torch.from_numpy(bias).to(dev), n_group=NG, topk_group=TG, routed_scaling_factor=SCALE,
        shared=tuple(QuantProj(t[0][0], t[1][0], t[2][0]) for t in (sh["gate"], sh["up"], sh["down"])))
    return layer, mats, sh, wr, bias, rng


@pytest.mark.parametrize("B, checked", [(1, 1), (64, 3)])
def test_deepseek_v3_full_shape(deepseek_layer, dev, B, checked):
    import torch

    layer, mats, sh, wr, bias, rng = deepseek_layer
    x = bf16_randn(rng, (B, H))
    print(f"deepseek full shape B={B}", flush=True)
    out, idx, w = layer(to_bf16(x, dev), return_routing=True)
    torch.cuda.synchronize()
    assert layer.sync_error() == 0
    idx, w, out = from_dev(idx).astype(np.int64), from_dev(w), from_dev(out)
    # routing of every token against the full router
    logits = O.dense_logits(x, wr)
    w_ref, i_ref = O.deepseek_router_topk_sigmoid(logits, bias, K, NG, TG, SCALE)
    np.testing.assert_array_equal(idx, i_ref)
    np.testing.assert_allclose(w, w_ref, rtol=1e-6, atol=1e-6)
    # outputs of the first tokens through their selected experts
    rows = np.arange(checked)
    experts = np.unique(idx[rows])
    remap = np.searchsorted(experts, idx[rows])
    banks = {n: _host_bank(*mats[n], experts) for n in ("gate", "up", "down")}
    y = O.moe_experts(x[rows], remap, banks["gate"].as_tuple(), banks["up"].as_tuple(), banks["down"].as_tuple())
    ref = O.bf16_round(O.moe_combine(y, w_ref[rows], "fp32_no_fma"))
    shb = {n: _host_bank(*sh[n], [0]) for n in ("gate", "up", "down")}
    ys = O.shared_expert(x[rows], *(tuple(a[0] for a in shb[n].as_tuple()) for n in ("gate", "up", "down")))
    ref = O.bf16_round(ref + ys)
    got = out[rows]
    # reference tolerance (1e-2), or where the terms are large next to the
    # output (8 expert outputs of |y| ~ 3 scaled to sum 2.5, plus the shared
    # expert) the bf16-ulp-scaled bound: every expert output may sit one bf16
    # ulp (2^-7 relative) from the float64 value, and so may the result
    scale = (np.abs(w_ref[rows])[:, :, None] * np.abs(y)).sum(1) + np.abs(ys) + np.abs(ref)
    bound = np.maximum(1e-2 + 1e-2 * np.abs(ref), 2.0**-7 * scale)
    bad = np.abs(got - ref) > bound
    assert not bad.any(), f"{bad.sum()} outputs beyond the bound, max excess {(np.abs(got - ref) - bound).max()}"
    ulp = O.bf16_ulp_diff(got, ref)
    assert (ulp == 0).mean() >= 0.90, f"exact fraction {(ulp == 0).mean():.4f}"
    # every token's output is finite and of the expected scale
    assert np.isfinite(out).all()


@pytest.fixture(scope="module")
def qwen3_layer(dev):
    import torch

    from zmlx_amd.layer import QuantizedMoELayer, QuantProj

    rng = np.random.default_rng(30)
    gen = torch.Generator(device=dev)
    gen.manual_seed(3)
    mats = {n: _gpu_bank(gen, dev, QE, *shape) for n, shape in (("gate", (QI, QH)), ("up", (QI, QH)), ("down", (QH, QI)))}
    wr = bf16_randn(rng, (QE, QH), 0.02)
    layer = QuantizedMoELayer.for_family("qwen3", to_bf16(wr, dev), *(QuantProj(*mats[n]) for n in ("gate", "up", "down")),
                                         top_k=QK)
    return layer, mats, wr, rng


@pytest.mark.parametrize("B, checked", [(1, 1), (4, 4), (16, 4)])
def test_qwen3_30b_a3b_full_shape(qwen3_layer, dev, B, checked):
    import torch

    layer, mats, wr, rng = qwen3_layer
    x = bf16_randn(rng, (B, QH))
    print(f"qwen3 full shape B={B}", flush=True)
    out, idx, w = layer(to_bf16(x, dev), return_routing=True)
    torch.cuda.synchronize()
    assert layer.sync_error() == 0
    idx, w, out = from_dev(idx).astype(np.int64), from_dev(w), from_dev(out)
    logits = O.dense_logits(x, wr)
    p = O.softmax_precise_bf16(logits)
    assert O.topk_is_valid(idx, p, QK).all()
    _, w_ref, _ = O.qwen_gating(logits, QK, True, idx=idx)
    assert O.bf16_ulp_diff(w, w_ref).max() <= 1
    rows = np.arange(checked)
    experts = np.unique(idx[rows])
    remap = np.searchsorted(experts, idx[rows])
    banks = {n: _host_bank(*mats[n], experts) for n in ("gate", "up", "down")}
    y = O.moe_experts(x[rows], remap, banks["gate"].as_tuple(), banks["up"].as_tuple(), banks["down"].as_tuple())
    ref = O.bf16_round(O.moe_combine(y, O.bf16_round(w[rows]), "native"))
    got = out[rows]
    np.testing.assert_allclose(got, ref, atol=1e-2, rtol=1e-2)
    ulp = O.bf16_ulp_diff(got, ref)
    assert (ulp == 0).mean() >= 0.90, f"exact fraction {(ulp == 0).mean():.4f}"
    assert np.isfinite(out).all()


def _zipf_tokens(rng, wr, B, skew=1.1, peak=3.0):
    """B tokens of N(0,1) plus a shared component along the router rows that
    adds a Zipf-skewed logit offset peak * rank^-skew to the experts (ranks
    over a random permutation): imbalanced expert loads, as the bench's
    prefill line (config 4)."""
    w = wr.astype(np.float64)
    rank = np.empty(w.shape[0])
    rank[rng.permutation(w.shape[0])] = np.arange(1, w.shape[0] + 1)
    off = peak * rank ** -skew
    v = ((off / (w * w).sum(1))[:, None] * w).sum(0)
    return O.bf16_round(rng.standard_normal((B, w.shape[1])) + v[None, :]).astype(np.float32)


def test_qwen3_prefill_512_zipf(qwen3_layer, dev):
    """Config 4: 512 Zipf-skewed tokens over all 128 experts through the
    layer's prefill path (pairs sorted by expert, grouped GEMMs on MFMA in
    64-row chunks).  Every token's routing is checked against the full
    router; the outputs of tokens that route to the heaviest expert -- the
    first and last of its rows (its first and last chunk) -- and of two
    others, through their experts read back, against the oracle."""
    import torch

    layer, mats, wr, _ = qwen3_layer
    rng = np.random.default_rng(512)
    B = 512
    x = _zipf_tokens(rng, wr, B)
    print("qwen3 prefill 512 zipf", flush=True)
    out, idx, w = layer(to_bf16(x, dev), return_routing=True)
    torch.cuda.synchronize()
    idx, w, out = from_dev(idx).astype(np.int64), from_dev(w), from_dev(out)
    logits = O.dense_logits(x, wr)
    assert O.topk_is_valid(idx, O.softmax_precise_bf16(logits), QK).all()
    _, w_ref, _ = O.qwen_gating(logits, QK, True, idx=idx)
    assert O.bf16_ulp_diff(w, w_ref).max() <= 1
    loads = np.bincount(idx.reshape(-1), minlength=QE)
    heavy = int(loads.argmax())
    assert loads[heavy] > 3 * 64, f"heaviest expert has only {loads[heavy]} rows (want 4+ chunks of 64)"
    on_heavy = np.nonzero((idx == heavy).any(1))[0]
    rows = np.unique(np.array([on_heavy[0], on_heavy[-1], 1, B // 2]))
    experts = np.unique(idx[rows])
    remap = np.searchsorted(experts, idx[rows])
    banks = {n: _host_bank(*mats[n], experts) for n in ("gate", "up", "down")}
    y = O.moe_experts(x[rows], remap, banks["gate"].as_tuple(), banks["up"].as_tuple(), banks["down"].as_tuple())
    ref = O.bf16_round(O.moe_combine(y, O.bf16_round(w[rows]), "native"))
    got = out[rows]
    np.testing.assert_allclose(got, ref, atol=1e-2, rtol=1e-2)
    ulp = O.bf16_ulp_diff(got, ref)
    assert (ulp == 0).mean() >= 0.90, f"exact fraction {(ulp == 0).mean():.4f}"
    assert np.isfinite(out).all()
