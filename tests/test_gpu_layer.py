"""GPU parity: the whole MoE block (zmoe_moe_layer) vs the oracle composition.

Per stage the oracle is fed the GPU's previous-stage decision where MLX's own
choice is unspecified (the top-k order inside a bf16 tie set), and checked:
routing = valid top-k of the oracle's probabilities; weights within 1 bf16
ulp; layer output within the reference tolerance (1e-2) and mostly
bit-identical.  Configs are the BASELINE shapes at small expert counts
(the per-expert shapes are the real ones)."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import moe_oracle as O
from tests.moe_case import bf16_randn, from_dev, make_bank, to_bf16

pytestmark = pytest.mark.gpu


def _build(dev, rng, *, H, E, I, K, mode="affine", gs=64, shared_I=0, router_std=0.02):
    import torch

    from zmlx_amd.layer import QuantProj

    banks = {n: make_bank(rng, E, *(shape), mode=mode, group_size=gs)
             for n, shape in (("gate", (I, H)), ("up", (I, H)), ("down", (H, I)))}
    wr = bf16_randn(rng, (E, H), router_std)
    sh = None
    if shared_I:
        sh = {n: make_bank(rng, 1, *(shape), mode=mode, group_size=gs)
              for n, shape in (("gate", (shared_I, H)), ("up", (shared_I, H)), ("down", (H, shared_I)))}

    def qp(bank, squeeze=False):
        w, s, b = bank.torch(dev)
        if squeeze:
            w, s = w[0], s[0]
            b = None if b is None else b[0]
        return QuantProj(w, s, b)

    tq = {n: qp(b) for n, b in banks.items()}
    tsh = None if sh is None else tuple(qp(sh[n], True) for n in ("gate", "up", "down"))
    return banks, wr, sh, tq, tsh, to_bf16(wr, dev)


def _oracle_out(x, idx, w, banks, sh, mode, gs, combine):
    y = O.moe_experts(x, idx, banks["gate"].as_tuple(), banks["up"].as_tuple(), banks["down"].as_tuple(),
                      group_size=gs, mode=mode)
    out = O.moe_combine(y, w, combine)
    out = O.bf16_round(out)
    if sh is not None:
        ys = O.shared_expert(x, tuple(a[0] if a is not None else None for a in sh["gate"].as_tuple()),
                             tuple(a[0] if a is not None else None for a in sh["up"].as_tuple()),
                             tuple(a[0] if a is not None else None for a in sh["down"].as_tuple()),
                             group_size=gs, mode=mode)
        out = O.bf16_round(out + ys)
    return out


def _cmp_out(got, ref):
    """Reference tolerance (1e-2, test_gather_qmm_swiglu.py:84-85) and >= 90%
    bit-identical: each output mixes K expert outputs, each of which may sit
    one bf16 ulp from the float64 oracle (fp32 GEMV accumulation), so a few
    percent of outputs legitimately differ in the last bit."""
    np.testing.assert_allclose(got, ref, atol=1e-2, rtol=1e-2)
    ulp = O.bf16_ulp_diff(got, ref)
    assert (ulp == 0).mean() >= 0.90, f"exact fraction {(ulp == 0).mean():.4f}"


@pytest.mark.parametrize("B", [1, 4, 16])
def test_layer_qwen3_shape(dev, B):
    """Qwen3-30B-A3B per-expert shapes (H 2048, I 768, top-8), 32 experts."""
    import torch

    from zmlx_amd.layer import QuantizedMoELayer

    rng = np.random.default_rng(100 + B)
    H, E, I, K = 2048, 32, 768, 8
    banks, wr, sh, tq, tsh, wr_t = _build(dev, rng, H=H, E=E, I=I, K=K)
    layer = QuantizedMoELayer.for_family("qwen3", wr_t, tq["gate"], tq["up"], tq["down"], top_k=K)
    x = bf16_randn(rng, (B, H))
    out, idx, w = layer(to_bf16(x, dev), return_routing=True)
    torch.cuda.synchronize()
    idx = from_dev(idx).astype(np.int64)
    logits = O.dense_logits(x, wr)
    p = O.softmax_precise_bf16(logits)
    assert O.topk_is_valid(idx, p, K).all()
    _, w_ref, _ = O.qwen_gating(logits, K, True, idx=idx)
    assert O.bf16_ulp_diff(from_dev(w), w_ref).max() <= 1
    ref = _oracle_out(x, idx, O.bf16_round(from_dev(w)), banks, None, "affine", 64, "native")
    _cmp_out(from_dev(out), ref)


def test_layer_lfm2_shape(dev):
    """LFM2-8B-A1B shapes: H 2048, 32 experts, top-4, I 1792 (config 1)."""
    import torch

    from zmlx_amd.layer import QuantizedMoELayer

    rng = np.random.default_rng(7)
    H, E, I, K = 2048, 32, 1792, 4
    banks, wr, sh, tq, tsh, wr_t = _build(dev, rng, H=H, E=E, I=I, K=K)
    layer = QuantizedMoELayer.for_family("lfm2", wr_t, tq["gate"], tq["up"], tq["down"], top_k=K)
    x = bf16_randn(rng, (1, H))
    out, idx, w = layer(to_bf16(x, dev), return_routing=True)
    torch.cuda.synchronize()
    idx = from_dev(idx).astype(np.int64)
    logits = O.dense_logits(x, wr)
    assert O.topk_is_valid(idx, logits, K).all()
    w_ref, _ = O.topk_gating_softmax(logits, K, None, True, idx=idx)
    np.testing.assert_array_equal(from_dev(w), O.bf16_round(w_ref))
    ref = _oracle_out(x, idx, O.bf16_round(w_ref), banks, None, "affine", 64, "native")
    _cmp_out(from_dev(out), ref)


@pytest.mark.parametrize("B", [1, 8])
def test_layer_glm_mxfp4_shared(dev, B):
    """GLM-4.7-Flash-like: 64 experts top-4 sigmoid + bias, shared expert,
    I 1536, mxfp4, fp32 no-FMA combine (config 3)."""
    import torch

    from zmlx_amd.layer import QuantizedMoELayer

    rng = np.random.default_rng(300 + B)
    H, E, I, K = 2048, 64, 1536, 4
    banks, wr, sh, tq, tsh, wr_t = _build(dev, rng, H=H, E=E, I=I, K=K, mode="mxfp4", gs=32, shared_I=1536)
    bias = (rng.standard_normal(E) * 0.05).astype(np.float32)
    layer = QuantizedMoELayer.for_family("glm", wr_t, tq["gate"], tq["up"], tq["down"], top_k=K,
                                         router_bias=torch.from_numpy(bias).to(dev), group_size=32, mode="mxfp4",
                                         routed_scaling_factor=1.8, shared=tsh)
    x = bf16_randn(rng, (B, H))
    out, idx, w = layer(to_bf16(x, dev), return_routing=True)
    torch.cuda.synchronize()
    logits = O.dense_logits(x, wr)
    w_ref, i_ref = O.deepseek_router_topk_sigmoid(logits, bias, K, 1, 1, 1.8)
    np.testing.assert_array_equal(from_dev(idx), i_ref)
    np.testing.assert_allclose(from_dev(w), w_ref, rtol=1e-6, atol=1e-7)
    ref = _oracle_out(x, i_ref, w_ref, banks, sh, "mxfp4", 32, "fp32_no_fma")
    _cmp_out(from_dev(out), ref)


@pytest.mark.parametrize("B", [32, 64])
def test_layer_prefill_grouped_qwen3(dev, B):
    """Prefill-sized batches (>= 32 tokens) run the routed experts as grouped
    GEMMs on MFMA (pairs sorted by expert): Qwen3 per-expert shapes, 32
    experts, checked against the oracle like the decode batches."""
    import torch

    from zmlx_amd.layer import QuantizedMoELayer

    rng = np.random.default_rng(500 + B)
    H, E, I, K = 2048, 32, 768, 8
    banks, wr, sh, tq, tsh, wr_t = _build(dev, rng, H=H, E=E, I=I, K=K)
    layer = QuantizedMoELayer.for_family("qwen3", wr_t, tq["gate"], tq["up"], tq["down"], top_k=K)
    x = bf16_randn(rng, (B, H))
    out, idx, w = layer(to_bf16(x, dev), return_routing=True)
    torch.cuda.synchronize()
    idx = from_dev(idx).astype(np.int64)
    logits = O.dense_logits(x, wr)
    assert O.topk_is_valid(idx, O.softmax_precise_bf16(logits), K).all()
    _, w_ref, _ = O.qwen_gating(logits, K, True, idx=idx)
    assert O.bf16_ulp_diff(from_dev(w), w_ref).max() <= 1
    ref = _oracle_out(x, idx, O.bf16_round(from_dev(w)), banks, None, "affine", 64, "native")
    _cmp_out(from_dev(out), ref)


def test_layer_prefill_grouped_glm_mxfp4_shared(dev):
    """Grouped MFMA experts with mxfp4 weights, the sigmoid router and the
    shared expert at a prefill-sized batch (40 tokens)."""
    import torch

    from zmlx_amd.layer import QuantizedMoELayer

    rng = np.random.default_rng(640)
    H, E, I, K, B = 2048, 64, 1536, 4, 40
    banks, wr, sh, tq, tsh, wr_t = _build(dev, rng, H=H, E=E, I=I, K=K, mode="mxfp4", gs=32, shared_I=1536)
    bias = (rng.standard_normal(E) * 0.05).astype(np.float32)
    layer = QuantizedMoELayer.for_family("glm", wr_t, tq["gate"], tq["up"], tq["down"], top_k=K,
                                         router_bias=torch.from_numpy(bias).to(dev), group_size=32, mode="mxfp4",
                                         routed_scaling_factor=1.8, shared=tsh)
    x = bf16_randn(rng, (B, H))
    out, idx, w = layer(to_bf16(x, dev), return_routing=True)
    torch.cuda.synchronize()
    logits = O.dense_logits(x, wr)
    w_ref, i_ref = O.deepseek_router_topk_sigmoid(logits, bias, K, 1, 1, 1.8)
    np.testing.assert_array_equal(from_dev(idx), i_ref)
    ref = _oracle_out(x, i_ref, w_ref, banks, sh, "mxfp4", 32, "fp32_no_fma")
    _cmp_out(from_dev(out), ref)


def test_layer_deepseek_grouped(dev):
    """DeepSeek-V3 routing (256 experts, 8 groups, top-4 groups, top-8,
    scale 2.5) with reduced H/I for oracle speed; shared expert."""
    import torch

    from zmlx_amd.layer import QuantizedMoELayer

    rng = np.random.default_rng(42)
    H, E, I, K = 1024, 256, 256, 8
    banks, wr, sh, tq, tsh, wr_t = _build(dev, rng, H=H, E=E, I=I, K=K, shared_I=512)
    bias = (rng.standard_normal(E) * 0.05).astype(np.float32)
    layer = QuantizedMoELayer.for_family("deepseek", wr_t, tq["gate"], tq["up"], tq["down"], top_k=K,
                                         router_bias=torch.from_numpy(bias).to(dev), n_group=8, topk_group=4,
                                         routed_scaling_factor=2.5, shared=tsh)
    x = bf16_randn(rng, (3, H))
    out, idx, w = layer(to_bf16(x, dev), return_routing=True)
    torch.cuda.synchronize()
    logits = O.dense_logits(x, wr)
    w_ref, i_ref = O.deepseek_router_topk_sigmoid(logits, bias, K, 8, 4, 2.5)
    np.testing.assert_array_equal(from_dev(idx), i_ref)
    np.testing.assert_allclose(from_dev(w), w_ref, rtol=1e-6, atol=1e-6)
    ref = _oracle_out(x, i_ref, w_ref, banks, sh, "affine", 64, "fp32_no_fma")
    _cmp_out(from_dev(out), ref)


def test_layer_zero_input_gives_zero(dev):
    """x = 0 => logits 0 => every expert output is exactly 0 (g = u = 0)."""
    import torch

    from zmlx_amd.layer import QuantizedMoELayer

    rng = np.random.default_rng(1)
    H, E, I, K = 2048, 16, 768, 8
    banks, wr, sh, tq, tsh, wr_t = _build(dev, rng, H=H, E=E, I=I, K=K)
    layer = QuantizedMoELayer.for_family("qwen3", wr_t, tq["gate"], tq["up"], tq["down"], top_k=K)
    out, idx, w = layer(torch.zeros((2, H), dtype=torch.bfloat16, device=dev), return_routing=True)
    torch.cuda.synchronize()
    assert (from_dev(out) == 0).all()
    # uniform probabilities: lowest 8 indices, weights 1/8 each
    assert (from_dev(idx) == np.arange(8)).all()
    np.testing.assert_array_equal(from_dev(w), np.full((2, 8), 0.125, np.float32))


def _layer_pair(dev, rng, family, *, H, E, I, K, mode="affine", gs=64, shared_I=0, **kw):
    """The same layer built twice: single-launch kernel and kernel sequence."""
    import torch

    from zmlx_amd.layer import QuantizedMoELayer

    banks, wr, sh, tq, tsh, wr_t = _build(dev, rng, H=H, E=E, I=I, K=K, mode=mode, gs=gs, shared_I=shared_I)
    if "router_bias" in kw and kw["router_bias"] is not None:
        kw["router_bias"] = torch.from_numpy(kw["router_bias"]).to(dev)
    mk = lambda single: QuantizedMoELayer.for_family(  # noqa: E731
        family, wr_t, tq["gate"], tq["up"], tq["down"], top_k=K, group_size=gs, mode=mode, shared=tsh,
        single_launch=single, **kw)
    return mk(True), mk(False)


FUSED_CASES = [
    ("qwen3", dict(H=2048, E=128, I=768, K=8), [1, 2, 4, 8, 16, 5]),
    # one-token kernel with units other than 8; shared expert with batches
    # (k_moe_decodeb)
    ("qwen3_k6", dict(H=2048, E=64, I=768, K=6), [1, 3, 16]),
    ("qwen3_shared", dict(H=2048, E=64, I=768, K=8, shared_I=768), [1, 2, 4, 3]),
    ("lfm2", dict(H=2048, E=32, I=1792, K=4), [1, 3, 16]),
    ("glm", dict(H=2048, E=64, I=1536, K=4, mode="mxfp4", gs=32, shared_I=1536), [1, 8, 16, 2]),
    ("deepseek", dict(H=1024, E=256, I=512, K=8, shared_I=512), [1, 2]),
    # hidden sizes other than 2048 take the one-token kernel's general path
    ("glm_h3072", dict(H=3072, E=64, I=1024, K=4, mode="mxfp4", gs=32, shared_I=1024), [1]),
    ("qwen3_h4096", dict(H=4096, E=64, I=1536, K=8), [1]),
]


@pytest.mark.parametrize("family,shape,batches", FUSED_CASES, ids=[c[0] for c in FUSED_CASES])
def test_single_launch_matches_kernel_sequence(dev, family, shape, batches):
    """The persistent single-launch layer kernel evaluates the same arithmetic
    as the kernel sequence: outputs and routing bit-identical, for repeated
    calls (barrier counters reset themselves) and ragged batch sizes."""
    import torch

    rng = np.random.default_rng(17)
    kw = {}
    family = family.split("_")[0]
    if family in ("glm", "deepseek"):
        kw["router_bias"] = (rng.standard_normal(shape["E"]) * 0.05).astype(np.float32)
        kw["routed_scaling_factor"] = 2.5
    if family == "deepseek":
        kw.update(n_group=8, topk_group=4)
    fused, multi = _layer_pair(dev, rng, family, **shape, **kw)
    for B in batches:
        x = to_bf16(bf16_randn(rng, (B, shape["H"])), dev)
        for rep in range(3):
            of, i_f, w_f = fused(x, return_routing=True)
            om, i_m, w_m = multi(x, return_routing=True)
            torch.cuda.synchronize()
            np.testing.assert_array_equal(from_dev(i_f), from_dev(i_m))
            np.testing.assert_array_equal(from_dev(w_f), from_dev(w_m))
            np.testing.assert_array_equal(from_dev(of), from_dev(om))
    assert fused.sync_error() == 0


@pytest.mark.parametrize("family,shape,batches", [
    ("qwen3", dict(H=2048, E=128, I=768, K=8), [16, 5, 2]),
    ("glm", dict(H=2048, E=64, I=1536, K=4, mode="mxfp4", gs=32, shared_I=1536), [8, 3]),
    ("lfm2", dict(H=2048, E=32, I=1792, K=4), [6]),
])
def test_batch_rows_match_single_tokens(dev, family, shape, batches):
    """Each token's output is computed with the same arithmetic whatever the
    batch's path (chunked or per-pair GEMV sequence, batched or one-token
    single-launch kernel): a batch's rows are bit-identical to one-token calls
    on each row, routing included."""
    import torch

    rng = np.random.default_rng(41)
    kw = {}
    if family == "glm":
        kw["router_bias"] = (rng.standard_normal(shape["E"]) * 0.05).astype(np.float32)
        kw["routed_scaling_factor"] = 1.8
    layer, _ = _layer_pair(dev, rng, family, **shape, **kw)
    for B in batches:
        print(f"[rows] {family} B={B}", flush=True)
        x = to_bf16(bf16_randn(rng, (B, shape["H"])), dev)
        ob, ib, wb = layer(x, return_routing=True)
        rows = [layer(x[b:b + 1], return_routing=True) for b in range(B)]
        torch.cuda.synchronize()
        np.testing.assert_array_equal(from_dev(ib), np.concatenate([from_dev(r[1]) for r in rows]))
        np.testing.assert_array_equal(from_dev(wb), np.concatenate([from_dev(r[2]) for r in rows]))
        np.testing.assert_array_equal(from_dev(ob), np.concatenate([from_dev(r[0]) for r in rows]))
    assert layer.sync_error() == 0


@pytest.mark.parametrize("family,shape,groups", [
    ("deepseek", dict(H=1024, E=256, I=512, K=8, shared_I=512), dict(n_group=8, topk_group=4)),
    ("glm", dict(H=2048, E=64, I=1536, K=4, mode="mxfp4", gs=32, shared_I=1536), {}),
])
def test_single_launch_routing_ties(dev, family, shape, groups):
    """Grouped sigmoid routing with tied scores (zero input, bias on a coarse
    grid): the single-launch kernel ranks fp32 keys with ties to the lower
    index and keeps the same groups as the argmax rounds of the kernel
    sequence; routing and outputs bit-identical."""
    import torch

    rng = np.random.default_rng(23)
    bias = (rng.integers(-2, 3, shape["E"]) * 0.25).astype(np.float32)
    fused, multi = _layer_pair(dev, rng, family, **shape, router_bias=bias, routed_scaling_factor=2.5, **groups)
    xs = [np.zeros((1, shape["H"]), np.float32), bf16_randn(rng, (1, shape["H"]))]
    for x in xs:
        xt = to_bf16(x, dev)
        of, i_f, w_f = fused(xt, return_routing=True)
        om, i_m, w_m = multi(xt, return_routing=True)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(from_dev(i_f), from_dev(i_m))
        np.testing.assert_array_equal(from_dev(w_f), from_dev(w_m))
        np.testing.assert_array_equal(from_dev(of), from_dev(om))
    assert fused.sync_error() == 0


def test_single_launch_softmax_tie_order(dev):
    """Softmax routing where the bf16 probabilities tie although the logits
    differ: the ranking (bf16 probability, then lower index) differs from
    plain logit order; the single-launch kernel's routing and outputs are
    those of the kernel sequence (bit-identical) and a valid top-k of the
    oracle's probabilities."""
    import torch

    from zmlx_amd.layer import QuantizedMoELayer

    rng = np.random.default_rng(29)
    H, E, I, K = 2048, 128, 768, 8
    banks, wr, sh, tq, tsh, _ = _build(dev, rng, H=H, E=E, I=I, K=K)
    # logits = wr[:, 0] for x = e_0: distinct, within 1.3e-2 of each other,
    # larger for higher indices; probabilities tie in bf16 in runs
    wr = np.zeros((E, H), np.float32)
    wr[:, 0] = ((np.arange(E) * 37) % E) * 1e-4
    wr_t = to_bf16(wr, dev)
    logits = O.bf16_round(wr[:, 0])
    probs = O.softmax_precise_bf16(logits)
    by_logit = np.argsort(-logits, kind="stable")[:K]
    by_prob = O.topk_desc(probs, K)
    assert set(by_logit) != set(by_prob)  # logit order would route differently
    mk = lambda single: QuantizedMoELayer.for_family(  # noqa: E731
        "qwen3", wr_t, tq["gate"], tq["up"], tq["down"], top_k=K, single_launch=single)
    fused, multi = mk(True), mk(False)
    x = np.zeros((1, H), np.float32)
    x[0, 0] = 1.0
    xt = to_bf16(x, dev)
    for rep in range(2):
        of, i_f, w_f = fused(xt, return_routing=True)
        om, i_m, w_m = multi(xt, return_routing=True)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(from_dev(i_f), from_dev(i_m))
        assert O.topk_is_valid(from_dev(i_f)[0], probs, K)
        np.testing.assert_array_equal(from_dev(w_f), from_dev(w_m))
        np.testing.assert_array_equal(from_dev(of), from_dev(om))
    assert fused.sync_error() == 0


@pytest.mark.parametrize("mode,gs", [("affine", 64), ("mxfp4", 32)])
def test_layer_expert_major_gemv(dev, mode, gs):
    """12 tokens over 16 experts (about 3 rows each): the kernel sequence runs
    the expert-major GEMV; hidden 1536 gives 3 segment steps per gate/up row
    and I 768 three per down row (several load-ring items per row)."""
    import torch

    from zmlx_amd.layer import QuantizedMoELayer

    rng = np.random.default_rng(77)
    H, E, I, K, B = 1536, 16, 768, 4, 12
    banks, wr, sh, tq, tsh, wr_t = _build(dev, rng, H=H, E=E, I=I, K=K, mode=mode, gs=gs)
    layer = QuantizedMoELayer.for_family("qwen3", wr_t, tq["gate"], tq["up"], tq["down"], top_k=K, group_size=gs,
                                         mode=mode)
    x = bf16_randn(rng, (B, H))
    out, idx, w = layer(to_bf16(x, dev), return_routing=True)
    torch.cuda.synchronize()
    idx = from_dev(idx).astype(np.int64)
    ref = _oracle_out(x, idx, O.bf16_round(from_dev(w)), banks, None, mode, gs, "native")
    _cmp_out(from_dev(out), ref)


@pytest.mark.parametrize("family,shape,B", [
    ("qwen3", dict(H=2048, E=32, I=768, K=8), 1),     # XCD-partitioned one-token kernel
    ("lfm2", dict(H=2048, E=32, I=1792, K=4), 1),     # the same, two XCDs per unit
    ("qwen3", dict(H=2048, E=32, I=768, K=4), 1),     # one-token kernel (grid-wide exchanges)
    ("glm", dict(H=2048, E=64, I=1536, K=4, mode="mxfp4", gs=32, shared_I=1536), 1),  # XCD kernel, 3 idle XCDs
    ("qwen3", dict(H=2048, E=32, I=768, K=8, shared_I=768), 4),  # batched kernel (shared expert)
])
def test_wait_give_up_is_loud(dev, family, shape, B):
    """A single-launch kernel whose cross-workgroup wait gives up (forced from
    the host with a spin limit of one poll, so every kernel still exits
    normally) leaves NaN in the outputs it could not compute, sets the sticky
    error word, and the next call raises ZmoeError.  Afterwards the layer
    computes normally again (bit-identical to the kernel sequence)."""
    import torch

    from zmlx_amd import ZmoeError
    from zmlx_amd import _native as N
    from zmlx_amd.layer import QuantizedMoELayer

    rng = np.random.default_rng(31)
    banks, wr, sh, tq, tsh, wr_t = _build(dev, rng, **shape)
    kw = {}
    if family == "glm":
        bias = (rng.standard_normal(shape["E"]) * 0.05).astype(np.float32)
        kw = dict(router_bias=torch.from_numpy(bias).to(dev), group_size=shape["gs"], mode=shape["mode"],
                  routed_scaling_factor=1.8)
    layer = QuantizedMoELayer.for_family(family, wr_t, tq["gate"], tq["up"], tq["down"], top_k=shape["K"], shared=tsh,
                                         **kw)
    assert layer._single_launch(B)
    x = to_bf16(bf16_randn(rng, (B, shape["H"])), dev)
    print(f"[give-up] {family} B={B}", flush=True)
    layer.desc.spin_limit = 1
    out = layer(x)
    torch.cuda.synchronize()
    assert torch.isnan(out.float()).any(), "a wait that gave up left no NaN in the output"
    assert layer.sync_error() != 0
    assert layer._err_flag[0] == 1
    layer.desc.spin_limit = 0
    with pytest.raises(ZmoeError):
        layer(x)
    assert layer.sync_error() == 0  # the workspaces were cleared
    got = layer(x)
    layer.desc.flags |= N.LAYER_FORCE_MULTI
    ref = layer(x)
    layer.desc.flags &= ~N.LAYER_FORCE_MULTI
    torch.cuda.synchronize()
    assert layer.sync_error() == 0
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
