"""GPU parity: combine kernels, bit-exact against the oracle in every mode.

Pins: tests/test_fused_ops.py:349-362 (no-FMA combine array_equal to MLX's
(eo*w[...,None]).sum(-2).astype(dtype)), moe.py:830-1127 (mode semantics),
moe.py:1820-1921 (streaming weighted accumulate)."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import moe_oracle as O
from tests.moe_case import bf16_randn, from_dev, to_bf16

pytestmark = pytest.mark.gpu

MODES = {
    "fp32_no_fma": "moe_combine_fp32_no_fma",
    "fp32": "moe_combine_fp32",
    "exact": "moe_combine_exact",
    "no_fma": "moe_combine_no_fma",
    "float": "moe_combine",
}


@pytest.mark.parametrize("B,K,D", [(1, 8, 2048), (3, 4, 64), (16, 8, 2048), (2, 1, 100), (5, 6, 7168)])
@pytest.mark.parametrize("mode", list(MODES) + ["native"])
def test_combine_bit_exact(dev, B, K, D, mode):
    import torch

    import zmlx_amd as Z

    rng = np.random.default_rng(B * 100 + K)
    y = bf16_randn(rng, (B, K, D))
    if mode in ("fp32", "fp32_no_fma", "no_fma", "float"):
        w = rng.standard_normal((B, K)).astype(np.float32)
        wt = torch.from_numpy(w).to(dev)
    else:
        w = bf16_randn(rng, (B, K))
        wt = to_bf16(w, dev)
    if mode == "native":
        got = Z.moe_combine(to_bf16(y, dev), wt, native=True)
    else:
        got = getattr(Z, MODES[mode])(to_bf16(y, dev), wt)
    torch.cuda.synchronize()
    ref = O.moe_combine(y, w, mode)
    np.testing.assert_array_equal(from_dev(got), ref)


def test_combine_no_fma_matches_mlx_semantics(dev):
    """(eo*w[...,None]).sum(-2) with f32 weights evaluated as f32 products
    then an ordered f32 sum, cast to bf16 == moe_combine_no_fma."""
    import torch

    import zmlx_amd as Z

    rng = np.random.default_rng(0)
    B, K, D = 3, 4, 64
    w = rng.standard_normal((B, K)).astype(np.float32)
    eo = bf16_randn(rng, (B, K, D))
    prods = (eo * w[..., None]).astype(np.float32)
    acc = np.zeros((B, D), np.float32)
    for k in range(K):
        acc = (acc + prods[:, k]).astype(np.float32)
    ref = O.bf16_round(acc)
    got = Z.moe_combine_no_fma(to_bf16(eo, dev), torch.from_numpy(w).to(dev))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(from_dev(got), ref)


@pytest.mark.parametrize("no_fma", [False, True])
@pytest.mark.parametrize("fp32", [False, True])
def test_weighted_accumulate(dev, no_fma, fp32):
    import torch

    import zmlx_amd as Z

    rng = np.random.default_rng(4)
    B, D = 3, 2048
    acc = rng.standard_normal((B, D)).astype(np.float32)
    if not fp32:
        acc = O.bf16_round(acc)
    proj = bf16_randn(rng, (B, D))
    g = rng.standard_normal(B).astype(np.float32)
    acc_t = torch.from_numpy(acc).to(dev)
    if not fp32:
        acc_t = acc_t.to(torch.bfloat16)
    got = Z.weighted_accumulate(acc_t, to_bf16(proj, dev), torch.from_numpy(g).to(dev), no_fma=no_fma)
    torch.cuda.synchronize()
    ref = O.weighted_accumulate(acc, proj, g, no_fma=no_fma, fp32_out=fp32)
    np.testing.assert_array_equal(from_dev(got), ref)


def test_gather_qmm_combine_quantized_streaming_vs_vectorized(dev):
    """test_gather_qmm_combine.py:182-207: streaming == non-streaming within
    tolerance; and both against the oracle (down-proj then combine)."""
    import torch

    import zmlx_amd as Z
    from tests.moe_case import make_bank

    rng = np.random.default_rng(9)
    E, B, K, Din, Dout = 8, 2, 4, 512, 256
    bank = make_bank(rng, E, Dout, Din)
    act = bf16_randn(rng, (B, K, Din))
    idx = rng.integers(0, E, (B, K))
    gate = rng.random((B, K)).astype(np.float32)
    w, s, b = bank.torch(dev)
    a_t = to_bf16(act, dev)
    i_t = torch.tensor(idx, dtype=torch.int32, device=dev)
    g_t = torch.from_numpy(gate).to(dev)
    out_s = Z.gather_qmm_combine_quantized(a_t, w, s, b, g_t, i_t, streaming=True, no_fma=True,
                                           output_dtype=torch.float32)
    out_v = Z.gather_qmm_combine_quantized(a_t, w, s, b, g_t, i_t, streaming=False, no_fma=True,
                                           output_dtype=torch.float32)
    torch.cuda.synchronize()
    proj = O.gather_qmm(act.reshape(B * K, 1, Din), bank.w, bank.s, bank.b, np.arange(B * K),
                        idx.reshape(-1)).reshape(B, K, Dout)
    ref = O.moe_combine(proj, gate, "fp32_no_fma")
    # a projection may sit 1 bf16 ulp from the float64 oracle (fp32 GEMV
    # accumulation); the reference's quantized tolerance is 5e-3 (:434-522)
    np.testing.assert_allclose(from_dev(out_s), ref, rtol=5e-3, atol=5e-3)
    # streaming (ordered no-FMA accumulate) and vectorized (no-FMA combine)
    # evaluate the same f32 operation sequence: bit-identical
    np.testing.assert_array_equal(from_dev(out_s), from_dev(out_v))
    # and exact against the oracle combine of the GPU's own projections
    proj_gpu = Z.gather_qmm(a_t.reshape(B * K, 1, Din), w, s, b,
                            lhs_indices=torch.arange(B * K, device=dev, dtype=torch.int32).reshape(B, K),
                            rhs_indices=i_t).reshape(B, K, Dout)
    np.testing.assert_array_equal(from_dev(out_v), O.moe_combine(from_dev(proj_gpu), gate, "fp32_no_fma"))
