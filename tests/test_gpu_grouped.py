"""GPU parity of the grouped (expert-sorted) MFMA gather_qmm against the
oracle: the same forward-error bound as the GEMV (exact products, fp32
accumulation in another order), for affine g32/g64/g128 and mxfp4, plain and
SwiGLU, with skewed expert loads, empty experts and ragged expert row counts
(not multiples of the 32-row MFMA block)."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import moe_oracle as O
from tests.moe_case import bf16_randn, check_gemv_bound, from_dev, make_bank, qmm_exact, seed_of, to_bf16

pytestmark = pytest.mark.gpu


def _pairs(rng, P, xb, E, skew):
    """Zipf-skewed expert choice (some experts empty, a few heavy)."""
    p = 1.0 / np.arange(1, E + 1) ** skew
    perm = rng.permutation(E)
    rhs = perm[rng.choice(E, size=P, p=p / p.sum())].astype(np.int64)
    lhs = rng.integers(0, xb, P).astype(np.int64)
    return lhs, rhs


@pytest.mark.parametrize("mode,gs", [("affine", 64), ("affine", 32), ("affine", 128), ("mxfp4", 32)])
@pytest.mark.parametrize("N,K,E,P", [(256, 512, 8, 300), (128, 2048, 16, 613)])
def test_grouped_qmm_vs_oracle(dev, mode, gs, N, K, E, P):
    import torch

    from zmlx_amd import ops

    rng = np.random.default_rng(seed_of(f"grouped-{mode}-{gs}-{N}-{K}-{E}-{P}"))
    bank = make_bank(rng, E, N, K, mode=mode, group_size=gs)
    xb = 97
    x = bf16_randn(rng, (xb, K))
    lhs, rhs = _pairs(rng, P, xb, E, 1.1)
    w, s, b = bank.torch(dev)
    out = ops.gather_qmm_grouped(to_bf16(x, dev), w, s, b, torch.from_numpy(lhs).to(dev),
                                 torch.from_numpy(rhs).to(dev), group_size=gs, mode=mode)
    torch.cuda.synchronize()
    exact, absd = qmm_exact(x[:, None, :], bank, lhs, rhs)
    check_gemv_bound(from_dev(out), exact[:, 0, :], absd[:, 0, :])


@pytest.mark.parametrize("mode,gs", [("affine", 64), ("mxfp4", 32)])
def test_grouped_swiglu_vs_oracle(dev, mode, gs):
    import torch

    from zmlx_amd import ops

    rng = np.random.default_rng(seed_of(f"grouped-swiglu-{mode}"))
    E, I, H, B, K = 16, 256, 1024, 64, 4
    gate = make_bank(rng, E, I, H, mode=mode, group_size=gs)
    up = make_bank(rng, E, I, H, mode=mode, group_size=gs)
    x = bf16_randn(rng, (B, H))
    rhs = np.stack([rng.choice(E, K, replace=False) for _ in range(B)]).reshape(-1)
    lhs = np.repeat(np.arange(B), K)
    gw, gsc, gb = gate.torch(dev)
    uw, usc, ub = up.torch(dev)
    out = ops.gather_qmm_grouped(to_bf16(x, dev), gw, gsc, gb, torch.from_numpy(lhs).to(dev),
                                 torch.from_numpy(rhs).to(dev), up=(uw, usc, ub), group_size=gs, mode=mode)
    torch.cuda.synchronize()
    ref = O.gather_qmm_swiglu(x[:, None, :], *gate.as_tuple(), *up.as_tuple(), lhs, rhs, group_size=gs,
                              mode=mode)[:, 0, :]
    got = from_dev(out)
    np.testing.assert_allclose(got, ref, atol=1e-2, rtol=1e-2)
    assert (O.bf16_ulp_diff(got, ref) == 0).mean() >= 0.97


def test_grouped_matches_gemv_path(dev):
    """Grouped MFMA vs the GEMV kernel on the same pairs: both sit within the
    forward-error bound of the same exact value, so they differ by at most the
    sum of the two bounds, and are almost always identical."""
    import torch

    from zmlx_amd import ops

    rng = np.random.default_rng(5)
    E, N, K, B, k = 8, 512, 2048, 32, 2
    bank = make_bank(rng, E, N, K)
    x = bf16_randn(rng, (B, K))
    rhs = np.stack([rng.choice(E, k, replace=False) for _ in range(B)])
    w, s, b = bank.torch(dev)
    xt = to_bf16(x, dev)
    ridx = torch.from_numpy(rhs).to(dev)
    lidx = torch.from_numpy(np.repeat(np.arange(B), k)).to(dev)
    g = ops.gather_qmm_grouped(xt, w, s, b, lidx, ridx.reshape(-1))
    v = ops.gather_qmm(xt[:, None, :], w, s, b, lhs_indices=lidx, rhs_indices=ridx.reshape(-1)).reshape(B * k, N)
    torch.cuda.synchronize()
    gv, vv = from_dev(g).astype(np.float64), from_dev(v).astype(np.float64)
    _, absd = qmm_exact(x[:, None, :], bank, np.repeat(np.arange(B), k), rhs.reshape(-1))
    ulp = np.ldexp(1.0, np.frexp(np.maximum(np.maximum(np.abs(gv), np.abs(vv)), 2.0**-126))[1] - 8)
    assert (np.abs(gv - vv) <= ulp + 2.0**-15 * absd[:, 0, :]).all()
    assert (gv == vv).mean() >= 0.97
