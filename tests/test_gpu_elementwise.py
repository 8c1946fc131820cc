"""GPU parity: swiglu2 (transformer.py:882-935) and moe_dispatch
(moe.py:776-827) against the oracle.

Pins: the reference's own swiglu2 test (tests/test_fused_ops.py:69-83:
float32 inputs, rtol 1e-4 against the float64 formula); the oracle's
swiglu / swiglu2 / dispatch functions are pinned in test_oracle_pins.py."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import moe_oracle as O
from tests.moe_case import bf16_randn, from_dev, to_bf16

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("shape", [(2, 8), (4, 64), (3, 5, 768), (1, 1), (0, 16)])
def test_swiglu2_f32(dev, shape):
    import torch

    import zmlx_amd as Z

    rng = np.random.default_rng(11)
    g = (rng.standard_normal(shape) * 3).astype(np.float32)
    u = rng.standard_normal(shape).astype(np.float32)
    y = Z.swiglu2(torch.from_numpy(g).to(dev), torch.from_numpy(u).to(dev))
    torch.cuda.synchronize()
    assert tuple(y.shape) == shape
    got = y.cpu().numpy()
    # the reference test's check, then the f32 oracle
    ref64 = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    np.testing.assert_allclose(got, ref64, rtol=1e-4, atol=1e-6)
    np.testing.assert_allclose(got, O.swiglu2_f32(g, u), rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("shape", [(2, 8), (16, 2048), (7, 1536)])
def test_swiglu2_bf16(dev, shape):
    """bf16 inputs: MLX's op-by-op rounding of nn.silu(g) * u; the sigmoid
    may sit one bf16 ulp from the correctly rounded one, so at most one ulp
    per output and almost all outputs exact."""
    import torch

    import zmlx_amd as Z

    rng = np.random.default_rng(12)
    g, u = bf16_randn(rng, shape), bf16_randn(rng, shape)
    y = Z.swiglu2(to_bf16(g, dev), to_bf16(u, dev))
    torch.cuda.synchronize()
    got = from_dev(y)
    ref = O.swiglu(g, u)
    ulp = O.bf16_ulp_diff(got, ref)
    assert ulp.max() <= 1
    assert (ulp == 0).mean() >= 0.98


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_swiglu2_backward(dev, dtype):
    import torch

    import zmlx_amd as Z

    rng = np.random.default_rng(13)
    shape = (6, 300)
    if dtype == "f32":
        g = (rng.standard_normal(shape) * 3).astype(np.float32)
        u = rng.standard_normal(shape).astype(np.float32)
        c = rng.standard_normal(shape).astype(np.float32)
        mk = lambda a: torch.from_numpy(a).to(dev).requires_grad_(True)  # noqa: E731
        tol = dict(rtol=1e-5, atol=1e-6)
    else:
        g, u, c = bf16_randn(rng, shape), bf16_randn(rng, shape), bf16_randn(rng, shape)
        mk = lambda a: to_bf16(a, dev).requires_grad_(True)  # noqa: E731
        tol = dict(rtol=1e-2, atol=1e-2)
    gt, ut = mk(g), mk(u)
    ct = torch.from_numpy(c).to(dev).to(gt.dtype)
    Z.swiglu2(gt, ut).backward(ct)
    torch.cuda.synchronize()
    dg_ref, du_ref = O.swiglu2_backward(g, u, c)
    np.testing.assert_allclose(gt.grad.float().cpu().numpy(), dg_ref, **tol)
    np.testing.assert_allclose(ut.grad.float().cpu().numpy(), du_ref, **tol)


def test_swiglu2_rejects_mismatch(dev):
    import torch

    import zmlx_amd as Z

    with pytest.raises(ValueError):
        Z.swiglu2(torch.zeros(4, device=dev), torch.zeros(5, device=dev))
    with pytest.raises(ValueError):
        Z.swiglu2(torch.zeros(4, device=dev, dtype=torch.float16), torch.zeros(4, device=dev, dtype=torch.float16))


@pytest.mark.parametrize("dtype,shape,K", [
    ("bf16", (4, 2048), 8),      # 16-byte rows
    ("f32", (3, 7), 4),          # ragged rows: element copies
    ("bf16", (2, 3, 100), 2),    # leading batch dims
    ("i32", (5, 64), 1),
    ("u8", (3, 33), 3),
    ("bf16", (0, 64), 4),        # empty batch
])
def test_moe_dispatch(dev, dtype, shape, K):
    import torch

    import zmlx_amd as Z

    rng = np.random.default_rng(14)
    if dtype == "bf16":
        x = to_bf16(bf16_randn(rng, shape), dev)
    elif dtype == "f32":
        x = torch.from_numpy(rng.standard_normal(shape).astype(np.float32)).to(dev)
    elif dtype == "i32":
        x = torch.from_numpy(rng.integers(-2**31, 2**31 - 1, shape, dtype=np.int64).astype(np.int32)).to(dev)
    else:
        x = torch.from_numpy(rng.integers(0, 256, shape, dtype=np.int64).astype(np.uint8)).to(dev)
    idx = torch.zeros((*shape[:-1], K), dtype=torch.int32, device=dev)
    out = Z.moe_dispatch(x, idx)
    torch.cuda.synchronize()
    assert tuple(out.shape) == (*shape[:-1], K, shape[-1])
    xs = x.view(torch.int16) if x.dtype == torch.bfloat16 else x
    os_ = out.view(torch.int16) if out.dtype == torch.bfloat16 else out
    np.testing.assert_array_equal(os_.cpu().numpy(), O.moe_dispatch(xs.cpu().numpy(), K))
