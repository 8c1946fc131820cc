"""zmoe_moe_layer_noalloc (the layer entry point that allocates nothing) vs
zmoe_moe_layer with its workspace, both through the C-ABI: two calls in a
row on the same GPU, the second with a smaller batch, must give the same
outputs bit for bit (the same kernels); a batch beyond the scratch array's
maximum is rejected before any GPU work."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from tests.moe_case import bf16_randn, to_bf16

pytestmark = pytest.mark.gpu


def _noalloc(layer, x, B):
    import torch

    from zmlx_amd import _native as N

    out = torch.empty_like(x)
    idx = torch.empty((B, layer.top_k), dtype=torch.int32, device=x.device)
    w = torch.empty((B, layer.top_k), dtype=torch.float32, device=x.device)
    rc = N.lib().zmoe_moe_layer_noalloc(torch.cuda.current_stream(x.device).cuda_stream, ctypes.byref(layer.desc),
                                        x.data_ptr(), B, out.data_ptr(), idx.data_ptr(), w.data_ptr())
    N.check(rc, "moe_layer_noalloc")
    return out, idx, w


@pytest.mark.parametrize("family,shape,batches", [
    ("qwen3", dict(H=2048, E=32, I=768, K=8), (8, 2)),
    ("qwen3", dict(H=2048, E=32, I=768, K=8), (64, 1)),        # grouped MFMA sequence, then one token
    ("glm", dict(H=2048, E=64, I=1536, K=4, shared_I=1536, mode="mxfp4", gs=32), (5, 3)),
])
def test_noalloc_matches_layer(family, shape, batches):
    import torch

    from tests.test_gpu_layer import _build
    from zmlx_amd.layer import QuantizedMoELayer

    dev = torch.device("cuda:0")
    rng = np.random.default_rng(77)
    shape = dict(shape)
    mode, gs = shape.pop("mode", "affine"), shape.pop("gs", 64)
    banks, wr, sh, tq, tsh, wr_t = _build(dev, rng, mode=mode, gs=gs, **shape)
    kw = {}
    if family == "glm":
        kw = dict(router_bias=torch.zeros(shape["E"], device=dev), routed_scaling_factor=1.8)
    layer = QuantizedMoELayer.for_family(family, wr_t, tq["gate"], tq["up"], tq["down"], top_k=shape["K"],
                                         group_size=gs, mode=mode, shared=tsh, **kw)
    for B in batches:
        print(f"[noalloc] {family} B={B}", flush=True)
        x = to_bf16(bf16_randn(rng, (B, shape["H"])), dev)
        ref, ridx, rw = layer(x, return_routing=True)
        got, gidx, gw = _noalloc(layer, x, B)
        torch.cuda.synchronize()
        assert torch.equal(gidx, ridx)
        assert torch.equal(gw, rw)
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


def test_noalloc_rejects_oversize():
    import torch

    from tests.test_gpu_layer import _build
    from zmlx_amd import _native as N
    from zmlx_amd.layer import QuantizedMoELayer

    dev = torch.device("cuda:0")
    rng = np.random.default_rng(5)
    H, E, I, K = 2048, 16, 768, 8
    banks, wr, sh, tq, tsh, wr_t = _build(dev, rng, H=H, E=E, I=I, K=K)
    layer = QuantizedMoELayer.for_family("qwen3", wr_t, tq["gate"], tq["up"], tq["down"], top_k=K)
    cap = int(N.lib().zmoe_moe_layer_noalloc_max_bytes())
    B = 8192  # y alone is B*K*H*2 = 256 MiB
    assert B * K * H * 2 > cap
    x = torch.zeros((B, H), dtype=torch.bfloat16, device=dev)
    out = torch.empty_like(x)
    rc = N.lib().zmoe_moe_layer_noalloc(torch.cuda.current_stream(dev).cuda_stream, ctypes.byref(layer.desc),
                                        x.data_ptr(), B, out.data_ptr(), None, None)
    with pytest.raises(ValueError, match="maximum"):
        N.check(rc, "moe_layer_noalloc")
