"""GPU parity on the committed fixtures (tests/golden/moe_golden.npz): the HIP
path through the C-ABI against the restatement-generated expected outputs.

* dequantisation: one-hot activations make gather_qmm return bf16(w_hat)
  per element -- compared bit for bit with the fixture's float32 dequant
  rounded to bf16 (affine and mxfp4);
* routers: indices and weights bit-exact;
* combines: fp32_no_fma / no_fma / exact bit-exact, the others within the
  fp32 / bf16 rounding of a reordered sum;
* whole layer (kernel sequence at this small H): experts exact, output within
  the reference tolerance and mostly bit-identical."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden" / "moe_golden.npz"


@pytest.fixture(scope="module")
def g():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _bits_t(b, dev):
    import torch

    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).to(dev).view(torch.bfloat16)


def _t(a, dev):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _bf(t) -> np.ndarray:
    import torch

    return t.float().cpu().numpy() if t.dtype == torch.bfloat16 else t.cpu().numpy()


def test_golden_dequant_one_hot(dev, g):
    import torch

    from zmlx_amd import ops

    K = 256
    x = torch.eye(K, dtype=torch.bfloat16, device=dev).reshape(1, K, K)  # M = K one-hot rows
    w = _t(g["deq_a_w"].view(np.int32), dev)
    out = ops.gather_qmm(x, w, _bits_t(g["deq_a_s"], dev), _bits_t(g["deq_a_b"], dev))
    got = _bf(out).reshape(K, -1).T  # [N, K]
    np.testing.assert_array_equal(O.bf16_to_bits(got), O.bf16_to_bits(g["deq_a_out"]))
    wm = _t(g["deq_m_w"].view(np.int32), dev)
    out = ops.gather_qmm(x, wm, _t(g["deq_m_e"], dev), None, group_size=32, mode="mxfp4")
    got = _bf(out).reshape(K, -1).T
    # by value: e2m1 code 8 is -0.0, and a dot product that is zero is +0.0
    np.testing.assert_array_equal(got, O.bf16_round(g["deq_m_out"]))


def test_golden_routers(dev, g):
    from zmlx_amd import ops

    idx, w = ops.qwen_gating(_bits_t(g["qwen_logits"], dev), 8, True)
    np.testing.assert_array_equal(_bf(idx), g["qwen_idx"])
    np.testing.assert_array_equal(O.bf16_to_bits(_bf(w)), g["qwen_w"])
    w, idx = ops.topk_gating_softmax(_t(g["lfm2_logits"], dev), 4)
    np.testing.assert_array_equal(_bf(idx), g["lfm2_idx"])
    np.testing.assert_allclose(_bf(w), g["lfm2_w"], rtol=2e-6, atol=1e-7)
    w, idx = ops.deepseek_router_topk_sigmoid(_t(g["ds_logits"], dev), _t(g["ds_bias"], dev), k=8, n_group=8,
                                              topk_group=4, routed_scaling_factor=2.5)
    np.testing.assert_array_equal(_bf(idx), g["ds_idx"])
    np.testing.assert_allclose(_bf(w), g["ds_w"], rtol=1e-6, atol=1e-7)


def test_golden_combines(dev, g):
    from zmlx_amd import ops

    y = _bits_t(g["comb_y"], dev)
    wf = _t(g["comb_wf"], dev)
    wb = _bits_t(g["comb_wb"], dev)
    np.testing.assert_array_equal(_bf(ops.moe_combine_fp32_no_fma(y, wf)), g["comb_out_fp32_no_fma"])
    np.testing.assert_allclose(_bf(ops.moe_combine_fp32(y, wf)), g["comb_out_fp32"], rtol=1e-5, atol=1e-6)
    np.testing.assert_array_equal(_bf(ops.moe_combine_no_fma(y, wb)), g["comb_out_no_fma"])
    np.testing.assert_array_equal(_bf(ops.moe_combine_exact(y, wb)), g["comb_out_exact"])
    np.testing.assert_allclose(_bf(ops.moe_combine(y, wb)), g["comb_out_float"], rtol=1e-2, atol=1e-2)
    np.testing.assert_allclose(_bf(ops.moe_combine(y, wb, native=True)), g["comb_out_native"], rtol=1e-2, atol=1e-2)


def test_golden_layer(dev, g):
    import torch

    from zmlx_amd.layer import QuantizedMoELayer, QuantProj

    proj = {n: QuantProj(_t(g[f"layer_{n}_w"], dev), _bits_t(g[f"layer_{n}_s"], dev), _bits_t(g[f"layer_{n}_b"], dev))
            for n in ("gate", "up", "down")}
    layer = QuantizedMoELayer.for_family("qwen3", _bits_t(g["layer_wr"], dev), proj["gate"], proj["up"],
                                         proj["down"], top_k=2)
    out, idx, w = layer(_bits_t(g["layer_x"], dev), return_routing=True)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_bf(idx), g["layer_idx"])
    np.testing.assert_array_equal(O.bf16_to_bits(O.bf16_round(_bf(w))), g["layer_w"])
    ref = O.bf16_from_bits(g["layer_out"])
    got = _bf(out)
    np.testing.assert_allclose(got, ref, atol=1e-2, rtol=1e-2)
    assert (O.bf16_ulp_diff(got, ref) == 0).mean() >= 0.9
